// Paged KV append: scatter flat K/V rows into the token-granular page pool.
//
// Behaviour follows python/aios/kernel/store.py:8-29 (one K row and one V
// row per token written at cache row out_loc[t]); the launch shape is this
// library's own: one lane per 16-byte chunk of a row, so consecutive lanes
// read and write consecutive 16-byte pieces of the same row and every store
// is a global_store_dwordx4.  Narrower accesses are used only when a row,
// stride or base pointer is not 16-byte aligned.
#include "kernels.hpp"

namespace aios {

template <typename V>
__global__ __launch_bounds__(256) void kv_append_kernel(
    char* __restrict__ k_cache, char* __restrict__ v_cache, int64_t num_slots,
    int64_t cache_stride_b, const int32_t* __restrict__ out_loc,
    const char* __restrict__ k, int64_t k_stride_b, const char* __restrict__ v,
    int64_t v_stride_b, int64_t n_tokens, int32_t chunks_per_row) {
  const int64_t total = n_tokens * (int64_t)chunks_per_row;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < total;
       gid += step) {
    const int64_t t = gid / chunks_per_row;
    const int32_t c = (int32_t)(gid - t * chunks_per_row);
    const int64_t slot = (int64_t)out_loc[t];
    if (slot < 0 || slot >= num_slots) continue;
    const V kv = *reinterpret_cast<const V*>(k + t * k_stride_b + (int64_t)c * sizeof(V));
    const V vv = *reinterpret_cast<const V*>(v + t * v_stride_b + (int64_t)c * sizeof(V));
    *reinterpret_cast<V*>(k_cache + slot * cache_stride_b + (int64_t)c * sizeof(V)) = kv;
    *reinterpret_cast<V*>(v_cache + slot * cache_stride_b + (int64_t)c * sizeof(V)) = vv;
  }
}

template <typename V>
static hipError_t launch_kv_append(char* kc, char* vc, int64_t num_slots, int64_t cs,
                                   const int32_t* loc, const char* k, int64_t ks,
                                   const char* v, int64_t vs, int64_t n_tokens,
                                   int64_t row_bytes, hipStream_t stream) {
  const int32_t cpr = (int32_t)(row_bytes / (int64_t)sizeof(V));
  const int64_t total = n_tokens * cpr;
  const int threads = 256;
  int64_t blocks = (total + threads - 1) / threads;
  // A grid-stride loop covers anything beyond 64 blocks per CU.
  const int64_t max_blocks = 256 * 64;
  if (blocks > max_blocks) blocks = max_blocks;
  hipLaunchKernelGGL(kv_append_kernel<V>, dim3((unsigned)blocks), dim3(threads), 0, stream,
                     kc, vc, num_slots, cs, loc, k, ks, v, vs, n_tokens, cpr);
  return hipGetLastError();
}

hipError_t kv_append(void* k_cache, void* v_cache, int64_t num_slots, int64_t cache_stride_b,
                     const int32_t* out_loc, const void* k, int64_t k_stride_b, const void* v,
                     int64_t v_stride_b, int64_t n_tokens, int64_t row_bytes,
                     hipStream_t stream) {
  if (n_tokens == 0) return hipSuccess;
  auto aligned = [&](int64_t a) {
    const uint64_t bits = (uint64_t)a | (uint64_t)row_bytes | (uint64_t)cache_stride_b |
                          (uint64_t)k_stride_b | (uint64_t)v_stride_b |
                          (uint64_t)(uintptr_t)k_cache | (uint64_t)(uintptr_t)v_cache |
                          (uint64_t)(uintptr_t)k | (uint64_t)(uintptr_t)v;
    return (bits & (uint64_t)(a - 1)) == 0;
  };
  char* kc = static_cast<char*>(k_cache);
  char* vc = static_cast<char*>(v_cache);
  const char* kp = static_cast<const char*>(k);
  const char* vp = static_cast<const char*>(v);
  if (aligned(16))
    return launch_kv_append<uint4>(kc, vc, num_slots, cache_stride_b, out_loc, kp, k_stride_b,
                                   vp, v_stride_b, n_tokens, row_bytes, stream);
  if (aligned(8))
    return launch_kv_append<uint2>(kc, vc, num_slots, cache_stride_b, out_loc, kp, k_stride_b,
                                   vp, v_stride_b, n_tokens, row_bytes, stream);
  if (aligned(4))
    return launch_kv_append<uint32_t>(kc, vc, num_slots, cache_stride_b, out_loc, kp,
                                      k_stride_b, vp, v_stride_b, n_tokens, row_bytes, stream);
  if (aligned(2))
    return launch_kv_append<uint16_t>(kc, vc, num_slots, cache_stride_b, out_loc, kp,
                                      k_stride_b, vp, v_stride_b, n_tokens, row_bytes, stream);
  return launch_kv_append<uint8_t>(kc, vc, num_slots, cache_stride_b, out_loc, kp, k_stride_b,
                                   vp, v_stride_b, n_tokens, row_bytes, stream);
}

// Flat page-index gather: indices[cu_k[b] + j] = page_table[row_ids[b], j].
__global__ __launch_bounds__(256) void build_indices_kernel(
    const int32_t* __restrict__ page_table, int64_t pt_stride,
    const int32_t* __restrict__ row_ids, const int32_t* __restrict__ cu_k, int32_t batch,
    int32_t* __restrict__ indices) {
  const int b = blockIdx.y;
  if (b >= batch) return;
  const int32_t begin = cu_k[b];
  const int32_t len = cu_k[b + 1] - begin;
  const int64_t row = (int64_t)row_ids[b] * pt_stride;
  for (int32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < len; j += gridDim.x * blockDim.x)
    indices[begin + j] = page_table[row + j];
}

hipError_t build_indices(const int32_t* page_table, int64_t pt_stride, const int32_t* row_ids,
                         const int32_t* cu_k, int32_t batch, int32_t max_len,
                         int32_t* indices, hipStream_t stream) {
  if (batch == 0 || max_len == 0) return hipSuccess;
  int bx = (max_len + 255) / 256;
  if (bx > 64) bx = 64;
  hipLaunchKernelGGL(build_indices_kernel, dim3(bx, batch), dim3(256), 0, stream, page_table,
                     pt_stride, row_ids, cu_k, batch, indices);
  return hipGetLastError();
}

}  // namespace aios
