// Varlen causal paged prefill (kernel (b)), also used for cross-keystroke
// LCP extension (a few new tokens against a cached prefix).
//
// One workgroup owns (request r, kv-head h, query tile): q_tile consecutive
// query tokens times the G query heads of h, packed into the 128 MFMA rows
// (row = token * G + head), and streams KV positions [0, cached_len +
// last token of the tile] of r through the tile engine with the offset
// causal mask key_pos <= cached_len + i (python/aios/attention/
// flashinfer.py:67-80).  Tiles entirely below the diagonal are unmasked; the
// mask only bites in the last sub-tiles.
#include "engine.hpp"

namespace aios {

template <int D>
__global__ __launch_bounds__(kEngineThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(PrefillArgs a) {
  __shared__ __align__(16) uint8_t lds[KVTile<D>::LDS_BYTES];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int G = a.group;
  // One flat grid: consecutive workgroups take consecutive kv-heads (the
  // hardware deals workgroups round-robin to the XCDs, so with 8 kv-heads
  // each XCD's L2 holds one head's K/V, read by all of that head's query
  // tiles), and the query tiles run from the last (the longest causal KV
  // range) to the first, so the short tiles fill in behind the long ones
  // instead of the long ones forming the tail.
  const int flat = blockIdx.x;
  const int h = flat % a.num_kv_heads;
  const int rest = flat / a.num_kv_heads;
  const int r = rest % a.batch;
  const int qt = a.q_tiles - 1 - rest / a.batch;
  const int q_start = a.cu_q[r];
  const int q_len = a.cu_q[r + 1] - q_start;
  if (qt * a.q_tile >= q_len) return;
  const int kv_base = a.cu_k[r];
  const int kv_len = a.cu_k[r + 1] - kv_base;
  const int cached = kv_len - q_len;
  const int q_hi = min(q_len, (qt + 1) * a.q_tile);

  TileEngine32<D, true> eng;
  // The lane's query row (lanes l and l ^ 32 share it).
  const int m = wave * 32 + (lane & 31);
  const int i = qt * a.q_tile + m / G;
  const int g = m - (m / G) * G;
  const bool ok = (m < a.q_tile * G) && (i < q_len);
  const bf16* qr = a.q + (int64_t)(q_start + i) * a.q_tok_stride + (int64_t)(h * G + g) * D;
  const int64_t out_off = ((int64_t)(q_start + i) * a.num_qo_heads + (h * G + g)) * D;
  eng.limit = cached + i;
  eng.min_limit = cached + qt * a.q_tile;
  // A wavefront whose 32 rows are all past the tile's tokens only helps
  // stream K/V; it skips the math.
  const int m0 = wave * 32;
  const bool active = m0 < a.q_tile * G && qt * a.q_tile + m0 / G < q_len;
  eng.run(lds, reinterpret_cast<const uint8_t*>(a.k_cache) + (int64_t)h * D * 2,
          reinterpret_cast<const uint8_t*>(a.v_cache) + (int64_t)h * D * 2, a.kv_tok_stride * 2,
          a.num_pages, a.indices + kv_base, 0, min(kv_len, cached + q_hi), a.scale_log2,
          [&] { eng.load_q(qr, ok); }, active);

  if (!ok) return;
  const float l_tot = eng.l_run;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  bf16* po = a.out + out_off + 4 * (lane >> 5);
  // o[nt] register 4j + i: dim 32 nt + 8j + 4h + i of the lane's row
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 packed;
      packed.x = pack_bf16x2(eng.o[nt][4 * j] * inv, eng.o[nt][4 * j + 1] * inv);
      packed.y = pack_bf16x2(eng.o[nt][4 * j + 2] * inv, eng.o[nt][4 * j + 3] * inv);
      *reinterpret_cast<uint2*>(po + nt * 32 + 8 * j) = packed;
    }
}

hipError_t launch_prefill(int D, int NW, const PrefillArgs& a, int q_tiles, int batch,
                          hipStream_t s) {
  (void)NW;
  const dim3 grid(q_tiles * a.num_kv_heads * batch);
  if (q_tiles == 0 || batch == 0) return hipSuccess;
  switch (D) {
    case 64: hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(kEngineThreads), 0, s, a); break;
    case 96: hipLaunchKernelGGL(prefill_kernel<96>, grid, dim3(kEngineThreads), 0, s, a); break;
    case 128: hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kEngineThreads), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace aios
