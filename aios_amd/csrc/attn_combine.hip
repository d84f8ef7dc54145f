// Log-sum-exp combine of a decode batch's partial softmax states: one
// workgroup per (row, kv-head) merges that row's parts (the prefix chunks'
// and the suffix items', layout in kernels.hpp) with m = max lse_j,
// w_j = 2^(lse_j - m) / sum_i 2^(lse_i - m), out = sum w_j o_j (the
// split/merge rule of online softmax,
// resources/lesson-41-flashattention-online-softmax/run_lesson41.py:7-18).
// Its own translation unit so that it can be scheduled on its own terms (see
// build.py).
#include "engine.hpp"

namespace aios {

constexpr int kCombineThreads = 256;
constexpr int kCombineMaxParts = 64;  // one part per lane of a wavefront
constexpr int kCombineBatch = 32;     // parts whose o loads one thread keeps in flight

// Max / sum over the 64 lanes of a wavefront (DPP inside 16-lane rows, then
// the lane swaps across rows); every lane receives the result.
__device__ __forceinline__ float wave_max(float x) {
  int v;
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false);
  x = vmax(x, __int_as_float(v));
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false);
  x = vmax(x, __int_as_float(v));
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false);
  x = vmax(x, __int_as_float(v));
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false);
  x = vmax(x, __int_as_float(v));
  return xrow_max(x);
}
__device__ __forceinline__ float wave_sum(float x) { return xrow_sum(row16_sum(x)); }

template <int D, int G>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(
    const float* __restrict__ lse, const bf16* __restrict__ po_base, int32_t n_parts, int32_t rows,
    int32_t num_kv_heads, DecodeArgs args) {
  // (the leading scalars are preloaded: see decode_main_kernel)
  DecodeArgs a = args;
  a.parts.lse = const_cast<float*>(lse);
  a.parts.o = const_cast<bf16*>(po_base);
  a.parts.n_parts = n_parts;
  a.parts.rows = rows;
  a.num_kv_heads = num_kv_heads;
  constexpr int E8 = G * D / 8;  // 8-dim (16-byte) elements per part
  static_assert(E8 <= kCombineThreads, "one element per thread per part");
  constexpr int R = kCombineThreads / E8;  // threads sharing one element (parts split)
  constexpr int NW = kCombineThreads / 64;
  constexpr int PB = (kCombineMaxParts + R - 1) / R;  // parts per thread, upper bound
  constexpr int BATCH = PB < kCombineBatch ? PB : kCombineBatch;
  // Weight of part j for query row g at w_s[g][j]; the row pitch of
  // kCombineMaxParts + 1 words keeps both the writes (a wavefront's 64 parts
  // of one row) and the reads (the G rows of one part) free of bank conflicts.
  constexpr int WP = kCombineMaxParts + 1;
  __shared__ float w_s[G * WP];
  __shared__ f32x4 red[2][kCombineThreads];  // [half][thread]: 16-byte stride, no conflicts

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int bh = blockIdx.x;
  const int b = bh / a.num_kv_heads;
  const int h = bh - b * a.num_kv_heads;
  const int np = a.parts.n_parts;
  const int e = tid % E8;
  const int r = tid / E8;
  const bool active = r < R;  // G * D / 8 need not divide the workgroup
  // Element e = 8 dims of one row: dims dt*16 + q8*8 .. +7 of head g, so
  // consecutive threads read the G adjacent rows of one 16-dim tile
  // (G * 32 contiguous bytes of a part).
  const int q8 = e & 1;
  const int g = (e >> 1) % G;
  const int dt = e / (2 * G);
  const int d = dt * 16 + q8 * 8;
  const int row = b * G + g;
  const int64_t part_stride = (int64_t)(D / 16) * a.parts.rows * 16;  // elements per part
  const uint4* po = reinterpret_cast<const uint4*>(a.parts.o + a.parts.o_index(D, h, 0, row, d));

  // The lse loads go out first, so the weights below wait only for them;
  // then this thread's o loads (parts r, r + R, ...).
  constexpr int LG = (G + NW - 1) / NW;  // query rows per wavefront
  float l[LG];
#pragma unroll
  for (int i = 0; i < LG; ++i) {
    const int gg = i * NW + wave;
    l[i] = gg < G && lane < np ? a.parts.lse[a.parts.lse_index(h, lane, b * G + gg)] : kNegInf;
  }
  uint4 v[BATCH];
#pragma unroll
  for (int k = 0; k < BATCH; ++k) {
    const int j = r + k * R;
    v[k] = active && j < np ? po[(int64_t)j * part_stride / 8] : make_uint4(0, 0, 0, 0);
  }
  // Normalised weights w_j = 2^(lse_j - m) / sum_i 2^(lse_i - m),
  // m = max_j lse_j: one wavefront per query row, lane j = part j (zero for
  // lanes past the last part).
#pragma unroll
  for (int i = 0; i < LG; ++i) {
    const int gg = i * NW + wave;
    if (gg < G) {  // uniform per wavefront
      const float mx = wave_max(l[i]);
      const float mu = (mx == kNegInf) ? 0.f : mx;
      const float w = lane < np ? fast_exp2(l[i] - mu) : 0.f;
      const float den = wave_sum(w);
      w_s[gg * WP + lane] = den > 0.f ? w / den : 0.f;
    }
  }
  __syncthreads();

  f32x4 acc0 = f32x4{0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  auto fold = [&](int j, const uint4& x) {
    const float w = w_s[g * WP + j];
    acc0 += f32x4{lo_bf16(x.x), hi_bf16(x.x), lo_bf16(x.y), hi_bf16(x.y)} * w;
    acc1 += f32x4{lo_bf16(x.z), hi_bf16(x.z), lo_bf16(x.w), hi_bf16(x.w)} * w;
  };
  // Parts past the last one hold zeros and weight zero (j < kCombineMaxParts
  // keeps every w_s read in bounds); the unrolled fold stops at the thread's
  // last part (the long-context rows have 36 parts: 9 of a thread's 16).
#pragma unroll
  for (int k = 0; k < BATCH; ++k) {
    if (r + k * R >= np) break;
    fold(min(r + k * R, kCombineMaxParts - 1), v[k]);
  }
  for (int j0 = r + BATCH * R; active && j0 < np; j0 += BATCH * R) {
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int j = j0 + k * R;
      v[k] = j < np ? po[(int64_t)j * part_stride / 8] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) fold(min(j0 + k * R, kCombineMaxParts - 1), v[k]);
  }
  if (R > 1) {
    red[0][tid] = acc0;
    red[1][tid] = acc1;
    __syncthreads();
    if (r == 0)
      for (int rr = 1; rr < R; ++rr) {
        acc0 += red[0][rr * E8 + e];
        acc1 += red[1][rr * E8 + e];
      }
  }
  if (active && r == 0) {
    const uint4 packed = make_uint4(pack_bf16x2(acc0[0], acc0[1]), pack_bf16x2(acc0[2], acc0[3]),
                                    pack_bf16x2(acc1[0], acc1[1]), pack_bf16x2(acc1[2], acc1[3]));
    *reinterpret_cast<uint4*>(a.out + ((int64_t)b * a.num_qo_heads + h * G + g) * D + d) = packed;
  }
}

template <int D>
static hipError_t launch_combine_d(const DecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.batch * a.num_kv_heads);
  if (grid.x == 0) return hipSuccess;
  const float* lse = a.parts.lse;
  const bf16* po = a.parts.o;
  const int32_t np = a.parts.n_parts, rows = a.parts.rows, hkv = a.num_kv_heads;
#define AIOS_COMBINE(GG)                                                                      \
  hipLaunchKernelGGL((decode_combine_kernel<D, GG>), grid, dim3(kCombineThreads), 0, s, lse, po, \
                     np, rows, hkv, a)
  switch (a.group) {
    case 1: AIOS_COMBINE(1); break;
    case 2: AIOS_COMBINE(2); break;
    case 3: AIOS_COMBINE(3); break;
    case 4: AIOS_COMBINE(4); break;
    case 6: AIOS_COMBINE(6); break;
    case 8: AIOS_COMBINE(8); break;
    default: return hipErrorInvalidValue;
  }
#undef AIOS_COMBINE
  return hipGetLastError();
}

hipError_t launch_decode_combine(int D, const DecodeArgs& a, hipStream_t s) {
  switch (D) {
    case 64: return launch_combine_d<64>(a, s);
    case 96: return launch_combine_d<96>(a, s);
    case 128: return launch_combine_d<128>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aios
