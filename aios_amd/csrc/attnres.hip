// Block-AttnRes depth mixer (the "attnres" routing of the 0.214B
// MiniMind-IME trunk): for each token n over the depth sources
// x_0 .. x_{S-1} = bank[0..S) (and the block's running partial, when given)
//   score_s = <x_s, wq> * rsqrt(mean(x_s^2) + eps)      fp32, wq = query * key_norm_w
//   w_s     = bf16(softmax_s(score))                     fp32 softmax, rounded to bf16
//   out     = bf16(sum_s w_s * x_s)                      fp32 sum
// as the two Triton kernels of python/aios/kernel/attnres.py:8-127 compute
// it (the expanded form of python/aios/models/minimind_ime.py:27-74 and the
// materialised reference :125-150).
//
// gfx950 design: the op moves S*N*D bf16 and does ~4 flops per byte, so it
// is a latency-bound gather.  One workgroup per token, one 8-element
// (16-byte) chunk of the hidden vector per thread: every thread issues all
// of its source loads at once (one HBM round trip), keeps them in registers
// (up to kMixKeep sources; more sources are re-read from cache for the
// weighted sum), reduces the 2*S per-source sums with DPP and lane swaps and
// one LDS exchange, and the first wavefront turns them into the S weights
// (one source per lane).  Bank and partial are read once, where the Triton
// pair reads them twice (score kernel, then value kernel).
//
// Fused extras (aios_attnres_mix_ex): the partial may be formed in the same
// launch as bf16(partial + delta) (the `partial + attention_delta` /
// `partial + mlp_delta` adds of minimind_ime.py:233-252) and written to
// partial_out -- which may be the bank's next slot, so a block's last mix
// also stores the new bank entry (minimind_ime.py:305-315).
#include "kernels.hpp"

namespace aios {
namespace {

constexpr int kMixKeep = 16;         // sources per register group
constexpr float kLog2e = 1.44269504088896341f;  // exp(x) = exp2(x * log2(e))
constexpr int kMixMaxSources = 64;   // bank + partial: one wavefront of weights
constexpr int kMixMaxWaves = 16;     // hidden <= 8192: one chunk per thread

__device__ __forceinline__ float mix_wave_sum(float x) { return xrow_sum(row16_sum(x)); }

__device__ __forceinline__ float mix_wave_max(float x) {
  for (int off = 32; off > 0; off >>= 1) x = vmax(x, __shfl_xor(x, off));
  return x;
}

// Eight bf16 as a plain vector type (HIP's uint4 struct, assigned on
// several paths, is kept in scratch memory by the compiler).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void unpack8f(const u32x4& v, float* f) {
  f[0] = lo_bf16(v[0]); f[1] = hi_bf16(v[0]);
  f[2] = lo_bf16(v[1]); f[3] = hi_bf16(v[1]);
  f[4] = lo_bf16(v[2]); f[5] = hi_bf16(v[2]);
  f[6] = lo_bf16(v[3]); f[7] = hi_bf16(v[3]);
}

__device__ __forceinline__ u32x4 pack8f(const float* f) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
               pack_bf16x2(f[6], f[7])};
}

__device__ __forceinline__ float round_to_bf16(float x) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, static_cast<bf16>(x)) << 16);
}

// KEEP: every source fits one register group (sources <= kMixKeep), so the
// weighted sum reuses the loaded values.
template <bool KEEP>
__global__ __launch_bounds__(kMixMaxWaves * 64) void attnres_mix_kernel(AttnResArgs a) {
  __shared__ float red[kMixMaxWaves][2][kMixMaxSources];
  __shared__ float wsh[kMixMaxSources];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int64_t tok = blockIdx.x;
  const bool act = tid * 8 < a.hidden;
  const int S = a.bank_sources;
  const bool has_p = a.partial != nullptr || a.delta != nullptr;
  const int ST = S + (has_p ? 1 : 0);
  const int64_t row_off = tok * a.hidden + tid * 8;
  const int64_t plane = a.num_tokens * (int64_t)a.hidden;

  float q[8];
  {
    const float* qp = a.wq + (act ? tid * 8 : 0);
    const float4 q0 = *reinterpret_cast<const float4*>(qp);
    const float4 q1 = *reinterpret_cast<const float4*>(qp + 4);
    q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w;
    q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
  }

  u32x4 pv = u32x4{0, 0, 0, 0};  // the partial source (below)

  // Source s of the token, as this thread's chunk (zeros past hidden).
  auto load_src = [&](int s) -> u32x4 {
    if (!act || s >= ST) return u32x4{0, 0, 0, 0};
    if (s == S) return pv;
    return *reinterpret_cast<const u32x4*>(a.bank + (int64_t)s * plane + row_off);
  };

  // Per-source sums of this thread's chunk, reduced over the wavefront;
  // lane 0 leaves them for the cross-wavefront sum.
  auto reduce_src = [&](int s, const u32x4& x8) {
    float x[8];
    unpack8f(x8, x);
    float ss = 0.f, dt = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss = fmaf(x[j], x[j], ss);
      dt = fmaf(x[j], q[j], dt);
    }
    ss = mix_wave_sum(ss);
    dt = mix_wave_sum(dt);
    if (lane == 0) {
      red[wave][0][s] = ss;
      red[wave][1][s] = dt;
    }
  };
  // Every load of the token's first group goes out unconditionally (a
  // thread past hidden reads chunk 0, a missing partial or delta reads the
  // bank, a source past the bank repeats its last one) and the results are
  // masked afterwards: loads under conditions compile into branches whose
  // joins wait for them, serialising the round trips.
  const int64_t off = act ? row_off : tok * a.hidden;
  const bf16* pp = a.partial != nullptr ? a.partial : a.bank;
  const bf16* dp = a.delta != nullptr ? a.delta : pp;
  u32x4 v[kMixKeep];
#pragma unroll
  for (int i = 0; i < kMixKeep; ++i)
    v[i] = *reinterpret_cast<const u32x4*>(a.bank + (int64_t)min(i, S - 1) * plane + off);
  const u32x4 pin = *reinterpret_cast<const u32x4*>(pp + off);
  const u32x4 din = *reinterpret_cast<const u32x4*>(dp + off);
  {
    float x[8], y[8];
    unpack8f(pin, x);
    unpack8f(din, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] += y[j];
    pv = (a.partial != nullptr && a.delta != nullptr) ? pack8f(x) : din;
    pv = act ? pv : u32x4{0, 0, 0, 0};
  }
  if (a.delta != nullptr && a.partial_out != nullptr && act)
    *reinterpret_cast<u32x4*>(a.partial_out + row_off) = pv;
#pragma unroll
  for (int i = 0; i < kMixKeep; ++i) {
    v[i] = (has_p && i == S) ? pv : v[i];
    v[i] = (act && i < ST) ? v[i] : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < kMixKeep; ++i) reduce_src(i, v[i]);
  if (!KEEP) {
    for (int g0 = kMixKeep; g0 < ST; g0 += kMixKeep) {
#pragma unroll
      for (int i = 0; i < kMixKeep; ++i) v[i] = load_src(g0 + i);
#pragma unroll
      for (int i = 0; i < kMixKeep; ++i)
        if (g0 + i < ST) reduce_src(g0 + i, v[i]);
    }
  }
  __syncthreads();

  // Scores and weights: wavefront 0, lane s = source s.
  if (wave == 0) {
    float score = kNegInf;
    if (lane < ST) {
      float ss = 0.f, dt = 0.f;
      for (int w = 0; w < nw; ++w) {
        ss += red[w][0][lane];
        dt += red[w][1][lane];
      }
      score = dt * rsqrtf(ss * (1.f / (float)a.hidden) + a.eps);
      if (a.scores != nullptr) a.scores[(int64_t)lane * a.num_tokens + tok] = score;
    }
    const float m = mix_wave_max(score);
    const float e = lane < ST ? __builtin_amdgcn_exp2f((score - m) * kLog2e) : 0.f;
    const float den = mix_wave_sum(e);
    if (lane < ST) wsh[lane] = round_to_bf16(e / den);
  }
  __syncthreads();

  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  auto fold = [&](const u32x4& x8, float w) {
    float x[8];
    unpack8f(x8, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = fmaf(x[j], w, acc[j]);
  };
  if (KEEP) {
#pragma unroll
    for (int i = 0; i < kMixKeep; ++i)
      if (i < ST) fold(v[i], wsh[i]);
  } else {
    for (int g0 = 0; g0 < ST; g0 += kMixKeep) {
#pragma unroll
      for (int i = 0; i < kMixKeep; ++i) v[i] = load_src(g0 + i);
#pragma unroll
      for (int i = 0; i < kMixKeep; ++i)
        if (g0 + i < ST) fold(v[i], wsh[g0 + i]);
    }
  }
  if (act) *reinterpret_cast<u32x4*>(a.out + row_off) = pack8f(acc);
}

// One wavefront per token for hidden = 256 * NC and at most KS sources:
// lane l holds elements [(c * 64 + l) * 4, +4) of each 256-element chunk
// c, so every sum is a wavefront reduction and every lane derives all the
// weights itself -- no LDS exchange and no barrier.  The loads are
// unconditional (a missing partial or delta reads the bank instead, a
// source index past the bank repeats its last source) and every later step
// masks by the source count: a load under a condition is compiled into a
// branch whose join waits for it, which would serialise the round trips.
template <int NC, int KS>
__global__ __launch_bounds__(64) void attnres_mix_wave_kernel(AttnResArgs a) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int lane = threadIdx.x;
  const int64_t tok = blockIdx.x;
  const int S = a.bank_sources;
  const bool has_p = a.partial != nullptr || a.delta != nullptr;
  const bool add = a.partial != nullptr && a.delta != nullptr;
  const int ST = S + (has_p ? 1 : 0);
  const int64_t plane = a.num_tokens * (int64_t)a.hidden;
  const int64_t base = tok * a.hidden + lane * 4;
  const bf16* pp = a.partial != nullptr ? a.partial : a.bank;
  const bf16* dp = a.delta != nullptr ? a.delta : pp;

  u32x2 x[KS][NC], pin[NC], din[NC];
  float q[NC][4];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const bf16* src = a.bank + (int64_t)min(s, S - 1) * plane + base;
#pragma unroll
    for (int c = 0; c < NC; ++c) x[s][c] = *reinterpret_cast<const u32x2*>(src + c * 256);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    pin[c] = *reinterpret_cast<const u32x2*>(pp + base + c * 256);
    din[c] = *reinterpret_cast<const u32x2*>(dp + base + c * 256);
    const float4 v = *reinterpret_cast<const float4*>(a.wq + lane * 4 + c * 256);
    q[c][0] = v.x; q[c][1] = v.y; q[c][2] = v.z; q[c][3] = v.w;
  }

  // The partial source: bf16(partial + delta), the delta alone, or the partial.
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const u32x2 sum = u32x2{pack_bf16x2(lo_bf16(pin[c][0]) + lo_bf16(din[c][0]),
                                        hi_bf16(pin[c][0]) + hi_bf16(din[c][0])),
                            pack_bf16x2(lo_bf16(pin[c][1]) + lo_bf16(din[c][1]),
                                        hi_bf16(pin[c][1]) + hi_bf16(din[c][1]))};
    const u32x2 pv = add ? sum : din[c];
#pragma unroll
    for (int s = 0; s < KS; ++s) x[s][c] = (has_p && s == S) ? pv : x[s][c];
    if (a.delta != nullptr && a.partial_out != nullptr)
      *reinterpret_cast<u32x2*>(a.partial_out + base + c * 256) = pv;
  }

  // Per-source sum of squares and query dot, over the wavefront.
  float ss[KS], dt[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    ss[s] = 0.f;
    dt[s] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float f[4] = {lo_bf16(x[s][c][0]), hi_bf16(x[s][c][0]), lo_bf16(x[s][c][1]),
                          hi_bf16(x[s][c][1])};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ss[s] = fmaf(f[j], f[j], ss[s]);
        dt[s] = fmaf(f[j], q[c][j], dt[s]);
      }
    }
  }
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    ss[s] = mix_wave_sum(ss[s]);
    dt[s] = mix_wave_sum(dt[s]);
  }

  // Scores, softmax over the sources, bf16 weights (every lane alike).
  // (the mean as a product with 1 / hidden and the exponentials as exp2 of
  // a scaled difference: the IEEE divisions and full-accuracy expf were a
  // third of the wavefront's serial VALU work; mixer 3.27 -> 3.04 us)
  float w[KS];
  float m = kNegInf;
  const float inv_h = 1.f / (float)a.hidden;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const float sc = dt[s] * rsqrtf(ss[s] * inv_h + a.eps);
    w[s] = s < ST ? sc : kNegInf;
    m = vmax(m, w[s]);
  }
  if (a.scores != nullptr) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
      if (lane == s && s < ST) a.scores[(int64_t)s * a.num_tokens + tok] = w[s];
  }
  float den = 0.f;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    w[s] = s < ST ? __builtin_amdgcn_exp2f((w[s] - m) * kLog2e) : 0.f;
    den += w[s];
  }
  const float inv = 1.f / den;
#pragma unroll
  for (int s = 0; s < KS; ++s) w[s] = round_to_bf16(w[s] * inv);

#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      acc[0] = fmaf(lo_bf16(x[s][c][0]), w[s], acc[0]);
      acc[1] = fmaf(hi_bf16(x[s][c][0]), w[s], acc[1]);
      acc[2] = fmaf(lo_bf16(x[s][c][1]), w[s], acc[2]);
      acc[3] = fmaf(hi_bf16(x[s][c][1]), w[s], acc[3]);
    }
    *reinterpret_cast<u32x2*>(a.out + base + c * 256) =
        u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
  }
}

template <int NC>
void launch_mix_wave(const AttnResArgs& a, int total, hipStream_t stream) {
  const dim3 grid((unsigned)a.num_tokens), block(64);
  if (total <= 4)
    attnres_mix_wave_kernel<NC, 4><<<grid, block, 0, stream>>>(a);
  else if (total <= 6)
    attnres_mix_wave_kernel<NC, 6><<<grid, block, 0, stream>>>(a);
  else if (total <= 8)
    attnres_mix_wave_kernel<NC, 8><<<grid, block, 0, stream>>>(a);
  else if (total <= 10)
    attnres_mix_wave_kernel<NC, 10><<<grid, block, 0, stream>>>(a);
  else if (total <= 12)
    attnres_mix_wave_kernel<NC, 12><<<grid, block, 0, stream>>>(a);
  else
    attnres_mix_wave_kernel<NC, 16><<<grid, block, 0, stream>>>(a);
}

}  // namespace

bool attnres_supported(int hidden, int total_sources) {
  return hidden > 0 && hidden % 8 == 0 && hidden <= kMixMaxWaves * 64 * 8 && total_sources >= 1 &&
         total_sources <= kMixMaxSources;
}

hipError_t attnres_mix(const AttnResArgs& a, hipStream_t stream) {
  const int total = a.bank_sources + ((a.partial != nullptr || a.delta != nullptr) ? 1 : 0);
  if (total <= kMixKeep && a.hidden % 256 == 0 && a.hidden >= 512 && a.hidden <= 1024) {
    if (a.hidden == 512)
      launch_mix_wave<2>(a, total, stream);
    else if (a.hidden == 768)
      launch_mix_wave<3>(a, total, stream);
    else
      launch_mix_wave<4>(a, total, stream);
    return hipGetLastError();
  }
  const int waves = (a.hidden / 8 + 63) / 64;
  if (total <= kMixKeep)
    attnres_mix_kernel<true><<<dim3((unsigned)a.num_tokens), dim3(waves * 64), 0, stream>>>(a);
  else
    attnres_mix_kernel<false><<<dim3((unsigned)a.num_tokens), dim3(waves * 64), 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace aios
