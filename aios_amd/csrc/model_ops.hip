// Decoder-layer elementwise ops around the attention backend, each one
// launch instead of a chain of framework ops:
//   rmsnorm / residual-add rmsnorm  (layers/norm.py:18-40: flashinfer rmsnorm
//                                    and fused_add_rmsnorm, fp32 math)
//   per-head q/k RMSNorm + RoPE     (models/qwen3.py:60-70 with
//                                    layers/attention.py:11-16: cos/sin cast
//                                    to bf16, products and sum rounded to bf16
//                                    as the bf16 tensor ops round them)
//   SiLU-and-mul                    (layers/activation.py:9-12)
#include "kernels.hpp"

namespace aios {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxVec = 4;  // 8-element vectors per thread: hidden <= 8192

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) t += red[w];
  return t;
}

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x);
  f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
  f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z);
  f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// One workgroup per row.  residual == nullptr: out = rmsnorm(x) * w.
// Otherwise r = x + residual (fp32), residual <- bf16(r), out = rmsnorm(r) * w.
// out may alias x: each thread writes only the elements it read.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const bf16* x, int64_t x_stride, bf16* residual, int64_t r_stride,
    const bf16* __restrict__ w, bf16* out, int64_t out_stride, int hidden, float eps) {
  __shared__ float red[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const bf16* xr = x + row * x_stride;
  bf16* rr = residual ? residual + row * r_stride : nullptr;
  float v[kNormMaxVec][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormMaxVec; ++k) {
    const int i = (k * kNormThreads + threadIdx.x) * 8;
    if (i < hidden) {
      unpack8(*reinterpret_cast<const uint4*>(xr + i), v[k]);
      if (rr) {
        float r[8];
        unpack8(*reinterpret_cast<const uint4*>(rr + i), r);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[k][j] += r[j];
        *reinterpret_cast<uint4*>(rr + i) = pack8(v[k]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(v[k][j], v[k][j], ss);
    }
  }
  const float inv = rsqrtf(block_sum(ss, red) / (float)hidden + eps);
  bf16* orow = out + row * out_stride;
#pragma unroll
  for (int k = 0; k < kNormMaxVec; ++k) {
    const int i = (k * kNormThreads + threadIdx.x) * 8;
    if (i < hidden) {
      float wf[8];
      unpack8(*reinterpret_cast<const uint4*>(w + i), wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[k][j] = v[k][j] * inv * wf[j];
      *reinterpret_cast<uint4*>(orow + i) = pack8(v[k]);
    }
  }
}

// One wavefront per token and four heads (one 16-lane row per head); lane
// l16 of a row holds dims [l16*E, l16*E + E) with E = D/16, so dim i and its
// rotation partner i +- D/2 sit in lanes l16 and l16 ^ 8.
template <int D>
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(
    const bf16* __restrict__ qkv, int64_t stride, int hq, int hkv, const bf16* __restrict__ qw,
    const bf16* __restrict__ kw, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t table_rows, const int32_t* __restrict__ positions,
    bf16* __restrict__ q_out, bf16* __restrict__ k_out, float eps) {
  constexpr int E = D / 16;
  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int head = blockIdx.y * 4 + (lane >> 4);
  const int64_t t = blockIdx.x;
  if (head >= hq + hkv) return;
  const bool is_q = head < hq;
  const int hh = is_q ? head : head - hq;
  const bf16* src = qkv + t * stride + (is_q ? 0 : (int64_t)hq * D) + (int64_t)hh * D + l16 * E;
  const bf16* wp = (is_q ? qw : kw) + l16 * E;
  float x[E], wv[E];
#pragma unroll
  for (int i = 0; i < E; i += 2) {
    const uint32_t a = *reinterpret_cast<const uint32_t*>(src + i);
    const uint32_t b = *reinterpret_cast<const uint32_t*>(wp + i);
    x[i] = lo_bf16(a);
    x[i + 1] = hi_bf16(a);
    wv[i] = lo_bf16(b);
    wv[i + 1] = hi_bf16(b);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) ss = fmaf(x[i], x[i], ss);
  const float inv = rsqrtf(row16_sum(ss) / (float)D + eps);
  float xn[E], pn[E];
#pragma unroll
  for (int i = 0; i < E; ++i) xn[i] = round_bf16(x[i] * inv * wv[i]);
#pragma unroll
  for (int i = 0; i < E; ++i) pn[i] = __shfl_xor(xn[i], 8);
  // Positions outside the table are clamped (never read out of bounds).
  const int64_t pos = min(max((int64_t)positions[t], (int64_t)0), table_rows - 1);
  const float* cr = cos_t + pos * D + l16 * E;
  const float* sr = sin_t + pos * D + l16 * E;
  const bool first_half = l16 < 8;
  float y[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float c = round_bf16(cr[i]);
    const float s = round_bf16(sr[i]);
    const float rot = first_half ? -pn[i] : pn[i];
    y[i] = round_bf16(round_bf16(xn[i] * c) + round_bf16(rot * s));
  }
  bf16* dst = (is_q ? q_out + (t * hq + hh) * D : k_out + (t * hkv + hh) * D) + l16 * E;
#pragma unroll
  for (int i = 0; i < E; i += 2)
    *reinterpret_cast<uint32_t*>(dst + i) = pack_bf16x2(y[i], y[i + 1]);
}

// out[r, i] = bf16(bf16(silu(x[r, i])) * x[r, inter + i]), 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const bf16* __restrict__ x,
                                                       int64_t x_stride, int inter,
                                                       bf16* __restrict__ out,
                                                       int64_t out_stride, int64_t total_vec) {
  const int vec_per_row = inter / 8;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < total_vec;
       v += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = v / vec_per_row;
    const int i = (int)(v - r * vec_per_row) * 8;
    float g[8], u[8];
    unpack8(*reinterpret_cast<const uint4*>(x + r * x_stride + i), g);
    unpack8(*reinterpret_cast<const uint4*>(x + r * x_stride + inter + i), u);
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = round_bf16(g[j] / (1.f + expf(-g[j]))) * u[j];
    *reinterpret_cast<uint4*>(out + r * out_stride + i) = pack8(g);
  }
}

}  // namespace

hipError_t rmsnorm(const void* x, int64_t x_stride, void* residual, int64_t r_stride,
                   const void* w, void* out, int64_t out_stride, int64_t rows, int hidden,
                   float eps, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, stream,
                     static_cast<const bf16*>(x), x_stride, static_cast<bf16*>(residual), r_stride,
                     static_cast<const bf16*>(w), static_cast<bf16*>(out), out_stride, hidden, eps);
  return hipGetLastError();
}

bool rmsnorm_supported(int hidden) {
  return hidden > 0 && hidden % 8 == 0 && hidden <= kNormThreads * 8 * kNormMaxVec;
}

hipError_t qk_norm_rope(const void* qkv, int64_t stride, int64_t tokens, int hq, int hkv, int D,
                        const void* qw, const void* kw, const float* cos_t, const float* sin_t,
                        int64_t table_rows, const int32_t* positions, void* q_out, void* k_out,
                        float eps, hipStream_t stream) {
  if (tokens == 0) return hipSuccess;
  const dim3 grid((unsigned)tokens, (unsigned)((hq + hkv + 3) / 4));
#define AIOS_QKR(DD)                                                                          \
  hipLaunchKernelGGL(qk_norm_rope_kernel<DD>, grid, dim3(64), 0, stream,                      \
                     static_cast<const bf16*>(qkv), stride, hq, hkv,                         \
                     static_cast<const bf16*>(qw), static_cast<const bf16*>(kw), cos_t, sin_t, \
                     table_rows, positions, static_cast<bf16*>(q_out), static_cast<bf16*>(k_out), eps)
  switch (D) {
    case 64: AIOS_QKR(64); break;
    case 96: AIOS_QKR(96); break;
    case 128: AIOS_QKR(128); break;
    default: return hipErrorInvalidValue;
  }
#undef AIOS_QKR
  return hipGetLastError();
}

hipError_t silu_mul(const void* x, int64_t x_stride, int64_t rows, int inter, void* out,
                    int64_t out_stride, hipStream_t stream) {
  const int64_t total = rows * (inter / 8);
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const bf16*>(x), x_stride, inter, static_cast<bf16*>(out),
                     out_stride, total);
  return hipGetLastError();
}

}  // namespace aios
