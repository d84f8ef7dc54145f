// y[M, N] = x[M, K] W[N, K]^T for the few-row projections of a decode step
// (M <= 64 rows: the active candidates), bf16 in, fp32 accumulate, bf16 out.
//
// A library GEMM tiles for large M; with 8 rows it pays a full tile
// schedule per call.  Here a workgroup owns 16 output columns (16 rows of
// W) and all M rows: its four wavefronts split K into quarters and stream
// their quarter of the 16 W rows once, each W fragment feeding one MFMA per
// 16-row tile of x (x is tiny and stays in L2).  The MFMA runs transposed,
// y^T = W x^T with v_mfma_f32_16x16x32_bf16 (A = W rows, B = x rows), so
// both operands are plain 16-byte row loads.  The K quarters are summed
// through LDS and the first wavefront writes the tile.
#include "kernels.hpp"

namespace aios {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kGemmBatch = 8;  // k-steps whose loads are issued together

template <int MT>
__global__ __launch_bounds__(kGemmThreads) void skinny_gemm_kernel(
    const bf16* __restrict__ x, int64_t x_stride, const bf16* __restrict__ w, int64_t w_stride,
    bf16* __restrict__ y, int64_t y_stride, int M, int K) {
  __shared__ f32x4 red[3][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int kq = K >> 2;  // multiple of 32
  const int k_begin = wave * kq;
  const int steps = kq >> 5;
  const bf16* wrow = w + (n0 + l16) * w_stride + k_begin + lg * 8;
  const bf16* xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + l16;
    xok[mt] = m < M;
    xrow[mt] = x + (int64_t)(xok[mt] ? m : 0) * x_stride + k_begin + lg * 8;
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < steps; s0 += kGemmBatch) {
    bf16x8 a[kGemmBatch];
    bf16x8 b[kGemmBatch][MT];
#pragma unroll
    for (int u = 0; u < kGemmBatch; ++u) {
      if (s0 + u < steps) {
        a[u] = *reinterpret_cast<const bf16x8*>(wrow + (s0 + u) * 32);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          b[u][mt] = xok[mt] ? *reinterpret_cast<const bf16x8*>(xrow[mt] + (s0 + u) * 32)
                             : bf16x8{};
      }
    }
#pragma unroll
    for (int u = 0; u < kGemmBatch; ++u) {
      if (s0 + u < steps) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16x16x32(a[u], b[u][mt], acc[mt]);
      }
    }
  }

  // acc[mt][i] = y[m = mt*16 + l16][n = n0 + lg*4 + i] (partial over this K quarter)
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave - 1][mt][lane] = acc[mt];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 v = acc[mt] + red[0][mt][lane] + red[1][mt][lane] + red[2][mt][lane];
    if (!xok[mt]) continue;
    uint2 packed;
    packed.x = pack_bf16x2(v[0], v[1]);
    packed.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(y + (int64_t)(mt * 16 + l16) * y_stride + n0 + lg * 4) = packed;
  }
}

}  // namespace

bool skinny_gemm_supported(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && M <= 64 && N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0 &&
         N / 16 <= 0x7fffffff;
}

hipError_t skinny_gemm(const void* x, int64_t x_stride, const void* w, int64_t w_stride, void* y,
                       int64_t y_stride, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const dim3 grid((unsigned)(N / 16));
  const int mt = (int)((M + 15) / 16);
#define AIOS_SKINNY(MT)                                                                         \
  hipLaunchKernelGGL(skinny_gemm_kernel<MT>, grid, dim3(kGemmThreads), 0, stream,               \
                     static_cast<const bf16*>(x), x_stride, static_cast<const bf16*>(w), w_stride, \
                     static_cast<bf16*>(y), y_stride, (int)M, (int)K)
  switch (mt) {
    case 1: AIOS_SKINNY(1); break;
    case 2: AIOS_SKINNY(2); break;
    case 3: AIOS_SKINNY(3); break;
    case 4: AIOS_SKINNY(4); break;
    default: return hipErrorInvalidValue;
  }
#undef AIOS_SKINNY
  return hipGetLastError();
}

}  // namespace aios
