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
//
// The ops around a projection can be folded into it, so they need no
// launch of their own:
//   prologue kAddNorm: x = bf16(RMSNorm(h + residual) * w) (the residual-add
//     RMSNorm of layers/norm.py:34-40; residual may be absent), every
//     workgroup recomputing the row norms of its few rows, and workgroup 0
//     writing bf16(h + residual) to residual_out;
//   epilogue kSiluPair: W holds gate rows then up rows (the merged gate/up
//     projection); a workgroup computes gate columns n0..n0+15 and the
//     matching up columns and writes bf16(bf16(silu(g)) * u), the
//     silu_and_mul of layers/activation.py:9-12, with g and u rounded to
//     bf16 first as the separate projection would store them.
#include "kernels.hpp"

namespace aios {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kGemmBatch = 8;     // k-steps whose loads are issued together
constexpr int kNormMaxFrags = 8;  // kAddNorm holds steps * MT <= this many x fragments

enum Prologue { kPlain = 0, kAddNorm = 1 };
enum Epilogue { kStore = 0, kSiluPair = 1 };

__device__ __forceinline__ void unpack8(const bf16x8& v, float* f) {
  const uint4 u = __builtin_bit_cast(uint4, v);
  f[0] = lo_bf16(u.x); f[1] = hi_bf16(u.x);
  f[2] = lo_bf16(u.y); f[3] = hi_bf16(u.y);
  f[4] = lo_bf16(u.z); f[5] = hi_bf16(u.z);
  f[6] = lo_bf16(u.w); f[7] = hi_bf16(u.w);
}

__device__ __forceinline__ bf16x8 pack8(const float* f) {
  return __builtin_bit_cast(
      bf16x8, make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                         pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])));
}

// The operands every workgroup needs before its first load lead the kernel
// arguments as scalars: compiled with kernel-argument preloading they arrive
// in SGPRs at wave start, instead of behind a load of the kernel-argument
// segment (LinearArgs, by value, cannot be preloaded).  The kernels then
// override the copies inside LinearArgs with them.
#define AIOS_LINEAR_HOT_PARAMS                                                              \
  const bf16 *__restrict__ hx_, const bf16 *__restrict__ hw_, const bf16 *hn_, const bf16 *hr_, \
      int32_t hxs_, int32_t hws_, int32_t hm_, int32_t hk_, int32_t hn32_, LinearArgs args_
#define AIOS_LINEAR_HOT_ARGS(a)                                                             \
  (a).x, (a).w, (a).norm_w, (a).residual, (int32_t)(a).x_stride, (int32_t)(a).w_stride, (a).M, \
      (a).K, (int32_t)(a).N, (a)
#define AIOS_LINEAR_HOT_BIND \
  LinearArgs a = args_;      \
  a.x = hx_;                 \
  a.w = hw_;                 \
  a.norm_w = hn_;            \
  a.residual = hr_;          \
  a.x_stride = hxs_;         \
  a.w_stride = hws_;         \
  a.M = hm_;                 \
  a.K = hk_;                 \
  a.N = hn32_;

// KS > 0: the K steps of a wavefront (K / 128) fixed at compile time, so
// the operand loads are one straight-line burst; KS = 0: read from K.
// NC = 8 / 4: a workgroup owns 8 / 4 output columns (the MFMA tile's other W
// rows are not loaded and read as zero), 2x / 4x the workgroups at 1/2 / 1/4
// of the weight bytes each, for projections with few column tiles.
template <int MT, int PRO, int EPI, int KS = 0, int NC = 16>
__global__ __launch_bounds__(kGemmThreads) void skinny_gemm_kernel(AIOS_LINEAR_HOT_PARAMS) {
  AIOS_LINEAR_HOT_BIND
  static_assert(NC == 16 || ((NC == 8 || NC == 4) && MT == 1), "narrow tiles: one row tile");
  constexpr int NP = EPI == kSiluPair ? 2 : 1;  // W row sets per workgroup
  __shared__ f32x4 red[3][NP][MT][64];
  __shared__ float ssq[4][MT][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * NC;
  const int kq = a.K >> 2;  // multiple of 32
  const int k_begin = wave * kq + lg * 8;
  const int steps = KS > 0 ? KS : kq >> 5;
  const bool wok = NC == 16 || l16 < NC;  // this lane's W row is one of the tile's
  const bf16* wrow[NP];
  wrow[0] = a.w + (n0 + (wok ? l16 : 0)) * a.w_stride + k_begin;
  if constexpr (NP == 2) wrow[NP - 1] = a.w + (a.N + n0 + (wok ? l16 : 0)) * a.w_stride + k_begin;
  int64_t xoff[MT], roff[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + l16;
    xok[mt] = m < a.M;
    xoff[mt] = (int64_t)(xok[mt] ? m : 0) * a.x_stride + k_begin;
    roff[mt] = (int64_t)(xok[mt] ? m : 0) * a.r_stride + k_begin;
  }
  f32x4 acc[NP][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[p][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (PRO == kAddNorm) {
    // The wave's whole K quarter of its rows, r = h (+ residual) in fp32
    // terms (kept as the bf16 operands; their fp32 sum is exact).
    constexpr int SMAX = kNormMaxFrags / MT;
    bf16x8 hf[SMAX][MT], rf[SMAX][MT];
    bf16x8 nw[SMAX];  // the norm weight of the quarter, loaded with the rest
    bf16x8 wa[NP][kGemmBatch];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int u = 0; u < kGemmBatch; ++u)
        if (u < steps) wa[p][u] = wok ? *reinterpret_cast<const bf16x8*>(wrow[p] + u * 32) : bf16x8{};
    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) ss[mt] = 0.f;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      if (s < steps) {
        nw[s] = *reinterpret_cast<const bf16x8*>(a.norm_w + k_begin + s * 32);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          hf[s][mt] = xok[mt] ? *reinterpret_cast<const bf16x8*>(a.x + xoff[mt] + s * 32)
                              : bf16x8{};
          rf[s][mt] = (xok[mt] && a.residual)
                          ? *reinterpret_cast<const bf16x8*>(a.residual + roff[mt] + s * 32)
                          : bf16x8{};
        }
      }
    }
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      if (s < steps) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float h8[8], r8[8];
          unpack8(hf[s][mt], h8);
          unpack8(rf[s][mt], r8);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float r = h8[j] + r8[j];
            ss[mt] = fmaf(r, r, ss[mt]);
          }
          if (a.residual_out && blockIdx.x == 0 && xok[mt]) {
            float s8[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) s8[j] = h8[j] + r8[j];
            *reinterpret_cast<bf16x8*>(a.residual_out +
                                       (int64_t)(mt * 16 + l16) * a.ro_stride + k_begin + s * 32) =
                pack8(s8);
          }
        }
      }
    }
    // Row sums over the four lane groups, then over the four wavefronts.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ss[mt] = xrow_sum(ss[mt]);
      if (lg == 0) ssq[wave][mt][l16] = ss[mt];
    }
    __syncthreads();
    float inv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      inv[mt] = rsqrtf((ssq[0][mt][l16] + ssq[1][mt][l16] + ssq[2][mt][l16] +
                        ssq[3][mt][l16]) / (float)a.K + a.eps);
#pragma unroll
    for (int s0 = 0; s0 < SMAX; s0 += kGemmBatch) {
      if (s0 >= steps) break;
      if (s0 > 0) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int u = 0; u < kGemmBatch; ++u)
            if (s0 + u < steps)
              wa[p][u] = wok ? *reinterpret_cast<const bf16x8*>(wrow[p] + (s0 + u) * 32) : bf16x8{};
      }
#pragma unroll
      for (int u = 0; u < kGemmBatch; ++u) {
        const int s = s0 + u;
        if (s < steps && s < SMAX) {
          float w8[8];
          unpack8(nw[s], w8);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            float h8[8], r8[8], x8[8];
            unpack8(hf[s][mt], h8);
            unpack8(rf[s][mt], r8);
#pragma unroll
            for (int j = 0; j < 8; ++j) x8[j] = (h8[j] + r8[j]) * inv[mt] * w8[j];
            const bf16x8 xb = xok[mt] ? pack8(x8) : bf16x8{};
#pragma unroll
            for (int p = 0; p < NP; ++p) acc[p][mt] = mfma16x16x32(wa[p][u], xb, acc[p][mt]);
          }
        }
      }
    }
  } else {
    // One row tile and one W row set: all of a 512-wide K quarter in one
    // round trip (the down projection's K = 2048).
    constexpr int B = (MT == 1 && NP == 1) ? 2 * kGemmBatch : kGemmBatch;
    for (int s0 = 0; s0 < steps; s0 += B) {
      bf16x8 wa[NP][B];
      bf16x8 b[B][MT];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        if (s0 + u < steps) {
#pragma unroll
          for (int p = 0; p < NP; ++p)
            wa[p][u] = wok ? *reinterpret_cast<const bf16x8*>(wrow[p] + (s0 + u) * 32) : bf16x8{};
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            b[u][mt] = xok[mt] ? *reinterpret_cast<const bf16x8*>(a.x + xoff[mt] + (s0 + u) * 32)
                               : bf16x8{};
        }
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        if (s0 + u < steps) {
#pragma unroll
          for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[p][mt] = mfma16x16x32(wa[p][u], b[u][mt], acc[p][mt]);
        }
      }
    }
  }

  // acc[p][mt][i] = y_p[m = mt*16 + l16][n = n0 + lg*4 + i] (partial over this K quarter)
  if (wave > 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[wave - 1][p][mt][lane] = acc[p][mt];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 v[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
      v[p] = acc[p][mt] + red[0][p][mt][lane] + red[1][p][mt][lane] + red[2][p][mt][lane];
    if (!xok[mt]) continue;
    f32x4 o = v[0];
    if constexpr (EPI == kSiluPair) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = round_bf16(v[0][i]);
        const float u = round_bf16(v[NP - 1][i]);
        o[i] = round_bf16(g / (1.f + expf(-g))) * u;
      }
    }
    if (lg * 4 >= NC) continue;  // columns NC..15 of the MFMA tile: not this tile's
    uint2 packed;
    packed.x = pack_bf16x2(o[0], o[1]);
    packed.y = pack_bf16x2(o[2], o[3]);
    *reinterpret_cast<uint2*>(a.y + (int64_t)(mt * 16 + l16) * a.y_stride + n0 + lg * 4) = packed;
  }
}

// Projections with many 16-column tiles and up to 16 rows (the LM head: 9,496
// tiles at a 151,936-id vocabulary), K = 128 * KS: a grid of a few
// workgroups per compute unit, each walking tiles blockIdx.x, + gridDim.x,
// ...  Its rows (normalised once with kAddNorm) stay in registers, and the W
// fragments of the next tile are loaded while the current tile is
// multiplied and reduced, so a workgroup pays the weight-load latency once
// instead of once per tile (and the row norm once instead of per tile).
// The loop issues loads only: the next tile's loads are unconditional (the
// index clamped to the last tile) and the tiles' outputs are staged in LDS
// and stored after the loop, so the compiler's load-counter waits let the
// next tile's loads stay in flight.
constexpr int kStreamWgsPerCu = 2;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer descriptor word 3 (32-bit data format)
constexpr int kStreamMaxIters = 32;  // tiles one workgroup stages in LDS

template <int PRO, int KS>
__global__ __launch_bounds__(kGemmThreads) void skinny_gemm_stream_kernel(AIOS_LINEAR_HOT_PARAMS) {
  AIOS_LINEAR_HOT_BIND
  __shared__ f32x4 red[2][4][64];  // per tile parity: the four wavefronts' partials
  __shared__ float ssq[4][16];
  __shared__ uint2 out_s[kStreamMaxIters][64];  // a tile: 16 rows x 4 groups of 4 columns
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int k_begin = wave * (KS * 32) + lg * 8;  // K / 4 = KS * 32
  const bool xok = l16 < a.M;
  const int64_t m = xok ? l16 : 0;
  const int64_t tiles = a.N / 16;
  const int64_t G = gridDim.x;
  // W through a raw buffer: the lane's offset is loop-invariant and a tile
  // moves only the scalar offset, so the loop needs no vector registers for
  // addresses (W below 2 GiB, checked by the launcher).
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, 0x7fffffff, kRsrcWord3);
  const int32_t lane_off = (int32_t)((l16 * a.w_stride + k_begin) * 2);
  const int64_t tile_bytes = 16 * a.w_stride * 2;
  auto load_w = [&](bf16x8 (&w)[KS], int64_t tile) {
    const int32_t soff = (int32_t)(min(tile, tiles - 1) * tile_bytes);
#pragma unroll
    for (int u = 0; u < KS; ++u)
      w[u] = __builtin_bit_cast(bf16x8,
                                __builtin_amdgcn_raw_buffer_load_b128(wrs, lane_off + u * 64, soff, 0));
  };
  int64_t t = blockIdx.x;  // < tiles: the grid is at most the tile count
  bf16x8 wa[KS], wb[KS];
  load_w(wa, t);

  bf16x8 xb[KS];
  if constexpr (PRO == kAddNorm) {
    bf16x8 hf[KS], rf[KS], nw[KS];
#pragma unroll
    for (int u = 0; u < KS; ++u) {
      nw[u] = *reinterpret_cast<const bf16x8*>(a.norm_w + k_begin + u * 32);
      hf[u] = xok ? *reinterpret_cast<const bf16x8*>(a.x + m * a.x_stride + k_begin + u * 32)
                  : bf16x8{};
      rf[u] = (xok && a.residual)
                  ? *reinterpret_cast<const bf16x8*>(a.residual + m * a.r_stride + k_begin + u * 32)
                  : bf16x8{};
    }
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < KS; ++u) {
      float h8[8], r8[8];
      unpack8(hf[u], h8);
      unpack8(rf[u], r8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float r = h8[j] + r8[j];
        ss = fmaf(r, r, ss);
      }
      if (a.residual_out && blockIdx.x == 0 && xok) {
        float s8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) s8[j] = h8[j] + r8[j];
        *reinterpret_cast<bf16x8*>(a.residual_out + m * a.ro_stride + k_begin + u * 32) =
            pack8(s8);
      }
    }
    ss = xrow_sum(ss);
    if (lg == 0) ssq[wave][l16] = ss;
    __syncthreads();
    const float inv =
        rsqrtf((ssq[0][l16] + ssq[1][l16] + ssq[2][l16] + ssq[3][l16]) / (float)a.K + a.eps);
#pragma unroll
    for (int u = 0; u < KS; ++u) {
      float w8[8], h8[8], r8[8], x8[8];
      unpack8(nw[u], w8);
      unpack8(hf[u], h8);
      unpack8(rf[u], r8);
#pragma unroll
      for (int j = 0; j < 8; ++j) x8[j] = (h8[j] + r8[j]) * inv * w8[j];
      xb[u] = xok ? pack8(x8) : bf16x8{};
    }
  } else {
#pragma unroll
    for (int u = 0; u < KS; ++u)
      xb[u] = xok ? *reinterpret_cast<const bf16x8*>(a.x + m * a.x_stride + k_begin + u * 32)
                  : bf16x8{};
  }

  // One tile: this wavefront's K-quarter product, the four partials summed
  // through LDS by lanes lg == wave of every wavefront (row l16, columns
  // 4 * wave ..), the result staged in out_s[it].
  auto tile = [&](const bf16x8 (&w)[KS], int it, int par) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < KS; ++u) acc = mfma16x16x32(w[u], xb[u], acc);
    red[par][wave][lane] = acc;
    __syncthreads();
    const int src = l16 + 16 * wave;
    const f32x4 o = red[par][0][src] + red[par][1][src] + red[par][2][src] + red[par][3][src];
    if (lg == wave) out_s[it][l16 * 4 + wave] = make_uint2(pack_bf16x2(o[0], o[1]),
                                                           pack_bf16x2(o[2], o[3]));
  };
  // Every load so far (the first tile's, then the rows') has landed before
  // the loop: with loads of unknown count pending where the loop header
  // merges, the compiler would wait for all of them (vmcnt(0)) at the top of
  // every iteration, before the next tile's loads go out.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  int it = 0;
  while (true) {
    load_w(wb, t + G);
    tile(wa, it++, 0);
    t += G;
    if (t >= tiles) break;
    load_w(wa, t + G);
    tile(wb, it++, 1);
    t += G;
    if (t >= tiles) break;
  }
  __syncthreads();
  // Tile i's rows: y[r][(blockIdx.x + i * G) * 16 + 4 * g ..] = out_s[i][r * 4 + g].
  for (int c = threadIdx.x; c < it * 64; c += kGemmThreads) {
    const int i = c >> 6;
    const int r = (c >> 2) & 15;
    const int g = c & 3;
    if (r < a.M)
      *reinterpret_cast<uint2*>(a.y + (int64_t)r * a.y_stride +
                                ((int64_t)blockIdx.x + (int64_t)i * G) * 16 + 4 * g) = out_s[i][c & 63];
  }
}

// Plain projections with K = 768 and up to 16 rows (the o projection and
// LM head of hidden-768 models): one wavefront per 16 output columns over the
// whole K, every load in one round trip, two interleaved MFMA chains, no LDS
// reduction or barrier.
constexpr int kColsSteps = 24;  // K = 768

// NC columns per wavefront (16, or 8 / 4 with the MFMA tile's other W rows
// read as zero, for projections with few column tiles).
template <int NC>
__global__ __launch_bounds__(64) void skinny_gemm_cols_kernel(AIOS_LINEAR_HOT_PARAMS) {
  AIOS_LINEAR_HOT_BIND
  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * NC;
  const bool wok = l16 < NC;
  const bf16* wr = a.w + (n0 + (wok ? l16 : 0)) * a.w_stride + lg * 8;
  const bool ok = l16 < a.M;
  const bf16* xr = a.x + (int64_t)(ok ? l16 : 0) * a.x_stride + lg * 8;
  bf16x8 w[kColsSteps], x[kColsSteps];
#pragma unroll
  for (int s = 0; s < kColsSteps; ++s) {
    w[s] = wok ? *reinterpret_cast<const bf16x8*>(wr + s * 32) : bf16x8{};
    x[s] = *reinterpret_cast<const bf16x8*>(xr + s * 32);
  }
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
  for (int s = 0; s < kColsSteps; s += 2) {
    acc0 = mfma16x16x32(w[s], x[s], acc0);
    acc1 = mfma16x16x32(w[s + 1], x[s + 1], acc1);
  }
  if (!ok || lg * 4 >= NC) return;
  const f32x4 o = acc0 + acc1;
  uint2 packed;
  packed.x = pack_bf16x2(o[0], o[1]);
  packed.y = pack_bf16x2(o[2], o[3]);
  *reinterpret_cast<uint2*>(a.y + (int64_t)l16 * a.y_stride + n0 + lg * 4) = packed;
}

template <int MT, int PRO, int EPI, int KS, int NC>
hipError_t launch_tiles(const LinearArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((skinny_gemm_kernel<MT, PRO, EPI, KS, NC>), dim3((unsigned)(a.N / NC)),
                     dim3(kGemmThreads), 0, stream, AIOS_LINEAR_HOT_ARGS(a));
  return hipGetLastError();
}

// nc: columns per workgroup for one row tile -- 8 for projections with at
// most one 16-column tile per two compute units, 4 for at most one per
// four (2x / 4x the workgroups at 1/2 / 1/4 of the weight bytes each; the
// MFMA tile's other W rows read as zero).  Measured per replayed decode step: the hidden-768
// models' qkv, gate/up and down (80, 128, 48 tiles) gain ~2%; Qwen3-0.6B's
// qkv and gate/up (256 and 192 tiles, each workgroup also re-reading its
// 32 KB of norm-prologue rows) lost 5% with 8-column tiles.  4 columns for
// the down and o projections (48-64 tiles) gained another 1-2%.
template <int PRO, int EPI, int KS>
hipError_t launch_one_tile(const LinearArgs& a, int nc, hipStream_t stream) {
  if (nc == 4) return launch_tiles<1, PRO, EPI, KS, 4>(a, stream);
  if (nc == 8) return launch_tiles<1, PRO, EPI, KS, 8>(a, stream);
  return launch_tiles<1, PRO, EPI, KS, 16>(a, stream);
}

template <int PRO, int EPI>
hipError_t launch_pe(const LinearArgs& a, int nc, hipStream_t stream) {
  if ((a.M + 15) / 16 == 1) {
    // the decode-step shapes: K = 768, 1024, 2048, 3072 with a fixed step count
    switch (a.K / 128) {
      case 6: return launch_one_tile<PRO, EPI, 6>(a, nc, stream);
      case 8: return launch_one_tile<PRO, EPI, 8>(a, nc, stream);
      case 16:
        if constexpr (PRO == kPlain) return launch_one_tile<PRO, EPI, 16>(a, nc, stream);
        break;
      case 24:  // K 3072 (the down projection of hidden-1024 models)
        if constexpr (PRO == kPlain) return launch_one_tile<PRO, EPI, 24>(a, nc, stream);
        break;
      default: break;
    }
    return launch_one_tile<PRO, EPI, 0>(a, nc, stream);
  }
  switch ((a.M + 15) / 16) {
    case 2: return launch_tiles<2, PRO, EPI, 0, 16>(a, stream);
    case 3: return launch_tiles<3, PRO, EPI, 0, 16>(a, stream);
    case 4: return launch_tiles<4, PRO, EPI, 0, 16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool skinny_gemm_supported(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && M <= 64 && N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0 &&
         N / 16 <= 0x7fffffff;
}

bool skinny_gemm_norm_supported(int64_t M, int64_t K) {
  const int64_t mt = (M + 15) / 16;
  return mt >= 1 && mt <= 4 && (K / 4) / 32 <= kNormMaxFrags / mt;
}

// Compute units of the current device (looked up once per process).
int stream_grid_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    cus = (hipGetDevice(&dev) == hipSuccess &&
           hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
           n > 0)
              ? n
              : 256;
  }
  return cus;
}

template <int PRO, int KS>
hipError_t launch_stream(const LinearArgs& a, int64_t grid, hipStream_t stream) {
  hipLaunchKernelGGL((skinny_gemm_stream_kernel<PRO, KS>), dim3((unsigned)grid),
                     dim3(kGemmThreads), 0, stream, AIOS_LINEAR_HOT_ARGS(a));
  return hipGetLastError();
}

hipError_t skinny_gemm(const LinearArgs& a, int prologue, int epilogue, hipStream_t stream) {
  // (the preloaded strides and column count are 32-bit)
  if (a.x_stride > 0x7fffffff || a.w_stride > 0x7fffffff || a.N > 0x7fffffff)
    return hipErrorInvalidValue;
  // Many column tiles, one row tile, K 768 / 1024: the streaming kernel,
  // when every workgroup then walks at least two tiles (and at most the
  // tiles it can stage).
  const int64_t stream_grid = (int64_t)kStreamWgsPerCu * stream_grid_cus();
  const int64_t tiles = a.N / 16;
  if (epilogue == kStore && a.M <= 16 && tiles >= 2 * stream_grid &&
      tiles <= (int64_t)kStreamMaxIters * stream_grid && (a.K == 768 || a.K == 1024) &&
      a.N * a.w_stride * 2 < ((int64_t)1 << 31)) {
    if (prologue == kPlain)
      return a.K == 768 ? launch_stream<kPlain, 6>(a, stream_grid, stream)
                        : launch_stream<kPlain, 8>(a, stream_grid, stream);
    if (prologue == kAddNorm)
      return a.K == 768 ? launch_stream<kAddNorm, 6>(a, stream_grid, stream)
                        : launch_stream<kAddNorm, 8>(a, stream_grid, stream);
  }
  if (prologue == kPlain && epilogue == kStore && a.M <= 16 && a.K == kColsSteps * 32) {
    const int cus = stream_grid_cus();
    if (4 * tiles <= cus)
      hipLaunchKernelGGL(skinny_gemm_cols_kernel<4>, dim3((unsigned)(a.N / 4)), dim3(64), 0, stream,
                         AIOS_LINEAR_HOT_ARGS(a));
    else if (2 * tiles <= cus)
      hipLaunchKernelGGL(skinny_gemm_cols_kernel<8>, dim3((unsigned)(a.N / 8)), dim3(64), 0, stream,
                         AIOS_LINEAR_HOT_ARGS(a));
    else
      hipLaunchKernelGGL(skinny_gemm_cols_kernel<16>, dim3((unsigned)(a.N / 16)), dim3(64), 0, stream,
                         AIOS_LINEAR_HOT_ARGS(a));
    return hipGetLastError();
  }
  const int cus = stream_grid_cus();
  const int nc = 4 * tiles <= cus ? 4 : (2 * tiles <= cus ? 8 : 16);
  if (prologue == kPlain && epilogue == kStore) return launch_pe<kPlain, kStore>(a, nc, stream);
  if (prologue == kPlain && epilogue == kSiluPair)
    return launch_pe<kPlain, kSiluPair>(a, nc, stream);
  if (prologue == kAddNorm && epilogue == kStore)
    return launch_pe<kAddNorm, kStore>(a, nc, stream);
  if (prologue == kAddNorm && epilogue == kSiluPair)
    return launch_pe<kAddNorm, kSiluPair>(a, nc, stream);
  return hipErrorInvalidValue;
}

}  // namespace aios
