// MFMA attention tile engine for gfx950: shared-prefix cascade decode
// (kernel (c)) and varlen causal paged prefill (kernel (b)).
//
// One workgroup owns one kv-head and NW*32 query rows.  A query row is a
// (candidate, q-head) pair in cascade mode and a (token, q-head) pair in
// prefill mode, so all query heads of a GQA group share one K/V stream.
// K/V are gathered through the page-index list 32 tokens at a time into
// LDS (double buffered, next tile prefetched into registers while the
// current one is consumed):
//   Ks[token][dim]   token-major, rows padded by 16 B (conflict-free reads)
//   Vt[dim][slot]    dim-major with the tile's tokens permuted so that the
//                    P^T fragment each lane already holds after the QK step
//                    is directly the B operand of the PV step.
// Each wave computes S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A = K from
// LDS, B = Q held in registers), keeps one query row per lane column so the
// online-softmax statistics are lane-local, and accumulates O^T = V^T P^T in
// registers.  The math is the offset-causal GQA softmax attention of
// python/aios/attention/flashinfer.py:33-91 (decode = the same with q_len 1).
#include "kernels.hpp"

namespace aios {

constexpr int kTileTok = 32;
constexpr int kVtStride = kTileTok + 8;  // Vt row stride (elements): 80 B

enum { kModeCascade = 0, kModePrefill = 1 };



// Slot of tile token t inside a Vt row: the lane group g holding tokens
// {4g..4g+3} and {16+4g..16+4g+3} after the S^T step reads slots 8g..8g+7.
__device__ __forceinline__ int vt_slot(int t) {
  return ((t & 15) >> 2) * 8 + (t >> 4) * 4 + (t & 3);
}

template <int D, int NW, int MODE>
__global__ __launch_bounds__(NW * 64) void attn_tile_kernel(TileArgs a) {
  constexpr int NT = NW * 64;
  constexpr int KSTEPS = D / 32;
  constexpr int DTILES = D / 16;
  constexpr int KSTR = D + 8;
  constexpr int CPR = D / 8;             // 16-byte chunks per token row
  constexpr int UNITS = 2 * 8 * CPR;     // (K|V) x token-quad x chunk
  constexpr int UPT = (UNITS + NT - 1) / NT;

  __shared__ __align__(16) bf16 Ks[2][kTileTok * KSTR];
  __shared__ __align__(16) bf16 Vt[2][D * kVtStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int h = blockIdx.y;
  const int G = a.group;

  // ---- work assignment --------------------------------------------------
  int kv_begin, kv_end, idx_base;
  int row_limit[2];     // prefill: last visible KV position per row
  bool row_ok[2];
  const bf16* qrow[2];
  int64_t out_off[2];   // prefill: element offset of the row's output
  int prow[2];          // cascade: row index into partials
  int q_start = 0, q_len = 0, cached = 0, qt = 0;
  if (MODE == kModeCascade) {
    const int chunk = blockIdx.x;
    kv_begin = chunk * a.chunk_len;
    kv_end = min(a.prefix_len, kv_begin + a.chunk_len);
    idx_base = 0;
    for (int rt = 0; rt < 2; ++rt) {
      const int m = blockIdx.z * (NW * 32) + wave * 32 + rt * 16 + l16;
      row_ok[rt] = m < a.m_rows;
      const int b = m / G, g = m - (m / G) * G;
      qrow[rt] = a.q + (int64_t)b * a.q_tok_stride + (int64_t)(h * G + g) * D;
      prow[rt] = m;
      row_limit[rt] = 0x7fffffff;
      out_off[rt] = 0;
    }
  } else {
    const int r = blockIdx.z;
    qt = blockIdx.x;
    q_start = a.cu_q[r];
    q_len = a.cu_q[r + 1] - q_start;
    if (qt * a.q_tile >= q_len) return;
    const int kv_len = a.cu_k[r + 1] - a.cu_k[r];
    cached = kv_len - q_len;
    const int q_hi = min(q_len, (qt + 1) * a.q_tile);
    kv_begin = 0;
    kv_end = min(kv_len, cached + q_hi);
    idx_base = a.cu_k[r];
    for (int rt = 0; rt < 2; ++rt) {
      const int m = wave * 32 + rt * 16 + l16;
      const int i = qt * a.q_tile + m / G;
      const int g = m - (m / G) * G;
      row_ok[rt] = (m < a.q_tile * G) && (i < q_len);
      qrow[rt] = a.q + (int64_t)(q_start + i) * a.q_tok_stride + (int64_t)(h * G + g) * D;
      out_off[rt] = ((int64_t)(q_start + i) * a.num_qo_heads + (h * G + g)) * D;
      row_limit[rt] = cached + i;
      prow[rt] = 0;
    }
  }

  // ---- Q fragments (B operand of S^T = K Q^T) ---------------------------
  bf16x8 qf[2][KSTEPS];
  for (int rt = 0; rt < 2; ++rt)
    for (int s = 0; s < KSTEPS; ++s) {
      if (row_ok[rt])
        qf[rt][s] = *reinterpret_cast<const bf16x8*>(qrow[rt] + s * 32 + lg * 8);
      else
        qf[rt][s] = bf16x8{};
    }

  f32x4 o[2][DTILES];
  for (int rt = 0; rt < 2; ++rt)
    for (int dt = 0; dt < DTILES; ++dt) o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {kNegInf, kNegInf};
  float l_run[2] = {0.f, 0.f};

  const bf16* kbase = a.k_cache + (int64_t)h * D;
  const bf16* vbase = a.v_cache + (int64_t)h * D;

  // ---- staging: registers <- HBM, LDS <- registers ----------------------
  uint4 stage[UPT][4];
  auto load_tile = [&](int kv0) {
#pragma unroll
    for (int up = 0; up < UPT; ++up) {
      const int u = tid + up * NT;
      if (u < UNITS) {
        const bool isv = u >= UNITS / 2;
        const int uu = isv ? u - UNITS / 2 : u;
        const int quad = uu / CPR;
        const int c = uu - quad * CPR;
        const bf16* base = isv ? vbase : kbase;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pos = kv0 + quad * 4 + i;
          const int64_t page = pos < kv_end ? (int64_t)a.indices[idx_base + pos] : -1;
          if ((uint64_t)page < (uint64_t)a.num_pages)
            stage[up][i] = *reinterpret_cast<const uint4*>(base + page * a.kv_tok_stride + c * 8);
          else
            stage[up][i] = make_uint4(0, 0, 0, 0);
        }
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int up = 0; up < UPT; ++up) {
      const int u = tid + up * NT;
      if (u < UNITS) {
        const bool isv = u >= UNITS / 2;
        const int uu = isv ? u - UNITS / 2 : u;
        const int quad = uu / CPR;
        const int c = uu - quad * CPR;
        if (!isv) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(&Ks[buf][(quad * 4 + i) * KSTR + c * 8]) = stage[up][i];
        } else {
          const int slot = vt_slot(quad * 4);
          const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&stage[up][0]);
          const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&stage[up][1]);
          const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&stage[up][2]);
          const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&stage[up][3]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // dims c*8 + 2e (low halves) and c*8 + 2e + 1 (high halves)
            uint2 lo, hi;
            lo.x = __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u);
            lo.y = __builtin_amdgcn_perm(w3[e], w2[e], 0x05040100u);
            hi.x = __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u);
            hi.y = __builtin_amdgcn_perm(w3[e], w2[e], 0x07060302u);
            *reinterpret_cast<uint2*>(&Vt[buf][(c * 8 + 2 * e) * kVtStride + slot]) = lo;
            *reinterpret_cast<uint2*>(&Vt[buf][(c * 8 + 2 * e + 1) * kVtStride + slot]) = hi;
          }
        }
      }
    }
  };

  const int n_tiles = (kv_end - kv_begin + kTileTok - 1) / kTileTok;
  if (n_tiles > 0) {
    load_tile(kv_begin);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int buf = it & 1;
    const int kv0 = kv_begin + it * kTileTok;
    if (it + 1 < n_tiles) load_tile(kv0 + kTileTok);

    // S^T tiles: st[rt][tt] holds S[row rt*16+l16][token tt*16 + lg*4 + i]
    f32x4 st[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      st[0][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
      st[1][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const bf16x8 kf =
            *reinterpret_cast<const bf16x8*>(&Ks[buf][(tt * 16 + l16) * KSTR + s * 32 + lg * 8]);
        st[0][tt] = mfma16x16x32(kf, qf[0][s], st[0][tt]);
        st[1][tt] = mfma16x16x32(kf, qf[1][s], st[1][tt]);
      }
    }

    // Online softmax (log2 domain), one query row per lane column.
    bf16x8 pb[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float x[8];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pos = kv0 + tt * 16 + lg * 4 + i;
          bool ok = pos < kv_end;
          if (MODE == kModePrefill) ok = ok && pos <= row_limit[rt];
          x[tt * 4 + i] = ok ? st[rt][tt][i] * a.scale_log2 : kNegInf;
        }
      float mx = x[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mx = fmaxf(mx, x[j]);
      mx = xrow_max(mx);
      const float m_new = fmaxf(m_run[rt], mx);
      const float m_use = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[rt] - m_use);
      float p[8];
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = fast_exp2(x[j] - m_use);
        psum += p[j];
      }
      l_run[rt] = l_run[rt] * alpha + psum;
      m_run[rt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) o[rt][dt] *= alpha;
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(p[2 * j], p[2 * j + 1]);
      pb[rt] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
    }

    // O^T += V^T P^T
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) {
      const bf16x8 vf =
          *reinterpret_cast<const bf16x8*>(&Vt[buf][(dt * 16 + l16) * kVtStride + lg * 8]);
      o[0][dt] = mfma16x16x32(vf, pb[0], o[0][dt]);
      o[1][dt] = mfma16x16x32(vf, pb[1], o[1][dt]);
    }

    if (it + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ------------------------------------------------------------
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const float l_tot = xrow_sum(l_run[rt]);
    if (!row_ok[rt]) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (MODE == kModeCascade) {
      const int64_t slot = ((int64_t)blockIdx.x * a.num_kv_heads + h) * a.m_rows + prow[rt];
      float* po = a.part_o + slot * D;
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        const f32x4 v = o[rt][dt] * inv;
        *reinterpret_cast<f32x4*>(po + dt * 16 + lg * 4) = v;
      }
      if (lg == 0)
        a.part_lse[slot] = l_tot > 0.f ? m_run[rt] + fast_log2(l_tot) : kNegInf;
    } else {
      bf16* po = a.out + out_off[rt];
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        const f32x4 v = o[rt][dt] * inv;
        uint2 packed;
        packed.x = pack_bf16x2(v[0], v[1]);
        packed.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(po + dt * 16 + lg * 4) = packed;
      }
    }
  }
}

template <int D, int NW, int MODE>
static hipError_t launch_tile(const TileArgs& a, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((attn_tile_kernel<D, NW, MODE>), grid, dim3(NW * 64), 0, stream, a);
  return hipGetLastError();
}

template <int MODE>
static hipError_t dispatch_tile(int D, int NW, const TileArgs& a, dim3 grid,
                                hipStream_t stream) {
#define AIOS_TILE_NW(DD)                                     \
  switch (NW) {                                              \
    case 1: return launch_tile<DD, 1, MODE>(a, grid, stream); \
    case 2: return launch_tile<DD, 2, MODE>(a, grid, stream); \
    case 3: return launch_tile<DD, 3, MODE>(a, grid, stream); \
    case 4: return launch_tile<DD, 4, MODE>(a, grid, stream); \
    default: return hipErrorInvalidValue;                    \
  }
  switch (D) {
    case 64: AIOS_TILE_NW(64)
    case 96: AIOS_TILE_NW(96)
    case 128: AIOS_TILE_NW(128)
    default: return hipErrorInvalidValue;
  }
#undef AIOS_TILE_NW
}

bool tile_supported(int D) { return D == 64 || D == 96 || D == 128; }

hipError_t launch_cascade(int D, int NW, const TileArgs& a, int chunks, int mgroups,
                          hipStream_t stream) {
  return dispatch_tile<kModeCascade>(D, NW, a, dim3(chunks, a.num_kv_heads, mgroups), stream);
}

hipError_t launch_prefill(int D, int NW, const TileArgs& a, int q_tiles, int batch,
                          hipStream_t stream) {
  return dispatch_tile<kModePrefill>(D, NW, a, dim3(q_tiles, a.num_kv_heads, batch), stream);
}

}  // namespace aios
