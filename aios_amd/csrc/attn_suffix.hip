// Per-row ragged paged decode (kernel (d)) and the log-sum-exp combine.
//
// One wavefront owns one (row, kv-head, split).  The 64 lanes form four
// 16-lane DPP rows; each DPP row walks its own KV positions (position
// t0 + 4u + row) and each of its 16 lanes holds D/16 consecutive dims of
// the K and V rows, so a dot product is a per-lane partial sum plus one
// 4-step DPP row reduction, and every K/V row is read as one contiguous
// D*2-byte segment.  All G query heads of the kv-head are processed
// together, so each K/V row is read once per candidate row.  The running
// softmax state (m, l, acc) of the four DPP rows is merged with cross-row
// shuffles at the end.
//
// With a shared prefix the cascade kernel leaves one normalised partial
// (o, lse) per prefix chunk; finalisation folds them into the wave's state
// using  m = max(m1, m2),  l = l1*2^(m1-m) + l2*2^(m2-m),
// acc = acc1*2^(m1-m) + acc2*2^(m2-m)  (log2 domain), the split/merge rule
// of online softmax (resources/lesson-41-flashattention-online-softmax/
// run_lesson41.py:7-18), then writes out = acc / l in bf16.
#include "kernels.hpp"

namespace aios {

template <int E>
struct RowSlice {
  uint32_t w[E / 2];
};

template <int E>
__device__ __forceinline__ RowSlice<E> load_slice(const bf16* p) {
  RowSlice<E> r;
  if constexpr (E == 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  } else if constexpr (E == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    r.w[0] = v.x; r.w[1] = v.y;
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < E / 2; ++i) r.w[i] = q[i];
  }
  return r;
}

template <int E>
__device__ __forceinline__ void slice_to_float(const RowSlice<E>& s, float (&x)[E]) {
#pragma unroll
  for (int i = 0; i < E / 2; ++i) {
    x[2 * i] = lo_bf16(s.w[i]);
    x[2 * i + 1] = hi_bf16(s.w[i]);
  }
}

template <int E, int G>
struct SoftState {
  float m[G];
  float l[G];
  float acc[G][E];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegInf;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
    }
  }
  // Fold in a normalised partial (o, lse) for head g.
  __device__ __forceinline__ void merge_partial(int g, float lse, const float (&o)[E]) {
    const float m_new = fmaxf(m[g], lse);
    const float mu = (m_new == kNegInf) ? 0.f : m_new;
    const float fa = fast_exp2(m[g] - mu);
    const float fb = fast_exp2(lse - mu);
    l[g] = l[g] * fa + fb;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = acc[g][e] * fa + o[e] * fb;
    m[g] = m_new;
  }
  // Merge the states of the four DPP rows; afterwards every lane of a
  // column holds the merged state.
  __device__ __forceinline__ void merge_rows() {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mx = xrow_max(m[g]);
      const float mu = (mx == kNegInf) ? 0.f : mx;
      const float f = fast_exp2(m[g] - mu);
      l[g] = xrow_sum(l[g] * f);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][e] = xrow_sum(acc[g][e] * f);
      m[g] = mx;
    }
  }
};

template <int D, int G, bool FINAL>
__global__ __launch_bounds__(64) void attn_suffix_kernel(SuffixArgs a) {
  constexpr int E = D / 16;
  constexpr int U = 2;  // KV positions per DPP row per iteration
  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int split = blockIdx.x;
  const int b = blockIdx.y;
  const int h = blockIdx.z;

  const int base = a.cu_k[b];
  const int kv_len = a.cu_k[b + 1] - base;
  const int s_begin = a.prefix_len + split * a.split_len;
  const int s_end = min(kv_len, s_begin + a.split_len);

  float q[G][E];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const RowSlice<E> qs =
        load_slice<E>(a.q + (int64_t)b * a.q_tok_stride + (int64_t)(h * G + g) * D + l16 * E);
    slice_to_float<E>(qs, q[g]);
  }

  SoftState<E, G> st;
  st.init();
  const bf16* kb = a.k_cache + (int64_t)h * D + l16 * E;
  const bf16* vb = a.v_cache + (int64_t)h * D + l16 * E;

  for (int t0 = s_begin; t0 < s_end; t0 += 4 * U) {
    RowSlice<E> ks[U], vs[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + 4 * u + lg;
      ok[u] = t < s_end;
      const int64_t page = ok[u] ? (int64_t)a.indices[base + t] : -1;
      if ((uint64_t)page < (uint64_t)a.num_pages) {
        ks[u] = load_slice<E>(kb + page * a.kv_tok_stride);
        vs[u] = load_slice<E>(vb + page * a.kv_tok_stride);
      } else {
#pragma unroll
        for (int i = 0; i < E / 2; ++i) ks[u].w[i] = vs[u].w[i] = 0u;
      }
    }
    float sc[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[E];
      slice_to_float<E>(ks[u], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) d = fmaf(q[g][e], kf[e], d);
        d = row16_sum(d);
        sc[u][g] = ok[u] ? d * a.scale_log2 : kNegInf;
      }
    }
    float vf[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) slice_to_float<E>(vs[u], vf[u]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, sc[u][g]);
      const float m_new = fmaxf(st.m[g], mx);
      const float mu = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = fast_exp2(st.m[g] - mu);
      float p[U];
      float ps = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[u] = fast_exp2(sc[u][g] - mu);
        ps += p[u];
      }
      st.l[g] = st.l[g] * alpha + ps;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float acc = st.acc[g][e] * alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) acc = fmaf(p[u], vf[u][e], acc);
        st.acc[g][e] = acc;
      }
      st.m[g] = m_new;
    }
  }

  if constexpr (FINAL) {
    // Fold in the prefix-chunk partials of rows b*G + g (chunks c = lg mod 4).
    for (int c = lg; c < a.pre_chunks; c += 4) {
      const int64_t slot0 = ((int64_t)c * a.num_kv_heads + h) * a.m_rows + (int64_t)b * G;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float lse = a.pre_lse[slot0 + g];
        const float* po = a.pre_o + (slot0 + g) * D + l16 * E;
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = po[e];
        st.merge_partial(g, lse, o);
      }
    }
  }
  st.merge_rows();

  if (lg != 0) return;
  if constexpr (FINAL) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float inv = st.l[g] > 0.f ? 1.f / st.l[g] : 0.f;
      bf16* po = a.out + ((int64_t)b * a.num_qo_heads + h * G + g) * D + l16 * E;
      uint32_t* pw = reinterpret_cast<uint32_t*>(po);
#pragma unroll
      for (int i = 0; i < E / 2; ++i)
        pw[i] = pack_bf16x2(st.acc[g][2 * i] * inv, st.acc[g][2 * i + 1] * inv);
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t slot = ((int64_t)b * a.num_splits + split) * a.num_qo_heads + h * G + g;
      const float inv = st.l[g] > 0.f ? 1.f / st.l[g] : 0.f;
      float* po = a.suf_o + slot * D + l16 * E;
#pragma unroll
      for (int e = 0; e < E; ++e) po[e] = st.acc[g][e] * inv;
      if (l16 == 0) a.suf_lse[slot] = st.l[g] > 0.f ? st.m[g] + fast_log2(st.l[g]) : kNegInf;
    }
  }
}

// Merge prefix-chunk partials and suffix-split partials of row b, kv-head h.
template <int D, int G>
__global__ __launch_bounds__(64) void attn_combine_kernel(SuffixArgs a) {
  constexpr int E = D / 16;
  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int b = blockIdx.x;
  const int h = blockIdx.y;

  SoftState<E, G> st;
  st.init();
  for (int c = lg; c < a.pre_chunks; c += 4) {
    const int64_t slot0 = ((int64_t)c * a.num_kv_heads + h) * a.m_rows + (int64_t)b * G;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float* po = a.pre_o + (slot0 + g) * D + l16 * E;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = po[e];
      st.merge_partial(g, a.pre_lse[slot0 + g], o);
    }
  }
  for (int s = lg; s < a.num_splits; s += 4) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t slot = ((int64_t)b * a.num_splits + s) * a.num_qo_heads + h * G + g;
      const float* po = a.suf_o + slot * D + l16 * E;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = po[e];
      st.merge_partial(g, a.suf_lse[slot], o);
    }
  }
  st.merge_rows();
  if (lg != 0) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float inv = st.l[g] > 0.f ? 1.f / st.l[g] : 0.f;
    bf16* po = a.out + ((int64_t)b * a.num_qo_heads + h * G + g) * D + l16 * E;
    uint32_t* pw = reinterpret_cast<uint32_t*>(po);
#pragma unroll
    for (int i = 0; i < E / 2; ++i)
      pw[i] = pack_bf16x2(st.acc[g][2 * i] * inv, st.acc[g][2 * i + 1] * inv);
  }
}

bool suffix_supported(int D, int G) {
  const bool d_ok = D == 64 || D == 96 || D == 128;
  const bool g_ok = G == 1 || G == 2 || G == 3 || G == 4 || G == 6 || G == 8;
  return d_ok && g_ok;
}

template <int D, int G>
static hipError_t suffix_dg(bool finalize, bool combine, const SuffixArgs& a,
                            hipStream_t stream) {
  if (combine) {
    hipLaunchKernelGGL((attn_combine_kernel<D, G>), dim3(a.batch, a.num_kv_heads), dim3(64), 0,
                       stream, a);
  } else {
    const dim3 grid(a.num_splits, a.batch, a.num_kv_heads);
    if (finalize)
      hipLaunchKernelGGL((attn_suffix_kernel<D, G, true>), grid, dim3(64), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_suffix_kernel<D, G, false>), grid, dim3(64), 0, stream, a);
  }
  return hipGetLastError();
}

template <int D>
static hipError_t suffix_d(int G, bool finalize, bool combine, const SuffixArgs& a,
                           hipStream_t stream) {
  switch (G) {
    case 1: return suffix_dg<D, 1>(finalize, combine, a, stream);
    case 2: return suffix_dg<D, 2>(finalize, combine, a, stream);
    case 3: return suffix_dg<D, 3>(finalize, combine, a, stream);
    case 4: return suffix_dg<D, 4>(finalize, combine, a, stream);
    case 6: return suffix_dg<D, 6>(finalize, combine, a, stream);
    case 8: return suffix_dg<D, 8>(finalize, combine, a, stream);
    default: return hipErrorInvalidValue;
  }
}

static hipError_t suffix_dispatch(int D, int G, bool finalize, bool combine,
                                  const SuffixArgs& a, hipStream_t stream) {
  switch (D) {
    case 64: return suffix_d<64>(G, finalize, combine, a, stream);
    case 96: return suffix_d<96>(G, finalize, combine, a, stream);
    case 128: return suffix_d<128>(G, finalize, combine, a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_suffix(int D, int G, bool finalize, const SuffixArgs& a, hipStream_t stream) {
  return suffix_dispatch(D, G, finalize, false, a, stream);
}

hipError_t launch_combine(int D, int G, const SuffixArgs& a, hipStream_t stream) {
  return suffix_dispatch(D, G, false, true, a, stream);
}

}  // namespace aios
