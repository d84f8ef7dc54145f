// Token selection with the raw log-probability of the chosen token:
// greedy_kernel (argmax) and sample_kernel (stateless temperature / top-k /
// top-p sampling, python/aios/engine/sample.py:12-160).
//
// Greedy:
// One workgroup per row.  token = the first index of the row maximum of the
// logits as stored (torch's argmax on the sampling logits); logprob =
// x[token] - logsumexp(x) in fp32 (log_softmax of the fp32-widened logits,
// gathered at the token).  Each lane keeps an online (max, first index,
// sum of exp(x - max)) state over its 8-logit chunks of the row (several
// 16-byte loads in flight: the row is read in a few memory round trips, not
// one per 256 logits); states merge across the wavefront with shuffles and
// across waves through LDS.
#include "kernels.hpp"

namespace aios {
namespace {

constexpr int kGreedyThreads = 256;

struct ArgState {
  float m;    // running maximum (log2-scaled)
  int32_t i;  // first index holding it
  float s;    // sum of 2^(x - m)
};

__device__ __forceinline__ ArgState merge(ArgState a, ArgState b) {
  ArgState r;
  if (b.m > a.m || (b.m == a.m && b.i < a.i)) {
    r.m = b.m;
    r.i = b.i;
  } else {
    r.m = a.m;
    r.i = a.i;
  }
  const float sa = a.m == kNegInf ? 0.f : a.s * fast_exp2(a.m - r.m);
  const float sb = b.m == kNegInf ? 0.f : b.s * fast_exp2(b.m - r.m);
  r.s = sa + sb;
  return r;
}

template <typename T>
__device__ __forceinline__ float load_logit(const T* p) {
  return static_cast<float>(*p);
}

// Eight consecutive logits (16-byte aligned) as fp32.
__device__ __forceinline__ void load8f(const bf16* p, float* f) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x); f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
  f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z); f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
}
__device__ __forceinline__ void load8f(const float* p, float* f) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

constexpr int kGreedyUnroll = 4;  // 8-logit chunks per thread in flight

template <typename T>
__global__ __launch_bounds__(kGreedyThreads) void greedy_kernel(
    const T* __restrict__ logits, int64_t row_stride, int32_t vocab,
    int64_t* __restrict__ token_out, float* __restrict__ logprob_out) {
  const int row = blockIdx.x;
  const T* x = logits + (int64_t)row * row_stride;
  ArgState st = {kNegInf, 0x7fffffff, 0.f};
  auto visit = [&](float v, int32_t j) {
    v *= kLog2e;
    if (v > st.m) {
      st.s = (st.m == kNegInf ? 0.f : st.s * fast_exp2(st.m - v)) + 1.f;
      st.m = v;
      st.i = j;
    } else if (v != kNegInf) {
      st.s += fast_exp2(v - st.m);
    }
  };
  // Whole 8-logit chunks with several 16-byte loads in flight per thread
  // (unconditional: a chunk past the last whole one re-reads that one and
  // is skipped), then the rest one by one.  Each thread visits its ids in
  // increasing order, so its state keeps the first index of its maximum.
  const int whole = ((uintptr_t)x & 15) == 0 ? (vocab & ~7) : 0;
  for (int base = 0; base < whole; base += kGreedyThreads * 8 * kGreedyUnroll) {
    float f[kGreedyUnroll][8];
    int i0[kGreedyUnroll];
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u) {
      i0[u] = base + (u * kGreedyThreads + (int)threadIdx.x) * 8;
      load8f(x + min(i0[u], whole - 8), f[u]);
    }
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u)
      if (i0[u] < whole) {
#pragma unroll
        for (int j = 0; j < 8; ++j) visit(f[u][j], i0[u] + j);
      }
  }
  for (int32_t j = whole + threadIdx.x; j < vocab; j += kGreedyThreads) visit(load_logit(x + j), j);
  for (int off = 32; off > 0; off >>= 1) {
    ArgState o;
    o.m = __shfl_xor(st.m, off);
    o.i = __shfl_xor(st.i, off);
    o.s = __shfl_xor(st.s, off);
    st = merge(st, o);
  }
  __shared__ ArgState waves[kGreedyThreads / 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (lane == 0) waves[wave] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgState r = waves[0];
    for (int w = 1; w < kGreedyThreads / 64; ++w) r = merge(r, waves[w]);
    token_out[row] = r.i;
    // log_softmax at the maximum: -ln(sum exp(x - max)).
    logprob_out[row] = -fast_log2(r.s) * 0.6931471805599453f;
  }
}

// ---------------------------------------------------------------------------
// Stateless sampling.  One workgroup of 256 threads per row:
//  1. forbidden ids (the global list while step < forbid_before_step, and
//     the row's own list) are deduplicated into LDS; the sampling logits are
//     the logits with those ids at -inf;
//  2. top-k by radix selection on an order-preserving integer key of the
//     logit (16-bit for bf16, 32-bit for fp32), four bits per pass: each
//     pass counts, in registers, the ids whose key matches the prefix
//     found so far and whose next digit is >= j for j = 1..15 (no
//     histogram atomics: logits crowd into a few high-order digits), then
//     the forbidden ids' contributions are moved to the -inf key.  The first
//     pass also accumulates the raw log-sum-exp (the returned log-prob is of
//     the unmodified distribution, sample.py:77);
//  3. the k winners are gathered in id order (tiles of 2048 ids, a block
//     scan gives each its slot; of the ids equal to the k-th key the lowest
//     ones are taken) and bitonic-sorted in LDS by (value desc, id asc);
//  4. wavefront 0: softmax of (value / temperature), cumulative sums, the
//     top-p cut, softmax again, and position = #(cumulative < u), clamped.
// top_k == 0 with top_p == 1 samples every id in id order (a block scan of
// the probabilities over tiles until u is passed).

constexpr int kSampleThreads = 256;
constexpr int kSampleWaves = kSampleThreads / 64;
constexpr int kSampleTile = kSampleThreads * 8;
constexpr int kSampleUnroll = 8;  // 16-byte chunks per thread in flight per sweep
// candidates (ids at or above the k-th key) gathered without order; more
// ties than fit take the id-ordered gather instead
constexpr int kSampleGatherCap = 2048;
constexpr int kSampleRankSort = 1024;
static_assert(kSampleGatherCap >= kSampleMaxTopK, "the sorted buffer holds the top k");

// Order-preserving keys: larger value <=> larger key.
__device__ __forceinline__ uint32_t order_key32(uint32_t b) {
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ uint32_t order_unkey32(uint32_t k) {
  return (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
}

template <typename T>
struct LogitTraits;
template <>
struct LogitTraits<bf16> {
  static constexpr int kBits = 16;
  static __device__ __forceinline__ uint32_t key(uint32_t bits16) {
    return order_key32(bits16 << 16) >> 16;
  }
  static __device__ __forceinline__ float value(uint32_t key) {
    return __uint_as_float(order_unkey32(key << 16) & 0xffff0000u);
  }
  // Eight consecutive logits: raw bit patterns.
  static __device__ __forceinline__ void load8(const bf16* p, uint32_t* b) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    b[0] = v.x & 0xffff; b[1] = v.x >> 16; b[2] = v.y & 0xffff; b[3] = v.y >> 16;
    b[4] = v.z & 0xffff; b[5] = v.z >> 16; b[6] = v.w & 0xffff; b[7] = v.w >> 16;
  }
  static __device__ __forceinline__ uint32_t load1(const bf16* p) {
    return __builtin_bit_cast(uint16_t, *p);
  }
  static __device__ __forceinline__ float to_float(uint32_t b) { return __uint_as_float(b << 16); }
};
template <>
struct LogitTraits<float> {
  static constexpr int kBits = 32;
  static __device__ __forceinline__ uint32_t key(uint32_t bits) { return order_key32(bits); }
  static __device__ __forceinline__ float value(uint32_t key) {
    return __uint_as_float(order_unkey32(key));
  }
  static __device__ __forceinline__ void load8(const float* p, uint32_t* b) {
    const uint4 v0 = *reinterpret_cast<const uint4*>(p);
    const uint4 v1 = *reinterpret_cast<const uint4*>(p + 4);
    b[0] = v0.x; b[1] = v0.y; b[2] = v0.z; b[3] = v0.w;
    b[4] = v1.x; b[5] = v1.y; b[6] = v1.z; b[7] = v1.w;
  }
  static __device__ __forceinline__ uint32_t load1(const float* p) {
    return __float_as_uint(*p);
  }
  static __device__ __forceinline__ float to_float(uint32_t b) { return __uint_as_float(b); }
};

__device__ __forceinline__ int wave_sum_i(int v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ int wave_incl_scan_i(int v, int lane) {
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off);
    if (lane >= off) v += t;
  }
  return v;
}
__device__ __forceinline__ float wave_incl_scan_f(float v, int lane) {
  for (int off = 1; off < 64; off <<= 1) {
    const float t = __shfl_up(v, off);
    if (lane >= off) v += t;
  }
  return v;
}

struct SampleShared {
  int32_t fset[kSampleMaxForbidden];   // distinct forbidden ids
  uint32_t fkey[kSampleMaxForbidden];  // their raw keys
  int nf;
  int ired[2][kSampleWaves][16];
  float fred[kSampleWaves][2];
  int iscan[kSampleWaves];
  float fscan[kSampleWaves];
  int ngather;
  unsigned long long cand[kSampleGatherCap];
  unsigned long long top[kSampleMaxTopK];  // the k winners, in order
};

template <typename T>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(SampleArgs a) {
  using L = LogitTraits<T>;
  constexpr int kPasses = L::kBits / 4;
  __shared__ SampleShared sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = blockIdx.x;
  const int vocab = a.vocab;
  const T* x = static_cast<const T*>(a.logits) + (int64_t)row * a.row_stride;
  const int64_t step = a.step != nullptr ? *a.step : 0;
  const uint32_t neg_key = L::key(L::kBits == 16 ? 0xff80u : 0xff800000u);

  // 1. forbidden set
  if (tid == 0) {
    int nf = 0;
    auto add = [&](int64_t id) {
      if (id < 0 || id >= vocab || nf >= kSampleMaxForbidden) return;
      for (int i = 0; i < nf; ++i)
        if (sh.fset[i] == (int32_t)id) return;
      sh.fset[nf++] = (int32_t)id;
    };
    if (a.forbidden != nullptr && step < a.forbid_before_step)
      for (int i = 0; i < a.n_forbidden; ++i) add(a.forbidden[i]);
    if (a.forbidden_by_row != nullptr)
      for (int i = 0; i < a.row_forbidden_count; ++i)
        add(a.forbidden_by_row[(int64_t)row * a.row_forbidden_count + i]);
    sh.nf = nf;
  }
  __syncthreads();
  const int nf = sh.nf;
  for (int i = tid; i < nf; i += kSampleThreads) sh.fkey[i] = L::key(L::load1(x + sh.fset[i]));
  __syncthreads();
  auto forbidden_id = [&](int id) {
    for (int i = 0; i < nf; ++i)
      if (sh.fset[i] == id) return true;
    return false;
  };

  // Eight consecutive ids of a tile (keys; ids past the row are invalid).
  auto tile8 = [&](int i0, uint32_t* bits, bool* ok) {
    if (i0 + 8 <= vocab) {
      L::load8(x + i0, bits);
#pragma unroll
      for (int j = 0; j < 8; ++j) ok[j] = true;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ok[j] = i0 + j < vocab;
        bits[j] = ok[j] ? L::load1(x + i0 + j) : 0u;
      }
    }
  };

  // Every id of the row once, in no particular order, with kSampleUnroll
  // 16-byte loads per thread issued before any is used (a load per
  // iteration would make each sweep one memory round trip per 2048 ids).
  // The loads are unconditional: a chunk past the last whole one re-reads
  // that one and is masked; the (< 8) ids past the last whole chunk are
  // read one by one.
  const int whole = vocab & ~7;
  auto sweep = [&](auto&& f) {
    for (int base = 0; base < whole; base += kSampleTile * kSampleUnroll) {
      uint32_t bits[kSampleUnroll][8];
      int i0[kSampleUnroll];
#pragma unroll
      for (int u = 0; u < kSampleUnroll; ++u) {
        i0[u] = base + (u * kSampleThreads + tid) * 8;
        L::load8(x + min(i0[u], whole - 8), bits[u]);
      }
#pragma unroll
      for (int u = 0; u < kSampleUnroll; ++u) {
        if (i0[u] < whole) {
#pragma unroll
          for (int j = 0; j < 8; ++j) f(i0[u] + j, bits[u][j]);
        }
      }
    }
    for (int i = whole + tid; i < vocab; i += kSampleThreads) f(i, L::load1(x + i));
  };

  const bool full_vocab = !a.greedy && a.top_k == 0;
  const int k = a.greedy ? 1 : min(a.top_k, vocab);

  // Block reductions through LDS (every thread gets the result).
  auto block_max = [&](float v) {
    for (int off = 32; off > 0; off >>= 1) v = vmax(v, __shfl_xor(v, off));
    __syncthreads();
    if (lane == 0) sh.fscan[wave] = v;
    __syncthreads();
    float r = kNegInf;
#pragma unroll
    for (int w = 0; w < kSampleWaves; ++w) r = vmax(r, sh.fscan[w]);
    return r;
  };
  auto block_sum = [&](float v) {
    v = wave_sum_f(v);
    __syncthreads();
    if (lane == 0) sh.fscan[wave] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int w = 0; w < kSampleWaves; ++w) r += sh.fscan[w];
    return r;
  };

  // 2a. maxima of the raw logits and of the sampling logits (a forbidden id
  // is looked up only when its value beats the thread's running maximum)
  float rmax = kNegInf, smax = kNegInf;
  sweep([&](int id, uint32_t bits) {
    const float v = L::to_float(bits);
    rmax = vmax(rmax, v);
    if (v > smax && !(nf > 0 && forbidden_id(id))) smax = v;
  });
  rmax = block_max(rmax);
  smax = block_max(smax);

  // 2b. the raw sum of exp (log-sum-exp of the unmodified logits), and how
  // many sampling logits lie within each window W of their maximum: the
  // smallest window holding k of them holds the whole top k (ties at the
  // k-th value included), so it is gathered and sorted instead of found
  // by radix selection.  W = 0 is the greedy case (the ids at the maximum).
  constexpr int kWin = 16;
  float thr[kWin];
  {
    const float wins[kWin] = {0.f,  0.125f, 0.25f, 0.5f, 0.75f, 1.f,  1.5f,  2.f,
                              3.f,  4.f,    6.f,   8.f,  12.f,  16.f, 32.f,  __builtin_inff()};
#pragma unroll
    for (int i = 0; i < kWin; ++i) thr[i] = smax - wins[i];
  }
  float rsum = 0.f;
  int wc[kWin];
#pragma unroll
  for (int i = 0; i < kWin; ++i) wc[i] = 0;
  sweep([&](int id, uint32_t bits) {
    const float v = L::to_float(bits);
    rsum += fast_exp2((v - rmax) * kLog2e);
#pragma unroll
    for (int i = 0; i < kWin; ++i) wc[i] += v >= thr[i] ? 1 : 0;
  });
  rsum = block_sum(rsum);
#pragma unroll
  for (int i = 0; i < kWin; ++i) wc[i] = wave_sum_i(wc[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < kWin; ++i) sh.ired[0][wave][i] = wc[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kWin; ++i) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < kSampleWaves; ++w) t += sh.ired[0][w][i];
    wc[i] = t;
  }
  __syncthreads();
  // a forbidden id counts at -inf, not at its value
  for (int f = 0; f < nf; ++f) {
    const float vf = L::value(sh.fkey[f]);
#pragma unroll
    for (int i = 0; i < kWin; ++i) wc[i] += (kNegInf >= thr[i] ? 1 : 0) - (vf >= thr[i] ? 1 : 0);
  }
  const float log_z = rmax + logf(rsum);
  // the step's column, clamped into the table the caller passed
  const int64_t col = step < 0 ? 0 : (step >= a.uniform_count ? a.uniform_count - 1 : step);
  const float u = a.uniforms != nullptr ? a.uniforms[(int64_t)row * a.uniform_stride + col] : 0.5f;
  int chosen = 0;

  if (full_vocab) {
    // 4'. every id in id order: p_i = exp(x_i / T - max) / S
    const float inv_t = 1.f / a.temperature;
    const float m = smax / a.temperature;
    float part = 0.f;
    for (int t0 = 0; t0 < vocab; t0 += kSampleTile) {
      const int i0 = t0 + tid * 8;
      if (i0 >= vocab) continue;
      uint32_t bits[8];
      bool ok[8];
      tile8(i0, bits, ok);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (ok[j] && !forbidden_id(i0 + j)) part += expf(L::to_float(bits[j]) / a.temperature - m);
    }
    (void)inv_t;
    part = wave_sum_f(part);
    if (lane == 0) sh.fscan[wave] = part;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kSampleWaves; ++w) total += sh.fscan[w];
    __syncthreads();
    // cumulative probabilities tile by tile until one reaches u
    float base = 0.f;
    int below = 0;
    for (int t0 = 0; t0 < vocab; t0 += kSampleTile) {
      const int i0 = t0 + tid * 8;
      float p[8];
      float loc = 0.f;
      if (i0 < vocab) {
        uint32_t bits[8];
        bool ok[8];
        tile8(i0, bits, ok);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          p[j] = (ok[j] && !forbidden_id(i0 + j))
                     ? expf(L::to_float(bits[j]) / a.temperature - m) / total
                     : 0.f;
          loc += p[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = 0.f;
      }
      const float incl = wave_incl_scan_f(loc, lane);
      if (lane == 63) sh.fscan[wave] = incl;
      __syncthreads();
      float wbase = 0.f, ttot = 0.f;
#pragma unroll
      for (int w = 0; w < kSampleWaves; ++w) {
        wbase += w < wave ? sh.fscan[w] : 0.f;
        ttot += sh.fscan[w];
      }
      __syncthreads();
      float c = base + wbase + incl - loc;
      int cntb = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c += p[j];
        cntb += (i0 + j < vocab && c < u) ? 1 : 0;
      }
      cntb = wave_sum_i(cntb);
      if (lane == 0) sh.iscan[wave] = cntb;
      __syncthreads();
      int tb = 0;
#pragma unroll
      for (int w = 0; w < kSampleWaves; ++w) tb += sh.iscan[w];
      __syncthreads();
      below += tb;
      base += ttot;
      if (tb < min(kSampleTile, vocab - t0)) break;  // u reached inside this tile
    }
    chosen = min(below, vocab - 1);
  } else {
    // 3. the candidates
    int win = -1;
#pragma unroll
    for (int i = kWin - 1; i >= 0; --i)
      if (wc[i] >= k) win = i;
    int n_sort;
    if (win >= 0 && wc[win] <= kSampleGatherCap) {
      // every sampling logit within the smallest window holding k of them
      float t = thr[0];
#pragma unroll
      for (int i = 1; i < kWin; ++i)
        if (i == win) t = thr[i];
      if (tid == 0) sh.ngather = 0;
      __syncthreads();
      sweep([&](int id, uint32_t bits) {
        if (!(L::to_float(bits) >= t)) return;
        uint32_t kk = L::key(bits);
        if (nf > 0 && forbidden_id(id)) {
          if (!(kNegInf >= t)) return;
          kk = neg_key;
        }
        const int slot = atomicAdd(&sh.ngather, 1);
        if (slot < kSampleGatherCap)
          sh.cand[slot] = ((unsigned long long)kk << 32) | (0xffffffffu - (uint32_t)id);
      });
      __syncthreads();
      n_sort = min(sh.ngather, kSampleGatherCap);
    } else {
    // radix selection of the k-th key, four bits per pass
    uint32_t pref = 0;
    int krem = k;
    int n_eq = 0;
    for (int pass = 0; pass < kPasses; ++pass) {
      const int shift = L::kBits - 4 * (pass + 1);
      const uint32_t hi_mask = pass == 0 ? 0u : ((~0u << (shift + 4)) & (L::kBits == 16 ? 0xffffu : ~0u));
      int cnt[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) cnt[j] = 0;
      sweep([&](int id, uint32_t bits) {
        const uint32_t key = L::key(bits);
        if ((key & hi_mask) == pref) {
          const int d = (key >> shift) & 15;
          cnt[0] += 1;
#pragma unroll
          for (int q = 1; q < 16; ++q) cnt[q] += d >= q ? 1 : 0;
        }
      });
      // block totals of the 16 counters
#pragma unroll
      for (int j = 0; j < 16; ++j) cnt[j] = wave_sum_i(cnt[j]);
      if (lane == 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) sh.ired[pass & 1][wave][j] = cnt[j];
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < kSampleWaves; ++w) t += sh.ired[pass & 1][w][j];
        cnt[j] = t;
      }
      // forbidden ids count at the -inf key
      for (int f = 0; f < nf; ++f) {
        const uint32_t rk = sh.fkey[f];
        if (rk == neg_key) continue;
        if ((rk & hi_mask) == pref) {
          const int d = (rk >> shift) & 15;
#pragma unroll
          for (int q = 0; q < 16; ++q) cnt[q] -= d >= q ? 1 : 0;
        }
        if ((neg_key & hi_mask) == pref) {
          const int d = (neg_key >> shift) & 15;
#pragma unroll
          for (int q = 0; q < 16; ++q) cnt[q] += d >= q ? 1 : 0;
        }
      }
      // largest digit whose ids (with this prefix) number at least krem
      // (q = 0 always qualifies: cnt[0] >= krem by construction)
      int dstar = 0, above = 0;
      bool found = false;
#pragma unroll
      for (int q = 15; q >= 0; --q) {
        const int c_next = q == 15 ? 0 : cnt[q + 1];
        if (!found && cnt[q] >= krem) {
          found = true;
          dstar = q;
          above = c_next;
        }
      }
      krem -= above;
      pref |= (uint32_t)dstar << shift;
      n_eq = cnt[dstar] - above;  // ids whose key equals the prefix so far
    }
    // the candidates: every id whose key is at least the k-th key
    const uint32_t tkey = pref;
    const int need = krem;
    const int n_gt = k - need;
    const int n_ge = n_gt + n_eq;
    if (n_ge <= kSampleGatherCap) {
      // all of them, in no order (the sort below puts the lower of equal
      // ids first and keeps the top k)
      if (tid == 0) sh.ngather = 0;
      __syncthreads();
      sweep([&](int id, uint32_t bits) {
        uint32_t kk = L::key(bits);
        if ((kk >= tkey || tkey <= neg_key) && nf > 0 && forbidden_id(id)) kk = neg_key;
        if (kk >= tkey) {
          const int slot = atomicAdd(&sh.ngather, 1);
          if (slot < kSampleGatherCap)
            sh.cand[slot] = ((unsigned long long)kk << 32) | (0xffffffffu - (uint32_t)id);
        }
      });
      __syncthreads();
      n_sort = min(sh.ngather, kSampleGatherCap);
    } else {
      // more ties at the k-th key than fit: take the lowest ids of them,
      // walking the row in id order
      int gt_base = 0, eq_base = 0;
      for (int t0 = 0; t0 < vocab; t0 += kSampleTile) {
        const int i0 = t0 + tid * 8;
        uint32_t key[8];
        bool ok[8];
        int ngt = 0, neq = 0;
        if (i0 < vocab) {
          uint32_t bits[8];
          tile8(i0, bits, ok);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            uint32_t kk = L::key(bits[j]);
            if (ok[j] && (kk >= tkey || tkey <= neg_key) && forbidden_id(i0 + j)) kk = neg_key;
            key[j] = ok[j] ? kk : 0u;
            ngt += (ok[j] && kk > tkey) ? 1 : 0;
            neq += (ok[j] && kk == tkey) ? 1 : 0;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            ok[j] = false;
            key[j] = 0u;
          }
        }
        const int packed = ngt | (neq << 16);
        const int incl = wave_incl_scan_i(packed, lane);
        if (lane == 63) sh.iscan[wave] = incl;
        __syncthreads();
        int wbase = 0, ttot = 0;
#pragma unroll
        for (int w = 0; w < kSampleWaves; ++w) {
          wbase += w < wave ? sh.iscan[w] : 0;
          ttot += sh.iscan[w];
        }
        __syncthreads();
        const int excl = wbase + incl - packed;
        int rg = gt_base + (excl & 0xffff);
        int re = eq_base + (excl >> 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (!ok[j]) continue;
          const unsigned long long ck =
              ((unsigned long long)key[j] << 32) | (0xffffffffu - (uint32_t)(i0 + j));
          if (key[j] > tkey) {
            if (rg < n_gt) sh.cand[rg] = ck;
            ++rg;
          } else if (key[j] == tkey) {
            if (re < need) sh.cand[n_gt + re] = ck;
            ++re;
          }
        }
        gt_base += ttot & 0xffff;
        eq_base += ttot >> 16;
        if (gt_base >= n_gt && eq_base >= need) break;
      }
      n_sort = k;
    }
    }
    // Order the candidates by (value desc, id asc): composite keys are
    // distinct, so an entry's position is the number of entries above it.
    // Up to kSampleRankSort entries: every thread ranks its entries against
    // all of them (broadcast LDS reads, one barrier); more: a bitonic sort.
    if (n_sort <= kSampleRankSort) {
      for (int i = tid; i < n_sort; i += kSampleThreads) {
        const unsigned long long ci = sh.cand[i];
        int r = 0;
        for (int j = 0; j < n_sort; ++j) r += sh.cand[j] > ci ? 1 : 0;
        if (r < k) sh.top[r] = ci;
      }
      __syncthreads();
    } else {
      int kp = 1;
      while (kp < n_sort) kp <<= 1;
      for (int i = n_sort + tid; i < kp; i += kSampleThreads) sh.cand[i] = 0ull;
      __syncthreads();
      for (int size = 2; size <= kp; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          for (int i = tid; i < (kp >> 1); i += kSampleThreads) {
            const int pos = 2 * i - (i & (stride - 1));
            const int oth = pos + stride;
            const bool desc = (pos & size) == 0;
            const unsigned long long p0 = sh.cand[pos], p1 = sh.cand[oth];
            if (desc ? (p0 < p1) : (p0 > p1)) {
              sh.cand[pos] = p1;
              sh.cand[oth] = p0;
            }
          }
          __syncthreads();
        }
      }
      for (int i = tid; i < k; i += kSampleThreads) sh.top[i] = sh.cand[i];
      __syncthreads();
    }

    // 4. softmax, top-p cut, inverse CDF (wavefront 0; lane l owns entries
    // [l * E, l * E + E))
    if (wave == 0 && !a.greedy) {
      constexpr int kMaxE = kSampleMaxTopK / 64;
      const int E = (k + 63) / 64;
      const float m = L::value((uint32_t)(sh.top[0] >> 32)) / a.temperature;
      float e[kMaxE];
      float loc = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxE; ++j) {
        const int i = lane * E + j;
        e[j] = 0.f;
        if (j < E && i < k)
          e[j] = expf(L::value((uint32_t)(sh.top[i] >> 32)) / a.temperature - m);
        loc += e[j];
      }
      const float sum = wave_sum_f(loc);
      if (a.top_p < 1.f) {
        // cumulative probability before each entry; remove where it exceeds top_p
        const float inv = 1.f / sum;
        float pl = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxE; ++j) pl += e[j] / sum;
        (void)inv;
        const float incl = wave_incl_scan_f(pl, lane);
        float c = incl - pl;
#pragma unroll
        for (int j = 0; j < kMaxE; ++j) {
          const int i = lane * E + j;
          const bool remove = i > 0 && c > a.top_p;
          c += e[j] / sum;
          if (remove) e[j] = 0.f;
        }
      }
      float loc2 = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxE; ++j) loc2 += e[j];
      const float sum2 = wave_sum_f(loc2);
      float pl = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxE; ++j) pl += e[j] / sum2;
      const float incl = wave_incl_scan_f(pl, lane);
      float c = incl - pl;
      int below = 0;
#pragma unroll
      for (int j = 0; j < kMaxE; ++j) {
        const int i = lane * E + j;
        c += e[j] / sum2;
        below += (j < E && i < k && c < u) ? 1 : 0;
      }
      below = wave_sum_i(below);
      if (lane == 0) sh.iscan[0] = min(below, k - 1);
    }
    __syncthreads();
    const int pos = a.greedy ? 0 : sh.iscan[0];
    chosen = (int)(0xffffffffu - (uint32_t)(sh.top[pos] & 0xffffffffu));
  }
  if (tid == 0) {
    a.token_out[row] = chosen;
    a.logprob_out[row] = L::to_float(L::load1(x + chosen)) - log_z;
  }
}

// One uniform per (row, step): SplitMix64 of seed + (step + 1) * golden
// ratio, 53 high bits + 0.5 over 2^53, rounded to fp32 (sample.py:12-47).
__global__ void uniforms_kernel(const int64_t* __restrict__ seeds, int32_t rows, int32_t steps,
                                float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)rows * steps) return;
  const int64_t r = i / steps, t = i - r * steps;
  uint64_t v = (uint64_t)seeds[r] + (uint64_t)(t + 1) * 0x9E3779B97F4A7C15ull;
  v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
  v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
  v ^= v >> 31;
  out[i] = (float)(((double)(v >> 11) + 0.5) / 9007199254740992.0);
}

}  // namespace

hipError_t sample_rows(const SampleArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  if (a.elem_bytes == 2)
    sample_kernel<bf16><<<dim3(a.rows), dim3(kSampleThreads), 0, stream>>>(a);
  else
    sample_kernel<float><<<dim3(a.rows), dim3(kSampleThreads), 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t stateless_uniforms(const int64_t* seeds, int32_t rows, int32_t steps, float* out,
                              hipStream_t stream) {
  const int64_t n = (int64_t)rows * steps;
  if (n == 0) return hipSuccess;
  uniforms_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(seeds, rows, steps,
                                                                              out);
  return hipGetLastError();
}

hipError_t greedy_select(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                         int32_t elem_bytes, int64_t* token_out, float* logprob_out,
                         hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (elem_bytes == 2) {
    hipLaunchKernelGGL(greedy_kernel<bf16>, dim3(rows), dim3(kGreedyThreads), 0, stream,
                       static_cast<const bf16*>(logits), row_stride, vocab, token_out,
                       logprob_out);
  } else {
    hipLaunchKernelGGL(greedy_kernel<float>, dim3(rows), dim3(kGreedyThreads), 0, stream,
                       static_cast<const float*>(logits), row_stride, vocab, token_out,
                       logprob_out);
  }
  return hipGetLastError();
}

}  // namespace aios
