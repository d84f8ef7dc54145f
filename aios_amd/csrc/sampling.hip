// Token selection with the raw log-probability of the chosen token:
// greedy_kernel (argmax), and stateless temperature / top-k / top-p sampling
// (python/aios/engine/sample.py:12-160) by sample_resident_kernel (top-k
// over rows of at most 16384 ids, the row held in registers) or
// sample_kernel (longer rows, and every id in id order, streaming the row).
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

constexpr int kGreedyThreads = 1024;  // rows above kGreedyWideFrom ids: 151,936 in ~2.4 round trips
constexpr int kGreedyThreadsNarrow = 256;  // shorter rows: one round trip, fewer wavefronts to merge
constexpr int kGreedyWideFrom = 32768;

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

constexpr int kGreedyUnroll = 8;  // 8-logit chunks per thread in flight (128 KiB per workgroup)

template <typename T, int NT>
__global__ __launch_bounds__(NT) void greedy_kernel(
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
  for (int base = 0; base < whole; base += NT * 8 * kGreedyUnroll) {
    float f[kGreedyUnroll][8];
    int i0[kGreedyUnroll];
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u) {
      i0[u] = base + (u * NT + (int)threadIdx.x) * 8;
      load8f(x + min(i0[u], whole - 8), f[u]);
    }
#pragma unroll
    for (int u = 0; u < kGreedyUnroll; ++u)
      if (i0[u] < whole) {
#pragma unroll
        for (int j = 0; j < 8; ++j) visit(f[u][j], i0[u] + j);
      }
  }
  for (int32_t j = whole + threadIdx.x; j < vocab; j += NT) visit(load_logit(x + j), j);
  for (int off = 32; off > 0; off >>= 1) {
    ArgState o;
    o.m = __shfl_xor(st.m, off);
    o.i = __shfl_xor(st.i, off);
    o.s = __shfl_xor(st.s, off);
    st = merge(st, o);
  }
  __shared__ ArgState waves[NT / 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (lane == 0) waves[wave] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgState r = waves[0];
    for (int w = 1; w < NT / 64; ++w) r = merge(r, waves[w]);
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

// ---------------------------------------------------------------------------
// Row-resident sampling: top_k >= 1 (greedy included) over at most
// kResMaxVocab ids.  One workgroup of NT threads per row (kResThreads); thread
// t keeps the 8-id chunks q = c * NT + t (c < NC) of the row in registers, so
// the row is read once and every later pass runs on registers:
//  1. the forbidden ids set bits of an LDS bitmap (duplicates are harmless),
//     read back as one byte per chunk;
//  2. the raw maximum rmax (block max);
//  3. one pass: the raw sum of exp, the sampling logits s (forbidden ids at
//     -inf) and each id's code c = min((bits(rmax - s) >> 19) - (118 << 4)
//     clamped at 0, 254): the float bits of a distance keep its order, so c
//     grows with the distance below rmax (c >> 4: its binary octave from
//     2^-9 to 2^7, c & 15: a sixteenth of that octave; 0 and 254 also take
//     everything nearer and farther, -inf included; 255 marks the ids past
//     the row).  A count of c >> 4 over 16 buckets (4-bit counters packed in
//     one 64-bit register per chunk, at most 8 per counter), reduced with the
//     sum of exp, finds the octave holding the k-th largest; when the ids up
//     to that octave far outnumber k, a second count of c & 15 inside it
//     narrows the bound to a sixteenth of an octave.  The ids with a code at
//     or below the bound are an upper set of the sampling logits with at
//     least k members, so they hold the top k;
//  4. those candidates are written to LDS as composite keys (value key above
//     ~id: distinct, larger = higher value, then lower id) at positions from
//     per-slot ballots, and ordered: up to kResRankMax of them by rank
//     counting (several threads per candidate, each over a contiguous run),
//     more by a bitonic sort;
//  5. more than kResCap candidates (ids tied at the bound): the k-th value
//     key, and the id cut among its ties when those overflow too, are found
//     by bisection with block counts, and exactly the top k are gathered;
//  6. wavefront 0: softmax of value / temperature over the top k, the top-p
//     cut and the inverse CDF with the formulas of sample_kernel (lane l owns
//     entries [l * E, l * E + E), their exponentials kept in LDS; DPP lane
//     sums and scans).
// Measured on MI355X (24 rows, bf16, top_k 50): 12.3 us per launch at 16384
// ids and 9.6 us at 6400, against 40-48 us for sample_kernel's three sweeps.
constexpr int kResMaxVocab = 16384;  // ids per row at most
constexpr int kResCap = 2048;     // candidates gathered and ordered at most
constexpr int kResRankMax = 256;  // candidates ordered by rank counting at most
static_assert(kResCap >= kSampleMaxTopK, "the exact top k fits the candidate buffer");

template <typename T>
struct ResKeyOf;
template <>
struct ResKeyOf<bf16> {
  using Key = uint32_t;  // value key << 16 | (0xffff - id)
  static constexpr int kIdBits = 16;
};
template <>
struct ResKeyOf<float> {
  using Key = unsigned long long;  // value key << 32 | (0xffffffff - id)
  static constexpr int kIdBits = 32;
};
static_assert(kResMaxVocab <= (1 << 16), "ids fit the 16-bit field of the bf16 keys");

template <typename Key, int NW>
struct ResShared {
  uint32_t fbits[kResMaxVocab / 32];   // forbidden ids, one bit each
  alignas(16) uint32_t red[2][NW][8];  // per-wavefront packed counts
  float fred[2][NW][2];                // per-wavefront max / sum
  uint32_t ired[2][NW];                // per-wavefront counts (bisection)
  uint32_t gscan[NW];                  // per-wavefront candidate counts
  alignas(16) Key cand[kResCap];
  Key top[kSampleMaxTopK];
  float ev[kSampleMaxTopK];  // exp of the top k (wavefront 0)
  int pos;
};

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sums / maxima over the 64 lanes (every lane receives the result): DPP
// inside each 16-lane row, then the gfx950 row and half swaps.
__device__ __forceinline__ uint32_t lanes_sum_u(uint32_t x) {
  x += dpp_u<0xB1>(x);
  x += dpp_u<0x4E>(x);
  x += dpp_u<0x141>(x);
  x += dpp_u<0x140>(x);
  auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = r[0] + r[1];
  r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return r[0] + r[1];
}
__device__ __forceinline__ float lanes_max_f(float x) {
  x = vmax(x, dpp_f<0xB1>(x));
  x = vmax(x, dpp_f<0x4E>(x));
  x = vmax(x, dpp_f<0x141>(x));
  x = vmax(x, dpp_f<0x140>(x));
  return xrow_max(x);
}
__device__ __forceinline__ float lanes_sum_f(float x) { return xrow_sum(row16_sum(x)); }

// Inclusive prefix sums over the lanes: Hillis-Steele inside each 16-lane
// row (row_shr 1, 2, 4, 8; lanes without a source add 0), then row 0's total
// into row 1 and row 2's into row 3 (row_bcast:15), then the total of rows
// 0-1 into rows 2-3 (row_bcast:31).
__device__ __forceinline__ uint32_t lanes_scan_u(uint32_t x) {
  x += dpp_u<0x111>(x);
  x += dpp_u<0x112>(x);
  x += dpp_u<0x114>(x);
  x += dpp_u<0x118>(x);
  x += dpp_u<0x142, 0xA>(x);
  x += dpp_u<0x143, 0xC>(x);
  return x;
}
__device__ __forceinline__ float lanes_scan_f(float x) {
  x += dpp_f<0x111>(x);
  x += dpp_f<0x112>(x);
  x += dpp_f<0x114>(x);
  x += dpp_f<0x118>(x);
  x += dpp_f<0x142, 0xA>(x);
  x += dpp_f<0x143, 0xC>(x);
  return x;
}

// Eight consecutive logits of a row as fp32; ids at or past vocab read -inf
// (a partial last chunk is read one id at a time).
__device__ __forceinline__ void res_load8(const bf16* x, int i0, int vocab, float (&f)[8]) {
  if (i0 + 8 <= vocab) {
    const uint4 r = *reinterpret_cast<const uint4*>(x + i0);
    f[0] = lo_bf16(r.x); f[1] = hi_bf16(r.x); f[2] = lo_bf16(r.y); f[3] = hi_bf16(r.y);
    f[4] = lo_bf16(r.z); f[5] = hi_bf16(r.z); f[6] = lo_bf16(r.w); f[7] = hi_bf16(r.w);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      f[j] = i0 + j < vocab ? bf16_bits_to_float(__builtin_bit_cast(uint16_t, x[i0 + j])) : kNegInf;
  }
}
__device__ __forceinline__ void res_load8(const float* x, int i0, int vocab, float (&f)[8]) {
  if (i0 + 8 <= vocab) {
    const float4 a = *reinterpret_cast<const float4*>(x + i0);
    const float4 b = *reinterpret_cast<const float4*>(x + i0 + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = i0 + j < vocab ? x[i0 + j] : kNegInf;
  }
}

// Value key (LogitTraits::key) of an fp32 copy of a logit.
__device__ __forceinline__ uint32_t res_vkey(float v, bf16*) {
  return LogitTraits<bf16>::key(__float_as_uint(v) >> 16);
}
__device__ __forceinline__ uint32_t res_vkey(float v, float*) {
  return LogitTraits<float>::key(__float_as_uint(v));
}

// Block totals of 16 counters held as 4-bit fields of one 64-bit register
// per chunk (at most 8 per field): the fields are spread to bytes (at most
// 8 * NC), then to 16-bit halves (bucket pairs (b, b + 4) per word), summed
// over the lanes and across the wavefronts.  Every thread receives them.
// A float partial (fsum, with its per-wavefront slots fred) is summed in the
// same pass when fred is given; returns its block total.
template <int NC, int NW>
__device__ __forceinline__ float res_block_counts(const uint64_t (&acc)[NC], uint32_t (*red)[8],
                                                  float (*fred)[2], float fsum, int lane, int wave,
                                                  int (&tot)[16]) {
  uint32_t bl[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t lo = (uint32_t)acc[c], hi = (uint32_t)(acc[c] >> 32);
    bl[0] += lo & 0x0f0f0f0fu;         // byte b: bucket 2b
    bl[1] += (lo >> 4) & 0x0f0f0f0fu;  // bucket 2b + 1
    bl[2] += hi & 0x0f0f0f0fu;         // bucket 8 + 2b
    bl[3] += (hi >> 4) & 0x0f0f0f0fu;  // bucket 9 + 2b
  }
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[2 * i] = bl[i] & 0x00ff00ffu;             // bytes 0, 2
    w[2 * i + 1] = (bl[i] >> 8) & 0x00ff00ffu;  // bytes 1, 3
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = lanes_sum_u(w[i]);
  if (fred != nullptr) fsum = lanes_sum_f(fsum);
  if (lane == 0) {
    reinterpret_cast<uint4*>(red[wave])[0] = make_uint4(w[0], w[1], w[2], w[3]);
    reinterpret_cast<uint4*>(red[wave])[1] = make_uint4(w[4], w[5], w[6], w[7]);
    if (fred != nullptr) fred[wave][0] = fsum;
  }
  __syncthreads();
  float ftot = 0.f;
  if (fred != nullptr)
#pragma unroll
    for (int v = 0; v < NW; ++v) ftot += fred[v][0];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = 0u;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    const uint4 p = reinterpret_cast<const uint4*>(red[v])[0];
    const uint4 q = reinterpret_cast<const uint4*>(red[v])[1];
    w[0] += p.x; w[1] += p.y; w[2] += p.z; w[3] += p.w;
    w[4] += q.x; w[5] += q.y; w[6] += q.z; w[7] += q.w;
  }
  // w[2i + h] holds bytes h and h + 2 of bl[i]: bl[0] byte b = bucket 2b,
  // bl[1] byte b = 2b + 1, bl[2] byte b = 8 + 2b, bl[3] byte b = 9 + 2b.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int base = (i & 1) + (i >> 1) * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      tot[base + 2 * h] = (int)(w[2 * i + h] & 0xffffu);
      tot[base + 2 * h + 4] = (int)(w[2 * i + h] >> 16);
    }
  }
  return ftot;
}

template <typename T, int NT, int NC>
__global__ __launch_bounds__(NT) void sample_resident_kernel(SampleArgs a) {
  constexpr int NW = NT / 64;
  static_assert(NT * 8 * NC <= kResMaxVocab && kSampleMaxForbidden <= NT, "row and lists fit");
  static_assert(NC * 8 <= 32, "a thread's ids index 32-bit masks");
  using L = LogitTraits<T>;
  using Key = typename ResKeyOf<T>::Key;
  constexpr int kIdBits = ResKeyOf<T>::kIdBits;
  constexpr Key kIdMask = (Key)((1ull << kIdBits) - 1);
  __shared__ ResShared<Key, NW> sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = blockIdx.x;
  const int vocab = a.vocab;
  const T* x = static_cast<const T*>(a.logits) + (int64_t)row * a.row_stride;
  const uint32_t neg_key = L::key(L::kBits == 16 ? 0xff80u : 0xff800000u);

  // The row (chunk c of this thread: ids 8 (c * NT + tid) + j).
  float v[NC][8];
  uint32_t valid = 0;  // bit 8c + j: id inside the row
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int i0 = (c * NT + tid) * 8;
    res_load8(x, i0, vocab, v[c]);
    const int nv = min(max(vocab - i0, 0), 8);
    valid |= ((1u << nv) - 1u) << (8 * c);
  }
  const int64_t step = a.step != nullptr ? *a.step : 0;
  // this thread's forbidden id (if any): the global list while
  // step < forbid_before_step, then row r's list
  int fid = -1;
  if (tid < a.n_forbidden) {
    const int32_t f = a.forbidden[tid];
    fid = (step < a.forbid_before_step && f >= 0 && f < vocab) ? f : -1;
  } else if (tid < a.n_forbidden + a.row_forbidden_count) {
    const int64_t f = a.forbidden_by_row[(int64_t)row * a.row_forbidden_count + tid - a.n_forbidden];
    fid = (f >= 0 && f < vocab) ? (int)f : -1;
  }
  const int64_t col = step < 0 ? 0 : (step >= a.uniform_count ? a.uniform_count - 1 : step);
  const float u = a.uniforms != nullptr ? a.uniforms[(int64_t)row * a.uniform_stride + col] : 0.5f;

  // 1. forbidden bitmap
  for (int i = tid; i < (vocab + 31) / 32; i += NT) sh.fbits[i] = 0u;
  __syncthreads();
  if (fid >= 0) atomicOr(&sh.fbits[fid >> 5], 1u << (fid & 31));

  // 2. raw maximum (its barrier also publishes the bitmap)
  float rm = kNegInf;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) rm = vmax(rm, v[c][j]);
  rm = lanes_max_f(rm);
  if (lane == 0) sh.fred[0][wave][0] = rm;
  __syncthreads();
  float rmax = kNegInf;
#pragma unroll
  for (int w = 0; w < NW; ++w) rmax = vmax(rmax, sh.fred[0][w][0]);

  // raw sum of exp; sampling logits (forbidden ids at -inf); each id's code
  // (the distance to rmax: an upper bound of the sampling logits, so codes
  // still grow as sampling logits fall) and the octave count.  Ids past the
  // row read -inf (code 255) and are taken out of bucket 15 afterwards.
  const float mu = rmax == kNegInf ? 0.f : rmax * kLog2e;
  float rs = 0.f;
  uint32_t code[NC][2];  // four 8-bit codes per word
  uint64_t acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int q = c * NT + tid;
    const uint32_t fb = q * 8 < vocab ? reinterpret_cast<const uint8_t*>(sh.fbits)[q] : 0u;
    code[c][0] = code[c][1] = 0u;
    acc[c] = 0ull;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      rs += fast_exp2(v[c][j] * kLog2e - mu);
      if ((fb >> j) & 1u) v[c][j] = kNegInf;
      const float d = rmax - v[c][j];  // +0 at the maximum; inf or NaN at -inf
      const uint32_t eb = __float_as_uint(d) >> 19;
      const uint32_t cb = min(eb - min(eb, 118u << 4), 254u);
      code[c][j >> 2] |= cb << (8 * (j & 3));
      acc[c] += 1ull << ((cb >> 4) * 4);
    }
    // ids past the row: code 255 (counted in bucket 15, taken out below)
    const int nv = min(max(vocab - q * 8, 0), 8);
    if (nv < 8) {
      code[c][0] |= nv >= 4 ? 0u : 0xffffffffu << (8 * nv);
      code[c][1] |= nv <= 4 ? 0xffffffffu : 0xffffffffu << (8 * (nv - 4));
    }
  }
  int tot[16];
  const float rsum = res_block_counts<NC, NW>(acc, sh.red[0], sh.fred[1], rs, lane, wave, tot);
  const int n_pad_ids = NC * NT * 8 - vocab;  // ids past the row, all in bucket 15
  tot[15] -= n_pad_ids;
  const float log_z = rmax + logf(rsum);
  const int k = min(a.top_k, vocab);
  int oct = 15, below = 0;
  {
    int cum = 0;
    bool found = false;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      if (!found && cum + tot[b] >= k) {
        found = true;
        oct = b;
        below = cum;
      }
      cum += tot[b];
    }
  }
  // (code 255 marks ids past the row: the bound stays below it)
  int bound = min(oct * 16 + 15, 254);
  int n = below + tot[oct];
  // the sixteenths of that octave when it holds many more than k
  if (n > 192 && n > k + (k >> 2)) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      acc[c] = 0ull;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t cb = (code[c][j >> 2] >> (8 * (j & 3))) & 0xffu;
        acc[c] += (uint64_t)((cb >> 4) == (uint32_t)oct ? 1u : 0u) << ((cb & 15u) * 4);
      }
    }
    res_block_counts<NC, NW>(acc, sh.red[1], nullptr, 0.f, lane, wave, tot);
    if (oct == 15) tot[15] -= n_pad_ids;
    int cum = below;
    bool found = false;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      if (!found && cum + tot[s] >= k) {
        found = true;
        bound = oct * 16 + s;
        n = cum + tot[s];
      }
      cum += tot[s];
    }
  }

  auto id_of = [&](int c, int j) { return (c * NT + tid) * 8 + j; };
  auto ckey = [&](int c, int j) {
    return ((Key)res_vkey(v[c][j], (T*)nullptr) << kIdBits) | (kIdMask - (Key)id_of(c, j));
  };
  // Writes the ids for which pred(c, j) holds to sh.cand (wavefront by
  // wavefront, id slot by id slot: one ballot per slot, positions from the
  // wavefront totals and mbcnt) and zero keys after them up to the next
  // power of two; returns how many.
  auto gather = [&](auto&& pred) -> int {
    uint32_t wcnt = 0u;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) wcnt += __popcll(__ballot(pred(c, j)));
    if (lane == 0) sh.gscan[wave] = wcnt;
    __syncthreads();
    uint32_t pos = 0u, total = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t t = sh.gscan[w];
      pos += w < wave ? t : 0u;
      total += t;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool pr = pred(c, j);
        const uint64_t mk = __ballot(pr);
        if (mk != 0ull) {
          const uint32_t at = pos + __builtin_amdgcn_mbcnt_hi(
                                        (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
          if (pr && at < (uint32_t)kResCap) sh.cand[at] = ckey(c, j);
          pos += __popcll(mk);
        }
      }
    const int cnt = (int)min(total, (uint32_t)kResCap);
    int npad = 1;
    while (npad < cnt) npad <<= 1;
    for (int i = cnt + tid; i < npad; i += NT) sh.cand[i] = 0;
    __syncthreads();
    return cnt;
  };

  auto in_row = [&](int c, int j) { return ((valid >> (8 * c + j)) & 1u) != 0u; };
  if (n <= kResCap) {
    n = gather([&](int c, int j) {
      return (int)((code[c][j >> 2] >> (8 * (j & 3))) & 0xffu) <= bound;
    });
  } else {
    // 5. ties at the bound overflow the buffer: bisection with block counts
    int parity = 0;
    auto count = [&](auto&& pred) -> int {
      uint32_t cnt = 0u;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          cnt += (((valid >> (8 * c + j)) & 1u) && pred(c, j)) ? 1u : 0u;
      cnt = lanes_sum_u(cnt);
      if (lane == 0) sh.ired[parity][wave] = cnt;
      __syncthreads();
      uint32_t t = 0u;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += sh.ired[parity][w];
      parity ^= 1;
      return (int)t;
    };
    // the k-th largest value key: the largest t with count(key >= t) >= k
    uint32_t lo = 0u, hi = L::kBits == 16 ? 0xffffu : 0xffffffffu;
    int n_ge = vocab;
    while (lo < hi) {
      const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) >> 1);
      const int cm = count([&](int c, int j) { return res_vkey(v[c][j], (T*)nullptr) >= mid; });
      if (cm >= k) {
        lo = mid;
        n_ge = cm;
      } else {
        hi = mid - 1;
      }
    }
    const uint32_t tkey = lo;
    if (n_ge <= kResCap) {
      n = gather([&](int c, int j) { return in_row(c, j) && res_vkey(v[c][j], (T*)nullptr) >= tkey; });
    } else {
      // the lowest ids of the ties: the smallest m with
      // count(key == tkey, id <= m) >= k - count(key > tkey)
      const int need = k - count([&](int c, int j) { return res_vkey(v[c][j], (T*)nullptr) > tkey; });
      int ilo = 0, ihi = vocab - 1;
      while (ilo < ihi) {
        const int mid = (ilo + ihi) >> 1;
        const int cm = count([&](int c, int j) {
          return res_vkey(v[c][j], (T*)nullptr) == tkey && id_of(c, j) <= mid;
        });
        if (cm >= need) ihi = mid;
        else ilo = mid + 1;
      }
      n = gather([&](int c, int j) {
        const uint32_t kk = res_vkey(v[c][j], (T*)nullptr);
        return in_row(c, j) && (kk > tkey || (kk == tkey && id_of(c, j) <= ilo));
      });
    }
  }

  // 4. order the candidates; the first k go to sh.top
  // (the gather left zero keys, below every real key, up to npad)
  int npad = 1;
  while (npad < n) npad <<= 1;
  if (n <= kResRankMax) {
    // tpe threads per candidate, each counting the larger keys in its own
    // contiguous run of L entries
    const int tpe = min(min(64, NT / npad), npad);
    const int L = npad / tpe;
    const int e = tid / tpe;
    const int p = tid - e * tpe;
    int r = 0;
    Key ce = 0;
    if (e < n) {
      ce = sh.cand[e];
      const Key* run = sh.cand + p * L;
      constexpr int KV = 16 / sizeof(Key);  // keys per 16-byte read
      if (L % KV == 0) {
        for (int j = 0; j < L; j += KV) {
          const uint4 q = *reinterpret_cast<const uint4*>(run + j);
          if constexpr (KV == 4) {
            r += (q.x > ce ? 1 : 0) + (q.y > ce ? 1 : 0) + (q.z > ce ? 1 : 0) + (q.w > ce ? 1 : 0);
          } else {
            r += ((((Key)q.y << 32) | q.x) > ce ? 1 : 0) + ((((Key)q.w << 32) | q.z) > ce ? 1 : 0);
          }
        }
      } else {
        for (int j = 0; j < L; ++j) r += run[j] > ce ? 1 : 0;
      }
    }
    for (int off = 1; off < tpe; off <<= 1) r += __shfl_xor(r, off);
    if (e < n && p == 0 && r < k) sh.top[r] = ce;
    __syncthreads();
  } else {
    for (int size = 2; size <= npad; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < (npad >> 1); i += NT) {
          const int pos = 2 * i - (i & (stride - 1));
          const int oth = pos + stride;
          const bool desc = (pos & size) == 0;
          const Key p0 = sh.cand[pos], p1 = sh.cand[oth];
          if (desc ? (p0 < p1) : (p0 > p1)) {
            sh.cand[pos] = p1;
            sh.cand[oth] = p0;
          }
        }
        __syncthreads();
      }
    }
    for (int i = tid; i < k; i += NT) sh.top[i] = sh.cand[i];
    __syncthreads();
  }

  // 6. softmax, top-p cut, inverse CDF (wavefront 0; lane l owns entries
  // [l * E, l * E + E))
  auto value_of = [&](Key ck) { return L::value((uint32_t)(ck >> kIdBits)); };
  if (wave == 0 && !a.greedy) {
    const int E = (k + 63) / 64;
    const int i0 = lane * E;
    const int i1 = min(i0 + E, k);
    const float m = value_of(sh.top[0]) / a.temperature;
    float loc = 0.f;
    for (int i = i0; i < i1; ++i) {
      const float ei = expf(value_of(sh.top[i]) / a.temperature - m);
      sh.ev[i] = ei;
      loc += ei;
    }
    const float sum = lanes_sum_f(loc);
    float sum2 = sum;
    if (a.top_p < 1.f) {
      // cumulative probability before each entry; remove where it exceeds top_p
      float pl = 0.f;
      for (int i = i0; i < i1; ++i) pl += sh.ev[i] / sum;
      float c = lanes_scan_f(pl) - pl;
      float loc2 = 0.f;
      for (int i = i0; i < i1; ++i) {
        const float ei = sh.ev[i];
        const bool remove = i > 0 && c > a.top_p;
        c += ei / sum;
        if (remove) sh.ev[i] = 0.f;
        else loc2 += ei;
      }
      sum2 = lanes_sum_f(loc2);
    }
    float pl = 0.f;
    for (int i = i0; i < i1; ++i) pl += sh.ev[i] / sum2;
    float c = lanes_scan_f(pl) - pl;
    uint32_t nb = 0u;
    for (int i = i0; i < i1; ++i) {
      c += sh.ev[i] / sum2;
      nb += c < u ? 1u : 0u;
    }
    nb = lanes_sum_u(nb);
    if (lane == 0) sh.pos = min((int)nb, k - 1);
  }
  __syncthreads();
  if (tid == 0) {
    const Key ck = sh.top[a.greedy ? 0 : sh.pos];
    const int chosen = (int)(kIdMask - (ck & kIdMask));
    const uint32_t vk = (uint32_t)(ck >> kIdBits);
    // a forbidden (or -inf) id carries the -inf key: its raw logit is read
    const float raw = vk == neg_key ? L::to_float(L::load1(x + chosen)) : L::value(vk);
    a.token_out[row] = chosen;
    a.logprob_out[row] = raw - log_z;
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

constexpr int kResThreads = 512;  // threads per row of the row-resident kernel

template <typename T>
static void launch_resident(const SampleArgs& a, hipStream_t stream) {
  constexpr int NT = kResThreads;
  const dim3 grid(a.rows), block(NT);
  if (a.vocab <= NT * 8)
    sample_resident_kernel<T, NT, 1><<<grid, block, 0, stream>>>(a);
  else if (a.vocab <= NT * 16)
    sample_resident_kernel<T, NT, 2><<<grid, block, 0, stream>>>(a);
  else
    sample_resident_kernel<T, NT, kResMaxVocab / (NT * 8)><<<grid, block, 0, stream>>>(a);
}

hipError_t sample_rows(const SampleArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  // top-k (greedy included) over a row that fits the registers of one
  // workgroup: the row-resident kernel; every id in id order (top_k 0) and
  // longer rows: the streaming kernel
  if (a.top_k >= 1 && a.vocab <= kResMaxVocab) {
    if (a.elem_bytes == 2)
      launch_resident<bf16>(a, stream);
    else
      launch_resident<float>(a, stream);
    return hipGetLastError();
  }
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
  const bool wide = vocab > kGreedyWideFrom;
  if (elem_bytes == 2) {
    const bf16* x = static_cast<const bf16*>(logits);
    if (wide)
      hipLaunchKernelGGL((greedy_kernel<bf16, kGreedyThreads>), dim3(rows), dim3(kGreedyThreads),
                         0, stream, x, row_stride, vocab, token_out, logprob_out);
    else
      hipLaunchKernelGGL((greedy_kernel<bf16, kGreedyThreadsNarrow>), dim3(rows),
                         dim3(kGreedyThreadsNarrow), 0, stream, x, row_stride, vocab, token_out,
                         logprob_out);
  } else {
    const float* x = static_cast<const float*>(logits);
    if (wide)
      hipLaunchKernelGGL((greedy_kernel<float, kGreedyThreads>), dim3(rows), dim3(kGreedyThreads),
                         0, stream, x, row_stride, vocab, token_out, logprob_out);
    else
      hipLaunchKernelGGL((greedy_kernel<float, kGreedyThreadsNarrow>), dim3(rows),
                         dim3(kGreedyThreadsNarrow), 0, stream, x, row_stride, vocab, token_out,
                         logprob_out);
  }
  return hipGetLastError();
}

}  // namespace aios
