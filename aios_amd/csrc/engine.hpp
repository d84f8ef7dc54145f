// MFMA attention tile engines for gfx950, shared by the shared-prefix cascade
// decode (kernel (c)), the varlen causal prefill (kernel (b)) and the
// per-row suffix items (kernel (d)).
//
// A 256-thread workgroup (4 wavefronts) owns one kv-head, one KV position
// range and up to 128 query rows (32 per wavefront).  A query row is any
// (token or candidate, q-head) pair of the GQA group, so all query heads
// sharing a kv-head share one K/V stream.
//
// Data movement (stream_kv): the range's page ids are staged in LDS, then
// K/V rows are gathered page by page straight from HBM into an LDS ring of
// four 32-token sub-tiles with raw-buffer LDS loads (buffer_load_dwordx4
// ... lds, no VGPR staging), two sub-tiles ahead of the one being consumed
// (three measured no faster).  Rows are stored token-major with the
// sixteen-byte chunks of each row rotated by a multiple of the token index
// (chosen per head size and engine, see KVTile) so that the MFMA operand
// reads avoid LDS bank conflicts.  Masked or out-of-range positions load a
// zero row.
//
// Math per 32-token sub-tile and wavefront (TileEngine32, the ring path):
//   S^T = K Q^T         v_mfma_f32_32x32x16_bf16, A = K rows (ds_read_b128),
//                       B = Q fragments kept in registers
//   online softmax      one query row per lane pair (l, l ^ 32); row max of
//                       16 scores in the lane plus v_permlane32_swap; log2
//                       domain; the reference max moves only when a row's max
//                       grows by more than 2^8, so O is rarely rescaled
//   O^T += V^T P^T      A = V^T read with ds_read_b64_tr_b16 (the LDS
//                       transpose read) from the token-major V rows, B = P^T,
//                       the fragment each lane holds after the S^T step
// TileEngine is the same math with 16 x 16 x 32 MFMA tiles, used with one
// 16-row tile by the suffix items (G <= 16 live rows).
// This is the offset-causal GQA softmax attention of
// python/aios/attention/flashinfer.py:33-91 (decode: q_len 1).
#pragma once

#include <type_traits>
#include <utility>

#include "kernels.hpp"

#define AIOS_LDS __attribute__((address_space(3)))

namespace aios {

constexpr int kSubTok = 32;       // KV positions per sub-tile
constexpr int kRing = 4;          // sub-tiles in the LDS ring
constexpr int kLookahead = 2;     // sub-tiles in flight ahead of the one consumed (< kRing)
static_assert(kLookahead < kRing, "the slot being consumed is never refilled");
constexpr int kIdWindow = 1024;   // page ids staged in LDS at a time
constexpr int kEngineThreads = 256;
// The softmax reference may lag a row's running max by up to 2^8.
constexpr float kRescaleSlack = 8.0f;

// Source of every masked / out-of-range K or V chunk of the suffix gathers.
static __device__ __align__(16) uint8_t g_zero_kv_row[512] = {0};

// Word 3 of a raw buffer descriptor on gfx9-family GPUs (32-bit data format).
constexpr int kBufferWord3 = 0x00020000;
// Cache policy of a buffer load: NT, the non-temporal (streaming) hint.
// The shared-prefix gathers of a decode read each prefix KV row once per
// launch; marked streaming they leave the caches to what the next launch
// reads again (page ids, query rows, partial states).  The per-row suffix
// gathers keep the default policy (a CandidateGroup step re-reads its
// rows' short KV every step, and measured slower streamed), and so does
// the prefill (the query tiles of one kv-head re-read its K/V from L2).
constexpr int kCpolStream = 2;

// s_waitcnt with vmcnt <= N and the other counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}

// Every LDS access this thread issued has completed; then a workgroup
// barrier.  Plain s_barrier (no fence): the asynchronous LDS loads are
// waited for explicitly with wait_vmcnt.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (LDS transpose read) as inline asm.  The compiler
// treats the builtin's read as possibly aliasing any LDS DMA in flight and
// waits for all of them (vmcnt(0)) before it, which would stall every
// sub-tile on the DMAs just issued for later ring slots; the ring protocol
// (explicit vmcnt waits, then a barrier) already orders each sub-tile's DMA
// before its reads.  The compiler does not count the asm read in lgkmcnt:
// lds_wait_tied waits for it with the results as operands, so no use of them
// can be scheduled above the wait.
__device__ __forceinline__ bf16x4 lds_read_tr(const uint8_t* p) {
  const uint32_t addr = (uint32_t)(uintptr_t)(AIOS_LDS const uint8_t*)p;
  uint64_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return __builtin_bit_cast(bf16x4, r);
}
// The same read at a compile-time byte offset from a 32-bit LDS address
// (the instruction's 16-bit offset field, so no address add per read).
template <uint32_t OFF>
__device__ __forceinline__ bf16x4 lds_read_tr_at(uint32_t addr) {
  static_assert(OFF < 65536, "ds offset field");
  uint64_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return __builtin_bit_cast(bf16x4, r);
}
__device__ __forceinline__ void lds_wait_tied(bf16x4& a, bf16x4& b) {
  uint64_t x = __builtin_bit_cast(uint64_t, a), y = __builtin_bit_cast(uint64_t, b);
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x), "+v"(y));
  a = __builtin_bit_cast(bf16x4, x);
  b = __builtin_bit_cast(bf16x4, y);
}

// W32: the layout read by TileEngine32 (32 x 32 MFMA tiles); otherwise the
// one read by TileEngine (16 x 16 tiles).  The gathers write either.
template <int D, bool W32 = false>
struct KVTile {
  static constexpr int ROWB = 2 * D;                 // bytes of one K or V row
  static constexpr int CPR = D / 8;                  // 16-byte chunks per row
  static constexpr int SUB_KB = kSubTok * ROWB;      // K bytes per sub-tile
  static constexpr int SUB_BYTES = 2 * SUB_KB;       // K then V
  static constexpr int LPS = SUB_BYTES / (kEngineThreads * 16);  // loads / thread / sub-tile
  static constexpr int RING_BYTES = kRing * SUB_BYTES;
  static constexpr int LDS_BYTES = RING_BYTES + kIdWindow * 4;
  static_assert(SUB_BYTES % (kEngineThreads * 16) == 0, "sub-tile must split evenly");

  // Chunk c of token t's row sits in slot (c + rot(t)) % CPR of the row.
  // The rotations were chosen by measuring LDS read rates on gfx950 (four
  // wavefronts, the exact lane patterns of the reads below): K (read with
  // ds_read_b128) conflict-free for D = 64 and 128 and at the best measured
  // rate for D = 96; V (read with ds_read_b64_tr_b16) conflict-free.
  // W32 (derived for 64 banks of 4 bytes, a 16-lane quarter of a
  // ds_read_b128 and a 32-lane half of a ds_read_b64_tr_b16 conflict-free):
  // K lanes t = 0..15 of one chunk column hit 16 distinct 16-byte bank
  // groups (D = 128: rotation t; D = 96: t / 4 against the 48-dword row
  // pitch; D = 64: t / 2 with two rows per bank period); V: the 4 tokens x 4
  // chunks of a half-read land in distinct groups (D = 128: 4t; D = 64:
  // 4 (t / 2); D = 96: none needed), and token t + 8 keeps token t's slot.
  static __device__ __forceinline__ int k_rot(int t) {
    if constexpr (W32) return D == 128 ? t : D == 96 ? t >> 2 : t >> 1;
    else return D == 128 ? 2 * t : D == 96 ? t >> 1 : t;
  }
  static __device__ __forceinline__ int v_rot(int t) {
    if constexpr (W32) return D == 128 ? 4 * t : D == 96 ? 0 : 4 * (t >> 1);
    else return D == 128 ? t : 2 * t;
  }
  static __device__ __forceinline__ int k_slot(int t, int c) { return (c + k_rot(t)) % CPR; }
  static __device__ __forceinline__ int v_slot(int t, int c) { return (c + v_rot(t)) % CPR; }
  // Inverses: which chunk a slot holds.
  static __device__ __forceinline__ int k_chunk(int t, int slot) {
    return (slot + CPR - k_rot(t) % CPR) % CPR;
  }
  static __device__ __forceinline__ int v_chunk(int t, int slot) {
    return (slot + CPR - v_rot(t) % CPR) % CPR;
  }
};

// Per-head RMSNorm + rotate-half RoPE of a query or key row on its way into
// the engines (q_norm / k_norm and the rotary embedding of
// python/aios/models/qwen3.py:52-67, with the roundings of
// qk_norm_rope_kernel): xn = bf16(x * rsqrt(mean(x^2) + eps) * w), then
// y = bf16(bf16(xn * c) + bf16(r * s)) with c, s the cos / sin table entries
// of the row's position rounded to bf16 (the tables come in bf16, so rounded
// already) and r = -xn[i + D/2] in the first half of the head, xn[i - D/2]
// in the second.

// xn = bf16(x * inv * w) over 8 dims (w: their 8 norm weights).
__device__ __forceinline__ void qk_norm8(float (&x)[8], float inv, const bf16x8& w) {
  float wf[8];
  unpack_bf16x8(w, wf);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = round_bf16(x[i] * inv * wf[i]);
}

// The rotation of 8 dims: xn, their partners p (xn at i + D/2 or i - D/2),
// first = the dims lie in the first half; c / s their table entries.
__device__ __forceinline__ bf16x8 qk_rope8(const float (&xn)[8], const float (&p)[8], bool first,
                                           const bf16x8& cb, const bf16x8& sb) {
  float c[8], s[8], y[8];
  unpack_bf16x8(cb, c);
  unpack_bf16x8(sb, s);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float r = first ? -p[i] : p[i];
    y[i] = round_bf16(round_bf16(xn[i] * c[i]) + round_bf16(r * s[i]));
  }
  return pack_bf16x8(y);
}
__device__ __forceinline__ bf16x8 qk_rope8(const float (&xn)[8], const float (&p)[8], bool first,
                                           const bf16* cr, const bf16* sr) {
  return qk_rope8(xn, p, first, *reinterpret_cast<const bf16x8*>(cr),
                  *reinterpret_cast<const bf16x8*>(sr));
}

// Streams KV positions [kv_begin, kv_end) of one kv-head (kc / vc point at
// head h of page 0; tok_bytes = page stride) whose page ids are
// idx[kv_begin .. kv_end) through the LDS ring (layout T) with all
// kEngineThreads threads of the workgroup; `qload()` issues the Q loads,
// `math(sb, kv0)` runs one sub-tile's math (ring slot at byte offset sb,
// positions kv0 ..) and is skipped when `active` is false (a wavefront whose
// rows are all padding only helps stream).
// CPOL: cache policy of the gathers.  ONCE: a range of at most kRing
// sub-tiles is requested whole at the start (no ring slot is refilled) and
// `pipe(wait_sub, n_sub)` runs the math of the whole range, calling
// wait_sub(i) (every thread's loads of sub-tile i have landed: a wait and a
// workgroup barrier) before it reads sub-tile i, for i = 0, 1, ... in order;
// longer ranges, and ONCE = false, stream through the ring kLookahead
// sub-tiles ahead with `math`.
struct NoPipe {
  template <typename W>
  __device__ void operator()(W&&, int) const {}
};
template <class T, int CPOL, bool ONCE, typename QLoad, typename Math, typename Pipe = NoPipe>
__device__ __forceinline__ void stream_kv(uint8_t* lds, const uint8_t* kc, const uint8_t* vc,
                                          int64_t tok_bytes, int64_t num_pages, const int32_t* idx,
                                          int kv_begin, int kv_end, QLoad&& qload, Math&& math,
                                          bool active, Pipe&& pipe = Pipe{}) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int n_sub = (kv_end - kv_begin + kSubTok - 1) / kSubTok;
  if (n_sub <= 0) return;

  int32_t* ids = reinterpret_cast<int32_t*>(lds + T::RING_BYTES);
  int win = kv_begin;
  auto stage_ids = [&]() {
    for (int i = tid; i < kIdWindow; i += kEngineThreads) {
      const int p = win + i;
      ids[i] = p < kv_end ? idx[p] : -1;
    }
  };
  stage_ids();
  lds_barrier();
  // Q is needed only at the first compute: its loads go out after the page
  // ids (which gate every DMA) and ahead of the DMAs, so the first wait
  // below covers them.
  qload();

  // Loop-invariant part of every DMA load of this thread: which token of
  // the sub-tile it serves, and the byte offset (rotated chunk) inside that
  // token's K or V row.  Whether load j of a wavefront fills K or V rows is
  // uniform over the wavefront (the K part of a sub-tile is a whole number
  // of 1 KiB wavefront loads), so it selects a buffer descriptor held in
  // scalar registers.
  static_assert(T::SUB_KB % (64 * 16) == 0, "K part of a sub-tile in whole wavefront loads");
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // When a whole load of the workgroup spans whole rows and the K part of
  // a sub-tile whole loads, load j's token is load 0's plus a constant.
  constexpr bool kTokStep = (kEngineThreads * 16) % T::ROWB == 0 &&
                            T::SUB_KB % (kEngineThreads * 16) == 0;
  int tok_j[T::LPS];
  uint32_t coff_j[T::LPS];
  bool isv_j[T::LPS];
#pragma unroll
  for (int j = 0; j < T::LPS; ++j) {
    const bool isv = (j * kEngineThreads + wave_u * 64) * 16 >= T::SUB_KB;
    const int off = (j * kEngineThreads + tid) * 16;
    const int o2 = isv ? off - T::SUB_KB : off;
    const int t = o2 / T::ROWB;
    const int slot = (o2 - t * T::ROWB) >> 4;
    tok_j[j] = t;
    isv_j[j] = isv;
    coff_j[j] = (uint32_t)((isv ? T::v_chunk(t, slot) : T::k_chunk(t, slot)) * 16);
  }
  // Raw buffer descriptors over this head's K and V rows: the last valid
  // byte is the end of the last page's row, so a page id clamped to
  // num_pages lands past it and the load returns zeros (the hardware range
  // check); the host keeps a layer's cache below 4 GiB so offsets are 32-bit
  // and the pool below 2^24 pages so a page id times the row stride is one
  // 24-bit multiply (v_mul_u32_u24, full rate).
  const uint32_t tok_b = (uint32_t)tok_bytes;
  const uint32_t n_pages = (uint32_t)num_pages;
  const int64_t n_rec64 = num_pages > 0 ? (num_pages - 1) * tok_bytes + T::ROWB : 0;
  const int n_rec = (int)(n_rec64 < 0xffffffffll ? n_rec64 : 0xffffffffll);
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)kc, (short)0, n_rec, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)vc, (short)0, n_rec, kBufferWord3);
  auto issue = [&](int s) {
    uint8_t* buf = lds + (s & (kRing - 1)) * T::SUB_BYTES;
    const int pos0 = kv_begin + s * kSubTok;
    // All page-id reads first: every LDS DMA rewrites M0, which waits for
    // outstanding LDS instructions, so reads interleaved with the DMAs
    // would each pay a full LDS round trip.
    // Positions past kv_end read the -1 that stage_ids left there (the
    // window always covers the sub-tile, lookahead sub-tiles included).
    uint32_t page[T::LPS];
#pragma unroll
    for (int j = 0; j < T::LPS; ++j) {
      if constexpr (kTokStep) {
        // load j serves token tok_j[0] + a compile-time step: one address
        constexpr int per = kEngineThreads * 16;
        page[j] = (uint32_t)ids[pos0 + tok_j[0] - win +
                                (j * per - (j * per >= T::SUB_KB ? T::SUB_KB : 0)) / T::ROWB];
      } else {
        page[j] = (uint32_t)ids[pos0 + tok_j[j] - win];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < T::LPS; ++j) {
      const uint32_t off = __umul24(min(page[j], n_pages), tok_b) + coff_j[j];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          isv_j[j] ? rv : rk, (AIOS_LDS void*)(buf + (j * kEngineThreads + wave_u * 64) * 16),
          16, off, 0, 0, CPOL);
    }
  };

  if constexpr (ONCE) {
    static_assert(kRing == 4, "the waits below count four sub-tiles");
    if (n_sub <= kRing) {
      // Every sub-tile of the range goes out now (those past the range read
      // the zero row: the range check answers them without a memory access).
      // The chip-wide burst makes the first sub-tile land a little later
      // than with two in flight, but the later ones land while the math of
      // the earlier ones runs, instead of being requested only after it.
#pragma unroll
      for (int s = 0; s < kRing; ++s) issue(s);
      // (called with compile-time i once the caller's loop is unrolled; the
      // Q loads went out first, so each wait covers them too)
      auto wait_sub = [&](int it) {
        if (it == 0)
          wait_vmcnt<3 * T::LPS>();
        else if (it == 1)
          wait_vmcnt<2 * T::LPS>();
        else if (it == 2)
          wait_vmcnt<T::LPS>();
        else
          wait_vmcnt<0>();
        lds_barrier();  // sub-tile `it` is in LDS (every thread's share)
      };
      if (__builtin_amdgcn_readfirstlane((int)active)) {
        pipe(wait_sub, n_sub);
      } else {
#pragma unroll
        for (int it = 0; it < kRing; ++it) {
          if (it >= n_sub) break;  // uniform
          wait_sub(it);
        }
      }
      wait_vmcnt<0>();  // the zero-row loads past the range have landed too
      return;
    }
  }

  // The lookahead sub-tiles are issued unconditionally (those past the
  // range gather the zero row into ring slots nobody reads), so one wait
  // with a fixed count covers the Q loads and sub-tile 0 on every path.
  // The compiler then sees Q complete before the loop; with Q possibly
  // still in flight it would wait for every outstanding DMA (vmcnt(0))
  // before each sub-tile's first MFMA and serialise the ring.
#pragma unroll
  for (int s = 0; s < kLookahead; ++s) issue(s);
  wait_vmcnt<(kLookahead - 1) * T::LPS>();

  // The loop is instantiated twice so that no branch around the math
  // sits inside it: a conditional compute makes the accumulators phi
  // values, and the compiler then copies every O tile once per sub-tile.
  auto loop = [&](auto with_math) {
    for (int it = 0; it < n_sub; ++it) {
      const int pend = min(kLookahead - 1, n_sub - 1 - it);
      if (pend >= 1)
        wait_vmcnt<T::LPS>();
      else
        wait_vmcnt<0>();
      lds_barrier();  // sub-tile `it` is in LDS; every wave is done with it-1
      const int s_next = it + kLookahead;
      if (s_next < n_sub) {
        if (kv_begin + s_next * kSubTok >= win + kIdWindow) {
          win += kIdWindow;
          stage_ids();
          lds_barrier();
        }
        issue(s_next);
      }
      if constexpr (decltype(with_math)::value)
        math((uint32_t)((it & (kRing - 1)) * T::SUB_BYTES), kv_begin + it * kSubTok);
    }
  };
  if (__builtin_amdgcn_readfirstlane((int)active))
    loop(std::true_type{});
  else
    loop(std::false_type{});
}

template <int D, bool CAUSAL, int RT = 2>
struct TileEngine {
  using T = KVTile<D>;
  static constexpr int KSTEPS = D / 32;
  static constexpr int DTILES = D / 16;

  bf16x8 qf[RT][KSTEPS];
  f32x4 o[RT][DTILES];
  float m_run[RT];
  float nm[RT];     // -(m_run, or 0 while m_run is -inf): the exponent offset
  float l_run[RT];  // row totals, set by finish()
  f32x4 ol[RT];     // row sums of P by MFMA (every element holds the sum)
  int limit[RT];   // CAUSAL: last visible KV position of the lane's rows
  int min_limit;   // CAUSAL: smallest limit of any row of the workgroup

  // Q fragment (B operand of S^T = K Q^T) of the lane's row in tile rt.
  __device__ __forceinline__ void load_q_tile(int rt, const bf16* q, bool ok) {
    const int lg = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      qf[rt][s] = ok ? *reinterpret_cast<const bf16x8*>(q + s * 32 + lg * 8) : bf16x8{};
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      m_run[rt] = kNegInf;
      nm[rt] = 0.f;
      l_run[rt] = 0.f;
      ol[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // Row totals (after the last compute).
  __device__ __forceinline__ void finish() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) l_run[rt] = ol[rt][0];
  }

  // The math of one 32-token sub-tile in LDS (KVTile layout) for the lane's
  // RT rows, in steps; positions >= kv_end (and, if CAUSAL, past each row's
  // limit) are masked.  (Deferring each sub-tile's O^T update into the next
  // iteration, behind the next S^T MFMAs, measured no faster.)

  // K rows (A of S^T = K Q^T), B = the Q fragments in registers.
  __device__ __forceinline__ void read_k(const uint8_t* kb, bf16x8 (&kf)[2][KSTEPS], int l16,
                                         int lg) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int t = tt * 16 + l16;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
        kf[tt][s] = *reinterpret_cast<const bf16x8*>(kb + t * T::ROWB +
                                                      T::k_slot(t, s * 4 + lg) * 16);
    }
  }

  // S^T tiles: st[rt][tt][i] = S[row rt*16 + l16][token tt*16 + lg*4 + i];
  // the accumulation chains are interleaved.
  __device__ __forceinline__ void mma_s(const bf16x8 (&kf)[2][KSTEPS], f32x4 (&st)[RT][2]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) st[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          st[rt][tt] = mfma16x16x32(kf[tt][s], qf[rt][s], st[rt][tt]);
  }

  // V^T fragments (A of O^T += V^T P^T) by LDS transpose reads: lane
  // (lg, l16) supplies V[token][dt*16 + 4*(l16%4)..+3] of tokens
  // lg*4 + l16/4 (first read) and 16 + lg*4 + l16/4 (second read) and
  // receives V[tokens][dt*16 + l16], the A fragment rows of the MFMA.
  __device__ __forceinline__ void load_v(const uint8_t* vb, bf16x4 (&va)[DTILES][2], int l16,
                                         int lg) {
    const int r = l16 >> 2;
    const int q4 = l16 & 3;
    const int t0 = lg * 4 + r;
    const int t1 = 16 + lg * 4 + r;
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) {
      const int dim = dt * 16 + 4 * q4;
      const int c = dim >> 3;
      const int boff = (dim & 7) * 2;
      va[dt][0] = lds_read_tr(vb + t0 * T::ROWB + T::v_slot(t0, c) * 16 + boff);
      va[dt][1] = lds_read_tr(vb + t1 * T::ROWB + T::v_slot(t1, c) * 16 + boff);
    }
  }

  // Online softmax with a lazily moved reference: m_run only moves when a
  // row's scaled max exceeds it by more than kRescaleSlack (p <= 2^slack
  // otherwise), so the O rescale below is skipped once the max settles.
  // P (bf16, the B operand of the O^T MFMA) goes to pb.
  __device__ __forceinline__ void softmax(const f32x4 (&st)[RT][2], int kv0, int kv_end,
                                          float scale_log2, int lg, bf16x8 (&pb)[RT]) {
    const bool full = kv0 + kSubTok <= kv_end && (!CAUSAL || kv0 + kSubTok - 1 <= min_limit);
    float x[RT][8];
    float mx[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) x[rt][tt * 4 + i] = st[rt][tt][i];
      if (__builtin_expect(!full, 0)) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = kv0 + tt * 16 + lg * 4 + i;
            bool ok = pos < kv_end;
            if (CAUSAL) ok = ok && pos <= limit[rt];
            if (!ok) x[rt][tt * 4 + i] = kNegInf;
          }
      }
      mx[rt] = vmax(vmax(vmax(x[rt][0], x[rt][1]), vmax(x[rt][2], x[rt][3])),
                    vmax(vmax(x[rt][4], x[rt][5]), vmax(x[rt][6], x[rt][7])));
    }
    bool need[RT];
    bool any = false;
    if constexpr (RT == 2) {
      xrow_max2(mx[0], mx[1]);
    } else {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) mx[rt] = xrow_max(mx[rt]);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      mx[rt] *= scale_log2;
      need[rt] = mx[rt] > m_run[rt] + kRescaleSlack;
      any = any || need[rt];
    }
    if (__builtin_amdgcn_ballot_w64(any)) {
      // Rows that keep their reference use alpha = 1 exactly (their reference
      // may still be -inf); a moved reference from -inf gives alpha = 0.
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const float al = need[rt] ? fast_exp2(m_run[rt] - mx[rt]) : 1.f;
        ol[rt][0] *= al;  // the other elements of ol are never read
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt) o[rt][dt] *= al;
        m_run[rt] = need[rt] ? mx[rt] : m_run[rt];
        nm[rt] = need[rt] ? -mx[rt] : nm[rt];
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = fast_exp2(fmaf(x[rt][j], scale_log2, nm[rt]));
      pb[rt] = __builtin_bit_cast(
          bf16x8, make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                             pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])));
    }
  }

  // O^T += V^T P^T, and the row sums of P by one more MFMA with an all-ones
  // A operand (the sum the O^T numerator sees, of the bf16 P).  V rows of
  // tokens >= n_valid may be stale LDS (gathers that skip them): their
  // fragments are zeroed so that P = 0 there cannot meet a NaN.
  __device__ __forceinline__ void accumulate(bf16x4 (&va)[DTILES][2], const bf16x8 (&pb)[RT],
                                             int n_valid, int lg) {
    const bf16x8 ones = (bf16x8)(bf16)1.0f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) ol[rt] = mfma16x16x32(ones, pb[rt], ol[rt]);
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) lds_wait_tied(va[dt][0], va[dt][1]);
    if (__builtin_expect(n_valid < kSubTok, 0)) {
      // va[dt][tt] element i belongs to token tt*16 + lg*4 + i.
      uint64_t keep[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        keep[tt] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tt * 16 + lg * 4 + i < n_valid) keep[tt] |= 0xffffull << (16 * i);
      }
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          va[dt][tt] = __builtin_bit_cast(bf16x4, __builtin_bit_cast(uint64_t, va[dt][tt]) & keep[tt]);
    }
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) {
      const bf16x8 vf = __builtin_shufflevector(va[dt][0], va[dt][1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) o[rt][dt] = mfma16x16x32(vf, pb[rt], o[rt][dt]);
    }
  }

  // All four steps on one sub-tile, every LDS read issued before the first
  // MFMA.
  __device__ __forceinline__ void compute(const uint8_t* kb, int kv0, int kv_end, float scale_log2,
                                          int l16, int lg) {
    bf16x8 kf[2][KSTEPS];
    bf16x4 va[DTILES][2];
    f32x4 st[RT][2];
    bf16x8 pb[RT];
    read_k(kb, kf, l16, lg);
    load_v(kb + T::SUB_KB, va, l16, lg);
    mma_s(kf, st);
    softmax(st, kv0, kv_end, scale_log2, lg, pb);
    accumulate(va, pb, kv_end - kv0, lg);
  }
};

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Sum of 16 values as a balanced tree (four levels of independent adds).
__device__ __forceinline__ float sum16(const float (&p)[16]) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = p[2 * i] + p[2 * i + 1];
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

// The tile engine with one 32-row tile per wavefront and
// v_mfma_f32_32x32x16_bf16: the same math as TileEngine<D, CAUSAL, 2> (32
// rows per wavefront, 128 per workgroup) with half the MFMA instructions
// (each 32x32x16 does the work of two 16x16x32 and costs the SIMD about as
// much vector issue as one), one row per lane pair, and a cheaper row max.
//
// Fragments (lane l, n = l % 32, h = l / 32), per 32-token sub-tile:
//   S^T = K Q^T   A = K: token n, dims 16s + 8h .. +7 (one ds_read_b128 per
//                 k-step s); B = Q^T: query row n, the same dims (kept in
//                 registers); D: query row n, tokens 8j + 4h + i in
//                 register 4j + i (j, i = 0..3)
//   softmax       16 scores of row n in the lane, the other 16 in lane l ^ 32
//   O^T += V^T P^T  per 32-dim tile and 16-token k-step, A = V^T from two LDS
//                 transpose reads (lane l: dim n of tokens 4h .. 4h+3 and
//                 8 + 4h .. 8 + 4h + 3, k-step 1 sixteen tokens on), B = P^T
//                 = the lane's own scores 0..7 (k-step 0) and 8..15 (k-step 1)
//                 as bf16 -- the permutation of the 16 tokens of a k-step is
//                 the same on both sides, so no data moves between lanes.
template <int D, bool CAUSAL>
struct TileEngine32 {
  using T = KVTile<D, true>;
  static constexpr int KS = D / 16;  // k-steps of S^T
  static constexpr int NT = D / 32;  // 32-dim tiles of O^T

  bf16x8 qf[KS];
  f32x16 o[NT];
  // Row sums of P.  CAUSAL (the prefill, whose VALU is the busier pipe): by
  // MFMA with a ones operand (element 0 is read; 4096-token prefill 166-169
  // us with the VALU sums below instead); otherwise the lane's sum over its
  // half of the row's positions, the halves added at the end (long-context
  // decode step 432.5-433.1 -> 429.8-430.5 us against the MFMA sums).
  f32x16 ol;
  float ls;
  float m_run;     // the lane's row reference (log2 domain)
  float nm;        // -(m_run, or 0 while m_run is -inf)
  float l_run;     // row total, set by finish()
  int limit;       // CAUSAL: last visible KV position of the lane's row
  int min_limit;   // CAUSAL: smallest limit of any row of the workgroup

  // Q fragments of the lane's row (B of S^T = K Q^T).
  __device__ __forceinline__ void load_q(const bf16* q, bool ok) {
    const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[s] = ok ? *reinterpret_cast<const bf16x8*>(q + s * 16 + h * 8) : bf16x8{};
  }

  // The same fragments from the raw projection q, normalised (weight w) and
  // rotated (cos / sin table rows cr, sr): lanes l and l ^ 32 hold the two
  // halves of the row (dims s * 16 + h * 8 + [0, 8)); a fragment's partner
  // (dims +- D/2) is the lane's own fragment s +- KS/2.
  __device__ __forceinline__ void load_q_rope(const bf16* q, bool ok, const bf16* w,
                                              const bf16* cr, const bf16* sr, float eps) {
    const int h = (threadIdx.x & 63) >> 5;
    float x[KS][8];
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      unpack_bf16x8(ok ? *reinterpret_cast<const bf16x8*>(q + s * 16 + h * 8) : bf16x8{}, x[s]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(x[s][i], x[s][i], ss);
    }
    ss = xor32_sum(ss);
    const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qk_norm8(x[s], inv, *reinterpret_cast<const bf16x8*>(w + s * 16 + h * 8));
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[s] = ok ? qk_rope8(x[s], x[(s + KS / 2) % KS], s < KS / 2, cr + s * 16 + h * 8,
                            sr + s * 16 + h * 8)
                 : bf16x8{};
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[t][i] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ol[i] = 0.f;
    ls = 0.f;
    m_run = kNegInf;
    nm = 0.f;
    l_run = 0.f;
  }

  // LDS addresses (ring slot 0) of the lane's reads: K for each k-step; V
  // for each 32-dim tile at its first token group (the other three groups,
  // tokens +8, +16, +24, keep the slot: constant offsets).
  struct LaneOff {
    uint32_t k[KS];
    uint32_t v[NT];
  };
  __device__ __forceinline__ LaneOff lane_offsets(const uint8_t* lds) const {
    static_assert(D == 64 || D == 96 || D == 128, "head size");
    LaneOff lo;
    const int lane = threadIdx.x & 63;
    const uint32_t base = (uint32_t)(uintptr_t)(AIOS_LDS const uint8_t*)lds;
    const int t = lane & 31, h = lane >> 5;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      lo.k[s] = base + (uint32_t)(t * T::ROWB + T::k_slot(t, 2 * s + h) * 16);
    // transpose read: in each 16-lane group g, lane j supplies dims
    // 4 (j % 4) .. +3 of token 4 (g / 2) + j / 4 within the tile's half g % 2
    const int g = lane >> 4, j = lane & 15;
    const int tv = 4 * (g >> 1) + (j >> 2);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int dim = nt * 32 + 16 * (g & 1) + 4 * (j & 3);
      lo.v[nt] = base + (uint32_t)(T::SUB_KB + tv * T::ROWB + T::v_slot(tv, dim >> 3) * 16 +
                                   (dim & 7) * 2);
    }
    return lo;
  }

  template <typename QLoad>
  __device__ void run(uint8_t* lds, const uint8_t* kc, const uint8_t* vc, int64_t tok_bytes,
                      int64_t num_pages, const int32_t* idx, int kv_begin, int kv_end,
                      float scale_log2, QLoad&& qload, bool active = true) {
    reset();
    const LaneOff lo = lane_offsets(lds);
    // The causal (prefill) engine re-reads K/V across query tiles; the
    // decode engine (shared prefix) streams it once.
    stream_kv<T, CAUSAL ? 0 : kCpolStream, !CAUSAL>(
        lds, kc, vc, tok_bytes, num_pages, idx, kv_begin, kv_end, qload,
        [&](uint32_t sb, int kv0) { compute_at(lo, sb, kv0, kv_end, scale_log2); }, active,
        [&](auto&& wait_sub, int n_sub) {
          switch (n_sub) {
            case 1: pipe_n<1>(lo, wait_sub, kv_begin, kv_end, scale_log2); break;
            case 2: pipe_n<2>(lo, wait_sub, kv_begin, kv_end, scale_log2); break;
            case 3: pipe_n<3>(lo, wait_sub, kv_begin, kv_end, scale_log2); break;
            default: pipe_n<4>(lo, wait_sub, kv_begin, kv_end, scale_log2); break;
          }
        });
    // (lanes l and l ^ 32 hold the two halves of a row)
    if constexpr (CAUSAL) l_run = ol[0];
    else l_run = xor32_sum(ls);
  }

  // --- the decode math of a range resident in LDS, software-pipelined ---
  // One sub-tile's math is three dependent steps: S^T (MFMA), the online
  // softmax (VALU, a quarter-rate exponential per score) and O^T (MFMA).
  // With every sub-tile of the range requested at once, iteration i runs
  // the softmax of sub-tile i beside the O^T MFMAs of sub-tile i - 1 (two
  // independent pieces of work, so the matrix core and the VALU run at once
  // instead of in turn), then waits for sub-tile i + 1 and issues its S^T
  // MFMAs, which the compiler schedules beside the softmax.  A moved
  // softmax reference rescales O after the O^T update of sub-tile i - 1
  // (whose P was relative to the old reference).
  __device__ __forceinline__ void read_k_at(const LaneOff& lo, uint32_t sb, bf16x8 (&kf)[KS]) const {
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kf[s] = *reinterpret_cast<AIOS_LDS const bf16x8*>((AIOS_LDS const uint8_t*)(uintptr_t)(lo.k[s] + sb));
  }
  // V^T fragments by LDS transpose reads in inline asm, waited for in
  // mma_o_at.  The compiler's own transpose-read builtin makes it wait for
  // every LDS DMA still in flight (vmcnt(0)) before the first read, which
  // held the whole pipeline behind the chunk's last sub-tile (long-context
  // step 446 -> 442 us without it).
  __device__ __forceinline__ void read_v_at(const LaneOff& lo, uint32_t sb, bf16x4 (&va)[NT][4]) const {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint32_t a = lo.v[nt] + sb;
      va[nt][0] = lds_read_tr_at<0>(a);
      va[nt][1] = lds_read_tr_at<8 * T::ROWB>(a);
      va[nt][2] = lds_read_tr_at<16 * T::ROWB>(a);
      va[nt][3] = lds_read_tr_at<24 * T::ROWB>(a);
    }
  }
  __device__ __forceinline__ f32x16 mma_s_at(const bf16x8 (&kf)[KS]) const {
    f32x16 st;
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) st = mfma32x32x16(kf[s], qf[s], st);
    return st;
  }
  // Softmax of one sub-tile's scores (positions kv0 ..): P as two bf16x8
  // B fragments; returns whether any lane's reference moved (then `al` is
  // the log2 of the factor its O and row sum must take, 0 for the others).
  // MASK: positions >= kv_end may lie in this sub-tile (selects, no branch).
  template <bool MASK>
  __device__ __forceinline__ bool softmax_at(const f32x16& st, int kv0, int kv_end, float scale_log2,
                                             bf16x8& pb0, bf16x8& pb1, float& al, float& psum) {
    const int h = (threadIdx.x & 63) >> 5;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = st[r];
    if constexpr (MASK) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        x[r] = kv0 + 8 * (r >> 2) + 4 * h + (r & 3) < kv_end ? x[r] : kNegInf;
    }
    float mx = vmax(vmax(vmax(vmax(x[0], x[1]), vmax(x[2], x[3])),
                         vmax(vmax(x[4], x[5]), vmax(x[6], x[7]))),
                    vmax(vmax(vmax(x[8], x[9]), vmax(x[10], x[11])),
                         vmax(vmax(x[12], x[13]), vmax(x[14], x[15]))));
    mx = xor32_max(mx) * scale_log2;
    const bool need = mx > m_run + kRescaleSlack;
    const bool any = __builtin_amdgcn_ballot_w64(need) != 0;
    // (the factor, one exponential, is formed only when some lane moved)
    al = need ? m_run - mx : 0.f;
    m_run = need ? mx : m_run;
    nm = need ? -mx : nm;
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(x[r], scale_log2, nm));
    psum = sum16(p);
    pb0 = __builtin_bit_cast(bf16x8, make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                                                pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])));
    pb1 = __builtin_bit_cast(bf16x8, make_uint4(pack_bf16x2(p[8], p[9]), pack_bf16x2(p[10], p[11]),
                                                pack_bf16x2(p[12], p[13]), pack_bf16x2(p[14], p[15])));
    return any;
  }
  // O^T += V^T P^T (the range's V rows past kv_end are zero rows, gathered
  // through the -1 page ids, so no masking here).
  __device__ __forceinline__ void mma_o_at(bf16x4 (&va)[NT][4], const bf16x8& pb0, const bf16x8& pb1) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      lds_wait_tied(va[nt][0], va[nt][1]);
      lds_wait_tied(va[nt][2], va[nt][3]);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const bf16x8 v0 = __builtin_shufflevector(va[nt][0], va[nt][1], 0, 1, 2, 3, 4, 5, 6, 7);
      const bf16x8 v1 = __builtin_shufflevector(va[nt][2], va[nt][3], 0, 1, 2, 3, 4, 5, 6, 7);
      o[nt] = mfma32x32x16(v0, pb0, o[nt]);
      o[nt] = mfma32x32x16(v1, pb1, o[nt]);
    }
  }
  // O and the row sum times 2^dm (dm = old reference - new, 0 for lanes
  // whose reference stayed).  Rare: the reference moves only when a row's
  // max grows by more than the slack.  The empty asm keeps the compiler from
  // speculating the 65 multiplies out of the branch that guards this call.
  __device__ __forceinline__ void rescale(float dm) {
    static_assert(!CAUSAL, "the pipelined decode path keeps the VALU row sums");
    asm volatile("");
    const float al = fast_exp2(dm);
    ls *= al;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[nt] *= al;
  }
  // Iteration I of N (N <= kRing sub-tiles of the range [kv_begin,
  // kv_end)); PARTIAL: the last sub-tile may end before its 32 positions.
  template <int N, bool PARTIAL, int I, typename WaitSub>
  __device__ __forceinline__ void pipe_iter(const LaneOff& lo, WaitSub& wait_sub, int kv_begin,
                                            int kv_end, float scale_log2, bf16x8 (&kf)[KS],
                                            bf16x4 (&va)[NT][4], f32x16& st, bf16x8& pp0,
                                            bf16x8& pp1) {
    constexpr bool NEXT = I + 1 < N;
    constexpr bool PREV = I > 0;
    // In source order the softmax of sub-tile I and the O^T of I - 1 come
    // ahead of the wait for sub-tile I + 1, and its K reads and S^T after
    // it; the compiler's own schedule then overlaps them.  Measured against
    // forcing that order with a scheduling barrier (442-443 us per
    // long-context step) and against `sched_group_barrier` groups of LDS
    // reads, VALU and MFMAs (441-442 us): 437.6-439.3 us.
    if constexpr (PREV) read_v_at(lo, (uint32_t)((I - 1) * T::SUB_BYTES), va);
    float al, psum;
    bf16x8 pc0, pc1;
    const bool moved = softmax_at<PARTIAL && !NEXT>(st, kv_begin + I * kSubTok, kv_end,
                                                    scale_log2, pc0, pc1, al, psum);
    if constexpr (PREV) mma_o_at(va, pp0, pp1);
    if (__builtin_expect(moved, 0)) rescale(al);
    ls += psum;  // (after the rescale: psum is relative to the new reference)
    if constexpr (NEXT) {
      wait_sub(I + 1);
      read_k_at(lo, (uint32_t)((I + 1) * T::SUB_BYTES), kf);
      st = mma_s_at(kf);
    }
    pp0 = pc0;
    pp1 = pc1;
  }
  template <int N, bool PARTIAL, typename WaitSub, int... Is>
  __device__ __forceinline__ void pipe_seq(const LaneOff& lo, WaitSub& wait_sub, int kv_begin,
                                           int kv_end, float scale_log2,
                                           std::integer_sequence<int, Is...>) {
    static_assert(N >= 1 && N <= kRing, "range resident in the ring");
    bf16x8 kf[KS];
    bf16x4 va[NT][4];
    bf16x8 pp0, pp1;
    wait_sub(0);
    read_k_at(lo, 0, kf);
    f32x16 st = mma_s_at(kf);
    (pipe_iter<N, PARTIAL, Is>(lo, wait_sub, kv_begin, kv_end, scale_log2, kf, va, st, pp0, pp1),
     ...);
    read_v_at(lo, (uint32_t)((N - 1) * T::SUB_BYTES), va);
    mma_o_at(va, pp0, pp1);
  }
  template <int N, typename WaitSub>
  __device__ __forceinline__ void pipe_n(const LaneOff& lo, WaitSub&& wait_sub, int kv_begin,
                                         int kv_end, float scale_log2) {
    if ((kv_end - kv_begin) % kSubTok == 0)
      pipe_seq<N, false>(lo, wait_sub, kv_begin, kv_end, scale_log2,
                         std::make_integer_sequence<int, N>{});
    else
      pipe_seq<N, true>(lo, wait_sub, kv_begin, kv_end, scale_log2,
                        std::make_integer_sequence<int, N>{});
  }

  __device__ __forceinline__ void compute_at(const LaneOff& lo, uint32_t sb, int kv0, int kv_end,
                                             float scale_log2) {
    const int h = (threadIdx.x & 63) >> 5;
    bf16x8 kf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      kf[s] = *reinterpret_cast<AIOS_LDS const bf16x8*>((AIOS_LDS const uint8_t*)(uintptr_t)(lo.k[s] + sb));
    bf16x4 va[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint32_t a = lo.v[nt] + sb;
      va[nt][0] = lds_read_tr_at<0>(a);
      va[nt][1] = lds_read_tr_at<8 * T::ROWB>(a);
      va[nt][2] = lds_read_tr_at<16 * T::ROWB>(a);
      va[nt][3] = lds_read_tr_at<24 * T::ROWB>(a);
    }
    f32x16 st;
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] = 0.f;
    // The prefill (two workgroups per CU, bound by LDS reads) raises a
    // wavefront's issue priority over its MFMA chains so the wavefronts of a
    // SIMD alternate between reading LDS and multiplying (4096-token prefill
    // 171-175 -> 160-166 us); the decode measured slower with it.
    if constexpr (CAUSAL) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < KS; ++s) st = mfma32x32x16(kf[s], qf[s], st);
    if constexpr (CAUSAL) __builtin_amdgcn_s_setprio(0);

    // Online softmax of the lane's row (the TileEngine rule: lazily moved
    // reference, log2 domain).
    const bool full = kv0 + kSubTok <= kv_end && (!CAUSAL || kv0 + kSubTok - 1 <= min_limit);
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = st[r];
    if (__builtin_expect(!full, 0)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int pos = kv0 + 8 * (r >> 2) + 4 * h + (r & 3);
        bool ok = pos < kv_end;
        if (CAUSAL) ok = ok && pos <= limit;
        if (!ok) x[r] = kNegInf;
      }
    }
    float mx = vmax(vmax(vmax(vmax(x[0], x[1]), vmax(x[2], x[3])),
                         vmax(vmax(x[4], x[5]), vmax(x[6], x[7]))),
                    vmax(vmax(vmax(x[8], x[9]), vmax(x[10], x[11])),
                         vmax(vmax(x[12], x[13]), vmax(x[14], x[15]))));
    mx = xor32_max(mx) * scale_log2;
    const bool need = mx > m_run + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float al = need ? fast_exp2(m_run - mx) : 1.f;
      if constexpr (CAUSAL) ol[0] *= al;  // the other elements of ol are never read
      else ls *= al;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] *= al;
      m_run = need ? mx : m_run;
      nm = need ? -mx : nm;
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(x[r], scale_log2, nm));
    if constexpr (!CAUSAL) ls += sum16(p);
    const bf16x8 pb0 = __builtin_bit_cast(
        bf16x8, make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                           pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])));
    const bf16x8 pb1 = __builtin_bit_cast(
        bf16x8, make_uint4(pack_bf16x2(p[8], p[9]), pack_bf16x2(p[10], p[11]),
                           pack_bf16x2(p[12], p[13]), pack_bf16x2(p[14], p[15])));

    // V fragments complete; tokens >= n_valid zeroed (stale LDS must not
    // meet P = 0 as a NaN).  va[nt][q] element e is token 8q + 4h + e.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      lds_wait_tied(va[nt][0], va[nt][1]);
      lds_wait_tied(va[nt][2], va[nt][3]);
    }
    const int n_valid = kv_end - kv0;
    if (__builtin_expect(n_valid < kSubTok, 0)) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint64_t keep = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (8 * q + 4 * h + e < n_valid) keep |= 0xffffull << (16 * e);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          va[nt][q] = __builtin_bit_cast(bf16x4, __builtin_bit_cast(uint64_t, va[nt][q]) & keep);
      }
    }
    if constexpr (CAUSAL) {
      const bf16x8 ones = (bf16x8)(bf16)1.0f;
      __builtin_amdgcn_s_setprio(1);
      ol = mfma32x32x16(ones, pb0, ol);
      ol = mfma32x32x16(ones, pb1, ol);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const bf16x8 v0 = __builtin_shufflevector(va[nt][0], va[nt][1], 0, 1, 2, 3, 4, 5, 6, 7);
      const bf16x8 v1 = __builtin_shufflevector(va[nt][2], va[nt][3], 0, 1, 2, 3, 4, 5, 6, 7);
      o[nt] = mfma32x32x16(v0, pb0, o[nt]);
      o[nt] = mfma32x32x16(v1, pb1, o[nt]);
    }
    if constexpr (CAUSAL) __builtin_amdgcn_s_setprio(0);
  }
};

}  // namespace aios
