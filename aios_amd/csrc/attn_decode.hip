// Paged decode for a CandidateGroup: shared-prefix cascade (kernel (c)),
// per-row ragged suffix (kernel (d)) and the log-sum-exp combine.
//
// decode_main_kernel is one launch with two kinds of workgroups:
//   * prefix workgroups (blockIdx.x < prefix_wgs): the 32-row MFMA tile
//     engine (TileEngine32) over one chunk of the shared prefix for one
//     kv-head and up to 128 of the batch*G query rows; the prefix KV is
//     therefore read once per kv-head for the whole group, not once per
//     candidate;
//   * suffix workgroups: one (row, kv-head, split) item of the row's own
//     pages after the prefix.  Its four wavefronts take the item's
//     32-position sub-tiles round-robin, gather each into their own LDS
//     region and run the tile engine's math with one 16-row MFMA tile
//     holding the row's G query heads.  With the cascade (the combine runs
//     anyway) every wavefront writes its own partial; otherwise the four
//     softmax states are merged through LDS.  With k_new / v_new given, the
//     row's new token is read from them and written to its page in the
//     same launch.
// Every workgroup writes a normalised partial (o, lse) into the parts array
// (layout in kernels.hpp); decode_combine_kernel (attn_combine.hip) merges
// the parts of each (row, kv-head).
// When a (row, head) has a single part the suffix workgroup writes bf16
// output directly and no combine runs.
#include "engine.hpp"

namespace aios {

// The rotation table row of row b (its position clamped into the table);
// b < 0 (a padding row, whose fragments are zero whatever it reads): row 0.
__device__ __forceinline__ int64_t decode_rope_row(const DecodeArgs& a, int b) {
  const int64_t pos = b >= 0 ? (int64_t)a.positions[b] : 0;
  return min(max(pos, (int64_t)0), a.rope_rows - 1);
}

// The words of the parts arguments that the prefix part does not use, read
// at its end: kept live, their registers are not reused while the kernel's
// first scalar loads are in flight, so no wait for those loads lands ahead
// of the page-id loads (long-context main launch 8.53 -> 8.47 us).
__device__ __forceinline__ void keep_parts_words(const DecodeArgs& a) {
  asm volatile("" ::"s"(a.parts.n_chunks), "s"(a.parts.spare));
}

// ---------------------------------------------------------------------------
// prefix part (ROPE: the query rows are normalised and rotated on load)
template <int D, int G, bool ROPE>
__device__ __forceinline__ void decode_prefix_part(uint8_t* lds, const DecodeArgs& a, int wg) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hl = lane >> 5;
  const int mg = wg % a.m_groups;
  const int unit = wg / a.m_groups;
  // Consecutive workgroups take different kv-heads: the hardware deals
  // workgroups round-robin to the XCDs, so with 8 kv-heads every chunk of
  // one head (and the combine of that head, which uses the same order) runs
  // on one XCD and its partials stay in that XCD's L2.
  const int h = unit % a.num_kv_heads;
  const int chunk = unit / a.num_kv_heads;

  TileEngine32<D, false> eng;
  eng.min_limit = 0x7fffffff;
  // The lane's query row (lanes l and l ^ 32 share it).
  const int m = mg * 128 + wave * 32 + (lane & 31);
  const bool ok = m < a.m_rows;
  const int b = m / G;
  const int g = m - b * G;
  const bf16* qr = a.q + (int64_t)b * a.q_tok_stride + (int64_t)(h * G + g) * D;
  const int kv_begin = chunk * a.chunk_len;
  const int kv_end = min(a.prefix_len, kv_begin + a.chunk_len);
  const int64_t tok_bytes = a.kv_tok_stride * 2;
  // A wavefront whose 32 rows are all padding only helps stream K/V.
  const bool active = mg * 128 + wave * 32 < a.m_rows;
  // (rotation on load: the position goes out now, with the page ids)
  const int64_t rrow = ROPE ? decode_rope_row(a, ok ? b : -1) : 0;
  eng.run(lds, reinterpret_cast<const uint8_t*>(a.k_cache) + (int64_t)h * D * 2,
          reinterpret_cast<const uint8_t*>(a.v_cache) + (int64_t)h * D * 2, tok_bytes,
          a.num_pages, a.indices, kv_begin, kv_end, a.scale_log2,
          [&] {
            if constexpr (ROPE)
              eng.load_q_rope(qr, ok, a.q_norm, a.rope_cos + rrow * D, a.rope_sin + rrow * D,
                              a.norm_eps);
            else
              eng.load_q(qr, ok);
          },
          active);

  if (!ok) {
    keep_parts_words(a);
    return;
  }
  const float l_tot = eng.l_run;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // o[nt] register 4j + i: dim 32 nt + 8j + 4h + i of the lane's row (h =
  // hl: lanes l and l ^ 32 hold the two halves of each 8-dim group).  For a
  // pair of groups (j, j + 1) the lanes swap one half each, so lane h = 0
  // holds group j whole and lane h = 1 group j + 1: one 16-byte store per
  // lane fills the row's 32-byte segment of a 16-dim tile, and each store
  // instruction writes 32 rows x 32 contiguous bytes.
#pragma unroll
  for (int nt = 0; nt < D / 32; ++nt)
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
      const int j0 = 2 * jp, j1 = j0 + 1;
      uint2 g0, g1;  // this lane's halves of groups j0, j1
      g0.x = pack_bf16x2(eng.o[nt][4 * j0] * inv, eng.o[nt][4 * j0 + 1] * inv);
      g0.y = pack_bf16x2(eng.o[nt][4 * j0 + 2] * inv, eng.o[nt][4 * j0 + 3] * inv);
      g1.x = pack_bf16x2(eng.o[nt][4 * j1] * inv, eng.o[nt][4 * j1 + 1] * inv);
      g1.y = pack_bf16x2(eng.o[nt][4 * j1 + 2] * inv, eng.o[nt][4 * j1 + 3] * inv);
      // lane h = 0 sends its half of j1 and takes the partner's half of j0;
      // lane h = 1 sends its half of j0 and takes the partner's half of j1
      const uint2 snd = hl ? g0 : g1;
      const auto rx = __builtin_amdgcn_permlane32_swap(snd.x, snd.x, false, false);
      const auto ry = __builtin_amdgcn_permlane32_swap(snd.y, snd.y, false, false);
      const uint2 rcv = hl ? make_uint2(rx[0], ry[0]) : make_uint2(rx[1], ry[1]);
      const uint4 v = hl ? make_uint4(rcv.x, rcv.y, g1.x, g1.y) : make_uint4(g0.x, g0.y, rcv.x, rcv.y);
      *reinterpret_cast<uint4*>(a.parts.o + a.parts.o_index(D, h, chunk, m, nt * 32 + 16 * jp + 8 * hl)) =
          v;
    }
  if (hl == 0)
    a.parts.lse[a.parts.lse_index(h, chunk, m)] =
        l_tot > 0.f ? eng.m_run + fast_log2(l_tot) : kNegInf;
  keep_parts_words(a);
}

// ---------------------------------------------------------------------------
// Rotation on load in a suffix item, in the pair layout: eight lanes per row
// (row 8 p + lane / 8 in pass p: the item's G query rows, then the new
// token's K row), lane c = lane % 8 holding the P = D / 16 pairs (i, i + D/2)
// for i in [P c, P c + P).  Each pair is rotated by the lane that holds both
// of its dims and a row's sum of squares takes three DPP steps, so a lane
// normalises and rotates 2 P elements per pass (12 at D = 96) with no
// partner exchange; in the 16-row tile layout (one query row per lane of a
// 16-lane group, G of its 16 rows live) a lane took 4 D / 16 of them plus
// the K row's.  The rows go to the wavefront's staging area in LDS as bf16
// and are read back as query fragments and as the K row's 16-byte chunks.
// Arithmetic and roundings are those of qk_norm8 / qk_rope8.
template <int D, int G>
struct RopePairs {
  static constexpr int P = D / 16;  // pairs per lane
  static constexpr int W = P / 2;   // 32-bit words per half row per lane
  static constexpr int ROWS = G + 1;
  static constexpr int NPASS = (ROWS + 7) / 8;
  static constexpr int STAGE_BYTES = (ROWS * D * 2 + 15) / 16 * 16;
  static_assert(P % 2 == 0, "whole words per half row");
  uint32_t x[NPASS][2][W], w[NPASS][2][W], c[NPASS][2][W], s[NPASS][2][W];

  // q0: the item's first query row, kn: the new K row (a valid row of D
  // bf16 either way), qw / kw: norm weights, cr / sr: the table rows of the
  // position.  Lanes past the last row load query row 0 again (not used):
  // the loads carry no branch.
  __device__ __forceinline__ void load(const bf16* q0, const bf16* kn, const bf16* qw,
                                       const bf16* kw, const bf16* cr, const bf16* sr) {
    const int lane = threadIdx.x & 63;
    const int c8 = lane & 7;
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int r = ps * 8 + (lane >> 3);
      const bool isk = r == G;
      const bf16* xs = isk ? kn : q0 + (r < G ? r : 0) * D;
      const bf16* ws = isk ? kw : qw;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int off = hf * (D / 2) + P * c8;
        const uint32_t* xp = reinterpret_cast<const uint32_t*>(xs + off);
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(ws + off);
        const uint32_t* cp = reinterpret_cast<const uint32_t*>(cr + off);
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(sr + off);
#pragma unroll
        for (int i = 0; i < W; ++i) {
          x[ps][hf][i] = xp[i];
          w[ps][hf][i] = wp[i];
          c[ps][hf][i] = cp[i];
          s[ps][hf][i] = sp[i];
        }
      }
    }
  }

  // Once the loads have landed: the rotated rows into stage ([ROWS][D] bf16).
  __device__ __forceinline__ void finish(uint8_t* stage, float eps) const {
    const int lane = threadIdx.x & 63;
    const int c8 = lane & 7;
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int r = ps * 8 + (lane >> 3);
      float xl[P], xh[P];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        xl[2 * i] = lo_bf16(x[ps][0][i]);
        xl[2 * i + 1] = hi_bf16(x[ps][0][i]);
        xh[2 * i] = lo_bf16(x[ps][1][i]);
        xh[2 * i + 1] = hi_bf16(x[ps][1][i]);
      }
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < P; ++i) ss = fmaf(xl[i], xl[i], ss);
#pragma unroll
      for (int i = 0; i < P; ++i) ss = fmaf(xh[i], xh[i], ss);
      ss = row8_sum(ss);
      const float inv = rsqrtf(ss / (float)D + eps);
      uint32_t yl[W], yh[W];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float ol[2], oh[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const uint32_t wl = w[ps][0][i], wh = w[ps][1][i];
          const uint32_t cl = c[ps][0][i], ch = c[ps][1][i];
          const uint32_t sl = s[ps][0][i], sh = s[ps][1][i];
          const float nl = round_bf16(xl[2 * i + k] * inv * (k ? hi_bf16(wl) : lo_bf16(wl)));
          const float nh = round_bf16(xh[2 * i + k] * inv * (k ? hi_bf16(wh) : lo_bf16(wh)));
          ol[k] = round_bf16(round_bf16(nl * (k ? hi_bf16(cl) : lo_bf16(cl))) +
                             round_bf16(-nh * (k ? hi_bf16(sl) : lo_bf16(sl))));
          oh[k] = round_bf16(round_bf16(nh * (k ? hi_bf16(ch) : lo_bf16(ch))) +
                             round_bf16(nl * (k ? hi_bf16(sh) : lo_bf16(sh))));
        }
        yl[i] = pack_bf16x2(ol[0], ol[1]);
        yh[i] = pack_bf16x2(oh[0], oh[1]);
      }
      if (r < ROWS) {
        uint32_t* dl = reinterpret_cast<uint32_t*>(stage + (r * D + P * c8) * 2);
        uint32_t* dh = reinterpret_cast<uint32_t*>(stage + (r * D + D / 2 + P * c8) * 2);
#pragma unroll
        for (int i = 0; i < W; ++i) {
          dl[i] = yl[i];
          dh[i] = yh[i];
        }
      }
    }
  }
};

// LDS of decode_main_kernel: the prefix part's ring and page-id window, or
// the suffix item's four sub-tile regions and the staging areas of the
// rotation on load.
template <int D, int G>
constexpr int decode_lds_bytes() {
  constexpr int a = KVTile<D>::LDS_BYTES;
  constexpr int b = KVTile<D>::RING_BYTES + (kEngineThreads / 64) * RopePairs<D, G>::STAGE_BYTES;
  return a > b ? a : b;
}

// ---------------------------------------------------------------------------
// suffix part: one workgroup per (row, kv-head, split) item.  Its four
// wavefronts take the item's 32-position sub-tiles round-robin; each gathers
// its sub-tile of the row's own pages into its own LDS region (the engine's
// layout) and runs the engine math with one 16-row MFMA tile whose first G
// rows are the row's query heads.  Each wavefront then writes its own
// partial state (DecodeArgs::wave_parts), or the four states are merged
// through LDS by the first wavefront.
template <int D, int G, bool ROPE>
__device__ __forceinline__ void decode_suffix_item(uint8_t* lds, const DecodeArgs& a, int item) {
  using T = KVTile<D>;
  constexpr int CH = T::SUB_BYTES / 16;  // 16-byte chunks per sub-tile (K then V)
  constexpr int NJ = CH / 64;            // DMA loads per lane per sub-tile
  constexpr int NW = kEngineThreads / 64;
  constexpr int DT = D / 16;
  static_assert(CH % 64 == 0, "sub-tile must split over one wavefront");
  static_assert((CH / 2) % 64 == 0, "each wavefront load is all K or all V");
  static_assert(G <= 16, "one MFMA row tile");
  static_assert(DT * 64 * 16 + 2 * 16 * 4 <= T::SUB_BYTES, "merge state fits the wave region");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  uint8_t* buf = lds + wave * T::SUB_BYTES;
  const int split = item % a.n_splits;
  const int bh = item / a.n_splits;
  const int h = bh % a.num_kv_heads;
  const int b = bh / a.num_kv_heads;

  // The row bounds gate everything: they go out first (cu_k is a preloaded
  // argument).
  const int base = a.cu_k[b];
  const int kv_len = a.cu_k[b + 1] - base;
  const bool append = a.out_loc != nullptr;  // out_loc and k_new come together
  const int s_begin = a.prefix_len + split * a.split_len;
  const int s_end = min(kv_len, s_begin + a.split_len);

  TileEngine<D, false, 1> eng;
  eng.reset();
  // Rotation on load (q_norm given): the row's position goes out with the
  // first sub-tile's page ids (which are waited for before the gathers
  // anyway, so it adds no round trip); the raw rows, norm weights and cos /
  // sin entries right behind the first sub-tile's loads (they land with
  // them, and nothing of them is held while those loads are issued); the
  // norm and rotation (RopePairs) run once they have landed.
  constexpr bool rope = ROPE;
  const bf16* qrow0 = a.q + (int64_t)b * a.q_tok_stride + (int64_t)(h * G) * D;
  const bf16* qrow = qrow0 + (int64_t)min(l16, G - 1) * D;
  int32_t pos_raw = 0;

  // Fused append: the row's last position is its new token, whose rows are
  // read from k_new / v_new beside its sub-tile's gathers (page selector
  // kNewTok; the gather itself reads the zero row), then written over the
  // zero row and to its page (no other workgroup of the launch reads that
  // page).  The caller's promise is that the slot out_loc[b] is the row's
  // last page id, so whether the rows enter the sub-tile is decided from
  // that page id, already loaded: one outside the pool leaves the zero row
  // (the row attends to zeros there) and the slot is not written, as the
  // separate append and decode would do.  The slot itself is needed only
  // for the stores: it is loaded with the first sub-tile's page ids.
  constexpr uint32_t kNoPage = 0xffffffffu;
  constexpr uint32_t kNewTok = 0xfffffffeu;
  const int t_new = append ? kv_len - 1 : -1;
  int64_t new_dst = -1;
  bool new_ok = false;
  bool slot_pending = append;
  int32_t slot_raw = -1;
  const uint8_t* kc = reinterpret_cast<const uint8_t*>(a.k_cache) + (int64_t)h * D * 2;
  const uint8_t* vc = reinterpret_cast<const uint8_t*>(a.v_cache) + (int64_t)h * D * 2;
  const uint8_t* kn = append
                          ? reinterpret_cast<const uint8_t*>(a.k_new + (int64_t)b * a.k_new_stride +
                                                             (int64_t)h * D)
                          : g_zero_kv_row;
  const uint8_t* vn = append
                          ? reinterpret_cast<const uint8_t*>(a.v_new + (int64_t)b * a.v_new_stride +
                                                             (int64_t)h * D)
                          : g_zero_kv_row;
  // With the rotation on load, the new token's K row is normalised and
  // rotated (by every wavefront, with its query rows; the one whose
  // sub-tile holds the token uses it), written over that sub-tile's loaded
  // K row once its loads land (lane c < CPR: dims 8c .. 8c + 7), and to the
  // cache page.
  using RP = RopePairs<D, G>;
  RP rp;
  uint8_t* stage = lds + T::RING_BYTES + wave * RP::STAGE_BYTES;
  bool rope_pending = rope;
  // Q goes out behind the first sub-tile's loads (it is needed only by the
  // math; issued first, its address would wait for the kernel arguments
  // that are not preloaded, ahead of the row bounds and page ids).
  bool q_pending = !rope;
  // The gathers are raw-buffer LDS loads over this head's K and V rows, as
  // in the prefix engine: the range ends with the last page's row, so a page
  // id clamped to num_pages reads zeros by the hardware range check (page
  // ids outside the pool, positions past the item's end, and the new token,
  // whose rows are written into the sub-tile below), and each load's offset
  // is one 24-bit multiply (the host keeps a layer's cache below 4 GiB and
  // the pool below 2^24 pages) plus the chunk's offset in the row.
  const uint32_t tok_b = (uint32_t)(a.kv_tok_stride * 2);
  const uint32_t n_pages = (uint32_t)a.num_pages;
  const int64_t n_rec64 = a.num_pages > 0 ? (a.num_pages - 1) * (int64_t)tok_b + T::ROWB : 0;
  const int n_rec = (int)(n_rec64 < 0xffffffffll ? n_rec64 : 0xffffffffll);
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)kc, (short)0, n_rec, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)vc, (short)0, n_rec, kBufferWord3);
  for (int kv0 = s_begin + wave * kSubTok; kv0 < s_end; kv0 += NW * kSubTok) {
    // The page ids are loaded by every lane (positions past the item's end
    // clamped to its last one, then not selected): no branch separates the
    // row's position, loaded here too, from the page ids, so both are in
    // flight together.
    const int pos = kv0 + lane;
    const uint32_t id = (uint32_t)a.indices[base + min(pos, s_end - 1)];
    if (rope_pending) pos_raw = a.positions[b];
    if (slot_pending) slot_raw = a.out_loc[b];
    __builtin_amdgcn_sched_barrier(0);
    // While they are in flight: each DMA load's chunk offset in its row (the
    // divisions by CPR included), held in registers so that none of it is
    // recomputed between the page ids' arrival and the last load's issue.
    // Load j and load j + NJ / 2 (K and V) cover the same tokens.
    int tok_j[NJ / 2];
    uint32_t coff_j[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = j * 64 + lane;
      const bool isv = c >= CH / 2;  // the same for the whole wavefront
      const int c2 = isv ? c - CH / 2 : c;
      const int t = c2 / T::CPR;
      const int slot = c2 - t * T::CPR;
      if (!isv) tok_j[j] = t;
      coff_j[j] = (uint32_t)((isv ? T::v_chunk(t, slot) : T::k_chunk(t, slot)) * 16);
      asm volatile("" : "+v"(coff_j[j]));
    }
    uint32_t sel = kNoPage;
    if (lane < kSubTok && pos < s_end) sel = pos != t_new ? id : id < n_pages ? kNewTok : kNoPage;
    // (the position and the slot are taken here, where they have landed
    // with the page ids: used only behind the DMA loads, they would
    // otherwise be loaded there, one more round trip)
    if (rope_pending) asm volatile("" : "+v"(pos_raw));
    if (slot_pending) asm volatile("" : "+v"(slot_raw));
    // Loads whose tokens all lie past the item's end are skipped (the math
    // masks those tokens and zeroes their V fragments).
    // All page-id exchanges first: each LDS DMA rewrites M0, which waits for
    // outstanding LDS instructions, and a load behind the exchanges would
    // also be waited for.
    const int n_valid = __builtin_amdgcn_readfirstlane(min(s_end - kv0, kSubTok));
    uint32_t prow[NJ / 2];  // page byte offset of load j's token
#pragma unroll
    for (int j = 0; j < NJ / 2; ++j)
      prow[j] = __umul24(min((uint32_t)__shfl((int)sel, tok_j[j]), n_pages), tok_b);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (((j * 64) % (CH / 2)) / T::CPR >= n_valid) continue;
      const bool isv = j * 64 >= CH / 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isv ? rv : rk,
                                               (AIOS_LDS void*)(buf + j * 64 * 16), 16,
                                               prow[j % (NJ / 2)] + coff_j[j], 0, 0, 0);
    }
    // The new token's raw K / V rows (lane c < CPR: K chunk c, CPR <= c <
    // 2 CPR: V chunk c - CPR), in flight with the gathers: written over the
    // zero row the gathers left for it once they land, and to its page.
    // (the item holding the token: a split item may end within a sub-tile
    // of it)
    const bool new_sub = kv0 <= t_new && t_new < kv0 + kSubTok && t_new < s_end;  // uniform
    uint4 nrow = make_uint4(0u, 0u, 0u, 0u);
    bool new_gather = false;
    if (new_sub) {
      const int c = lane < T::CPR ? lane : lane < 2 * T::CPR ? lane - T::CPR : 0;
      nrow = *reinterpret_cast<const uint4*>((lane < T::CPR ? kn : vn) + c * 16);
      new_gather = __builtin_amdgcn_readlane((int)sel, t_new - kv0) == (int)kNewTok;
    }
    if (q_pending || slot_pending) {
      __builtin_amdgcn_sched_barrier(0);
      if (q_pending) eng.load_q_tile(0, qrow, l16 < G);
      if (slot_pending) {
        new_dst = (int64_t)slot_raw;
        new_ok = (uint64_t)new_dst < (uint64_t)a.num_pages;
      }
      __builtin_amdgcn_sched_barrier(0);
      q_pending = slot_pending = false;
    }
    if (rope_pending) {
      // The rotation inputs go out right behind the sub-tile's loads and
      // are waited for with them: the scheduling barriers keep the
      // compiler from hoisting them above the page-id loads (the in-order
      // load counter would then hold the page ids behind the table loads)
      // or sinking them below the wait (a second round trip).
      __builtin_amdgcn_sched_barrier(0);
      const int64_t rrow = min(max((int64_t)pos_raw, (int64_t)0), a.rope_rows - 1);
      rp.load(qrow0, reinterpret_cast<const bf16*>(kn), a.q_norm, a.k_norm,
              a.rope_cos + rrow * D, a.rope_sin + rrow * D);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();
    if (rope_pending) {
      rp.finish(stage, a.norm_eps);
      // (the wavefront's own LDS writes, read back in order)
#pragma unroll
      for (int s = 0; s < D / 32; ++s) {
        const bf16x8 f =
            *reinterpret_cast<const bf16x8*>(stage + (min(l16, G - 1) * D + s * 32 + lg * 8) * 2);
        eng.qf[0][s] = l16 < G ? f : bf16x8{};
      }
      rope_pending = false;
    }
    if (new_sub) {
      // The rotated K row stays in the staging area (every wavefront
      // rotated it with its query rows); the raw rows came with the
      // gathers.  K: the rotated row where the slot is in the pool, else
      // the raw row where the page id is; V: the raw row where the page id
      // is (otherwise the zero row stays), as a separate append and decode
      // would read them.  Both go to the slot's page now (no other
      // workgroup reads that page in this launch).
      const int tl = t_new - kv0;
      const bool krot = rope && new_ok;
      if (lane < T::CPR) {
        // (assigned under a branch: a conditional of two lvalues is a select
        // of their addresses, which put nrow in scratch)
        uint4 kv = nrow;
        if (krot) kv = *reinterpret_cast<const uint4*>(stage + (G * D + lane * 8) * 2);
        if (krot || new_gather)
          *reinterpret_cast<uint4*>(buf + tl * T::ROWB + T::k_slot(tl, lane) * 16) = kv;
        if (new_ok)
          *reinterpret_cast<uint4*>(const_cast<uint8_t*>(kc) + new_dst * tok_b + lane * 16) = kv;
      }
      if (lane >= T::CPR && lane < 2 * T::CPR) {
        const int c = lane - T::CPR;
        if (new_gather)
          *reinterpret_cast<uint4*>(buf + T::SUB_KB + tl * T::ROWB + T::v_slot(tl, c) * 16) = nrow;
        if (new_ok)
          *reinterpret_cast<uint4*>(const_cast<uint8_t*>(vc) + new_dst * tok_b + c * 16) = nrow;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    eng.compute(buf, kv0, s_end, a.scale_log2, l16, lg);
  }
  eng.finish();

  // Write the G x D rows o / l of one state: staged in LDS (the caller's
  // free region) in the order of the destination, then full-width 16-byte
  // stores (one store instruction per 64 chunks instead of one per 16-dim
  // tile from the G active lanes).  final: bf16 output rows; otherwise part
  // `part` of the parts array and its lse.
  auto write_rows = [&](const f32x4 (&acc)[DT], float l_tot, float m, uint8_t* stage_buf,
                        int part, bool final) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    bf16* srows = reinterpret_cast<bf16*>(stage_buf);
    if (l16 < G) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4 v = acc[dt] * inv;
        const int e = final ? l16 * D + dt * 16 + lg * 4 : (dt * G + l16) * 16 + lg * 4;
        *reinterpret_cast<uint2*>(srows + e) = make_uint2(pack_bf16x2(v[0], v[1]),
                                                         pack_bf16x2(v[2], v[3]));
      }
    }
    // The same wavefront reads the staged rows back: its LDS accesses
    // complete in order.
    constexpr int NCH = G * D / 8;  // 16-byte chunks of the rows
    for (int c = lane; c < NCH; c += 64) {
      const uint4 v = reinterpret_cast<const uint4*>(srows)[c];
      bf16* dst;
      if (final) {
        dst = a.out + ((int64_t)b * a.num_qo_heads + h * G) * D + c * 8;
      } else {
        const int dt = c * 8 / (G * 16);
        const int r = c * 8 - dt * G * 16;
        dst = a.parts.o + a.parts.o_index(D, h, part, b * G + r / 16, dt * 16 + (r & 15));
      }
      *reinterpret_cast<uint4*>(dst) = v;
    }
    if (!final && lg == 0 && l16 < G)
      a.parts.lse[a.parts.lse_index(h, part, b * G + l16)] =
          l_tot > 0.f ? m + fast_log2(l_tot) : kNegInf;
  };

  if (a.wave_parts) {
    // One part per wavefront (a wavefront without positions writes an empty
    // part, l = 0): no merge, no waiting for the slowest wavefront.
    write_rows(eng.o[0], eng.l_run[0], eng.m_run[0], buf, a.parts.n_chunks + split * NW + wave,
               false);
    return;
  }

  // Merge the four wavefronts' states (o relative to each wave's reference
  // m, row totals l) through LDS.
  f32x4* so = reinterpret_cast<f32x4*>(buf);
  float* sm = reinterpret_cast<float*>(buf + DT * 64 * 16);
  float* sl = sm + 16;
  if (wave > 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) so[dt * 64 + lane] = eng.o[0][dt];
    if (lg == 0) {
      sm[l16] = eng.m_run[0];
      sl[l16] = eng.l_run[0];
    }
  }
  __syncthreads();
  if (wave > 0) return;
  float mw[NW], lw[NW];
  mw[0] = eng.m_run[0];
  lw[0] = eng.l_run[0];
  float mx = mw[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    const float* smw = reinterpret_cast<const float*>(lds + w * T::SUB_BYTES + DT * 64 * 16);
    mw[w] = smw[l16];
    lw[w] = smw[16 + l16];
    mx = fmaxf(mx, mw[w]);
  }
  float f[NW];
  float l_tot = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    f[w] = (mw[w] == kNegInf) ? 0.f : fast_exp2(mw[w] - mx);
    l_tot += lw[w] * f[w];
  }
  f32x4 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    acc[dt] = eng.o[0][dt] * f[0];
#pragma unroll
    for (int w = 1; w < NW; ++w)
      acc[dt] += reinterpret_cast<const f32x4*>(lds + w * T::SUB_BYTES)[dt * 64 + lane] * f[w];
  }

  write_rows(acc, l_tot, mx, lds, a.parts.n_chunks + split, a.final_out != 0);
}

// The fields every workgroup needs before its first memory access lead the
// kernel arguments as scalars: compiled with kernel-argument preloading they
// arrive in SGPRs at wave start (the by-value DecodeArgs cannot be
// preloaded, and loading it is a memory round trip ahead of the page-id
// loads).  The copies inside DecodeArgs are overridden with them.
// splits_flags carries n_splits (below 2^16: the planner bounds the parts
// of a row at 64; the launch checks it) in its low 16 bits and
// the suffix items' two output flags above them (final_out: bit 16,
// wave_parts: bit 17): read only at the end, they were otherwise loaded
// beside the row bounds, and a scalar load's wait covers every scalar load
// in flight (they complete out of order), so they added a round trip ahead
// of the page ids.
struct DecodeHot {
  const int32_t* indices;
  const int32_t* cu_k;
  const int32_t* out_loc;  // null: no fused append
  int32_t prefix_wgs, prefix_len, chunk_len, m_groups, num_kv_heads, splits_flags, split_len,
      m_rows;
};
__host__ __device__ inline DecodeHot decode_hot(const DecodeArgs& a) {
  const int32_t sf = a.n_splits | (a.final_out ? 1 << 16 : 0) | (a.wave_parts ? 1 << 17 : 0);
  return DecodeHot{a.indices,  a.cu_k,         a.out_loc, a.prefix_wgs, a.prefix_len, a.chunk_len,
                   a.m_groups, a.num_kv_heads, sf,        a.split_len,  a.m_rows};
}

template <int D, int G, bool ROPE>
__global__ __launch_bounds__(kEngineThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_main_kernel(
    const int32_t* __restrict__ indices, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ out_loc, int32_t prefix_wgs,
    int32_t prefix_len, int32_t chunk_len, int32_t m_groups, int32_t num_kv_heads,
    int32_t splits_flags, int32_t split_len, int32_t m_rows, DecodeArgs args) {
  __shared__ __align__(16) uint8_t lds[decode_lds_bytes<D, G>()];
  DecodeArgs a = args;
  a.indices = indices;
  a.cu_k = cu_k;
  a.out_loc = out_loc;
  a.prefix_wgs = prefix_wgs;
  a.prefix_len = prefix_len;
  a.chunk_len = chunk_len;
  a.m_groups = m_groups;
  a.num_kv_heads = num_kv_heads;
  a.n_splits = splits_flags & 0xffff;
  a.final_out = (splits_flags >> 16) & 1;
  a.wave_parts = (splits_flags >> 17) & 1;
  a.split_len = split_len;
  a.m_rows = m_rows;
  // Prefix workgroups first: they carry most of the bytes, and dispatching
  // the suffix items ahead of them measured slower (their loads delay the
  // prefix streaming more than the suffix items gain).
  const int wg = blockIdx.x;
  if (wg < a.prefix_wgs) {
    decode_prefix_part<D, G, ROPE>(lds, a, wg);
  } else {
    decode_suffix_item<D, G, ROPE>(lds, a, wg - a.prefix_wgs);
  }
}

bool head_dim_supported(int D) { return D == 64 || D == 96 || D == 128; }
bool group_supported(int G) {
  return G == 1 || G == 2 || G == 3 || G == 4 || G == 6 || G == 8;
}

template <int D, int G>
static hipError_t launch_main_dg(const DecodeArgs& a, hipStream_t s) {
  const int suffix_wgs = a.suffix_items;
  const dim3 grid(a.prefix_wgs + suffix_wgs);
  if (grid.x == 0) return hipSuccess;
  if (a.n_splits < 1 || a.n_splits >= (1 << 16)) return hipErrorInvalidValue;
  const DecodeHot h = decode_hot(a);
  if (a.q_norm != nullptr)
    hipLaunchKernelGGL((decode_main_kernel<D, G, true>), grid, dim3(kEngineThreads), 0, s,
                       h.indices, h.cu_k, h.out_loc, h.prefix_wgs, h.prefix_len, h.chunk_len,
                       h.m_groups,
                       h.num_kv_heads, h.splits_flags, h.split_len, h.m_rows, a);
  else
    hipLaunchKernelGGL((decode_main_kernel<D, G, false>), grid, dim3(kEngineThreads), 0, s,
                       h.indices, h.cu_k, h.out_loc, h.prefix_wgs, h.prefix_len, h.chunk_len,
                       h.m_groups,
                       h.num_kv_heads, h.splits_flags, h.split_len, h.m_rows, a);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_main_d(const DecodeArgs& a, hipStream_t s) {
  switch (a.group) {
    case 1: return launch_main_dg<D, 1>(a, s);
    case 2: return launch_main_dg<D, 2>(a, s);
    case 3: return launch_main_dg<D, 3>(a, s);
    case 4: return launch_main_dg<D, 4>(a, s);
    case 6: return launch_main_dg<D, 6>(a, s);
    case 8: return launch_main_dg<D, 8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_main(int D, const DecodeArgs& a, hipStream_t s) {
  switch (D) {
    case 64: return launch_main_d<64>(a, s);
    case 96: return launch_main_d<96>(a, s);
    case 128: return launch_main_d<128>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aios
