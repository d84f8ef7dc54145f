// C ABI of the attention backend: validation, host-side planning and launch.
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/aios_attn.h"
#include "kernels.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return AIOS_OK;
  return fail(AIOS_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

int32_t cdiv(int32_t a, int32_t b) { return (a + b - 1) / b; }

// Shared prefixes shorter than this are read per row (no second launch).
constexpr int32_t kMinCascadePrefix = 256;
// Partial states per (row, kv-head) the combine merges (one per lane of a
// wavefront when it computes the merge weights).
constexpr int32_t kMaxParts = 64;

// Compute units of the current device, looked up once per process (host
// query only; no device synchronisation).
int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

}  // namespace

extern "C" {

const char* aios_last_error(void) { return g_err; }

const char* aios_version(void) { return "aios-mi355x-attn 0.1 gfx950"; }

int aios_kv_append(void* k_cache, void* v_cache, int64_t num_slots, int64_t cache_tok_stride,
                   const int32_t* out_loc, const void* k, int64_t k_tok_stride, const void* v,
                   int64_t v_tok_stride, int64_t n_tokens, int64_t width, int32_t elem_bytes,
                   void* stream) {
  if (n_tokens < 0 || width <= 0 || num_slots < 0)
    return fail(AIOS_ERR_INVALID, "kv_append: bad sizes (n_tokens=%lld width=%lld)",
                (long long)n_tokens, (long long)width);
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return fail(AIOS_ERR_UNSUPPORTED, "kv_append: elem_bytes %d", elem_bytes);
  if (cache_tok_stride < width || k_tok_stride < 0 || v_tok_stride < 0)
    return fail(AIOS_ERR_INVALID, "kv_append: stride smaller than row width");
  if (n_tokens == 0) return AIOS_OK;
  if (!k_cache || !v_cache || !out_loc || !k || !v)
    return fail(AIOS_ERR_INVALID, "kv_append: null pointer");
  const hipError_t e = aios::kv_append(
      k_cache, v_cache, num_slots, cache_tok_stride * elem_bytes, out_loc, k,
      k_tok_stride * elem_bytes, v, v_tok_stride * elem_bytes, n_tokens, width * elem_bytes,
      static_cast<hipStream_t>(stream));
  return check_hip(e, "kv_append launch");
}

int aios_attn_plan(int32_t phase, const int32_t* cu_q, const int32_t* cu_k, int32_t batch,
                   int32_t hq, int32_t hkv, int32_t d, int32_t page_size, int32_t shared_prefix,
                   int64_t ws_bytes, int32_t prefix_chunk_len, int32_t suffix_split_len,
                   aios_attn_plan_t* p) {
  if (!p) return fail(AIOS_ERR_INVALID, "plan: null plan");
  memset(p, 0, sizeof(*p));
  if (phase != AIOS_PHASE_PREFILL && phase != AIOS_PHASE_DECODE)
    return fail(AIOS_ERR_INVALID, "plan: unknown phase %d", phase);
  if (page_size != 1) return fail(AIOS_ERR_UNSUPPORTED, "plan: only page_size=1 is supported");
  if (batch < 0 || !cu_q || !cu_k) return fail(AIOS_ERR_INVALID, "plan: bad batch arrays");
  if (hq <= 0 || hkv <= 0 || d <= 0)
    return fail(AIOS_ERR_INVALID, "plan: head counts and head_dim must be positive");
  if (hq % hkv) return fail(AIOS_ERR_INVALID, "query head count must be divisible by KV head count");
  const int32_t G = hq / hkv;
  if (!aios::head_dim_supported(d) || !aios::group_supported(G))
    return fail(AIOS_ERR_UNSUPPORTED, "plan: head_dim %d with group %d is not built", d, G);
  if (cu_q[0] != 0 || cu_k[0] != 0) return fail(AIOS_ERR_INVALID, "plan: cu_seqlens must start at 0");
  int32_t max_q = 0, max_kv = 0, min_kv = 0x7fffffff;
  for (int32_t b = 0; b < batch; ++b) {
    const int32_t ql = cu_q[b + 1] - cu_q[b];
    const int32_t kl = cu_k[b + 1] - cu_k[b];
    if (ql < 0 || kl < 0) return fail(AIOS_ERR_INVALID, "plan: cu_seqlens must be non-decreasing");
    if (kl < ql) return fail(AIOS_ERR_INVALID, "cached_len + query length must equal KV length");
    if (phase == AIOS_PHASE_DECODE && ql != 1)
      return fail(AIOS_ERR_INVALID, "decode batch must contain one flat token per request");
    if (ql > max_q) max_q = ql;
    if (kl > max_kv) max_kv = kl;
    if (kl < min_kv) min_kv = kl;
  }
  if (batch == 0) min_kv = 0;
  p->phase = phase;
  p->batch_size = batch;
  p->num_qo_heads = hq;
  p->num_kv_heads = hkv;
  p->head_dim = d;
  p->group = G;
  p->total_q = cu_q[batch];
  p->total_kv = cu_k[batch];
  p->max_q_len = max_q;
  p->max_kv_len = max_kv;
  p->min_kv_len = min_kv;
  const int cus = device_cus();

  if (phase == AIOS_PHASE_PREFILL) {
    // 128 MFMA rows per workgroup = q_tile tokens x G heads.
    const int32_t q_tile = 128 / G;
    p->prefill_q_tile = q_tile;
    p->num_q_tiles = max_q > 0 ? cdiv(max_q, q_tile) : 0;
    return AIOS_OK;
  }

  // ---- decode ----------------------------------------------------------------
  if (shared_prefix < 0 || shared_prefix > min_kv)
    return fail(AIOS_ERR_INVALID,
                "plan: shared_prefix_len %d exceeds the shortest row (%d KV positions)",
                shared_prefix, min_kv);
  const int32_t m_rows = batch * G;
  // Reading the prefix once per kv-head pays off when the prefix is long
  // enough to amortise a second launch and the group fills an MFMA tile;
  // a positive prefix_chunk_len forces it.
  const bool cascade = shared_prefix > 0 && batch > 1 && m_rows >= 16 &&
                       (prefix_chunk_len > 0 || shared_prefix >= kMinCascadePrefix);
  const int32_t P = cascade ? shared_prefix : 0;
  int32_t chunk = 0, n_chunks = 0, mgroups = 0;
  if (cascade) {
    mgroups = cdiv(m_rows, 128);
    if (prefix_chunk_len > 0) {
      chunk = (int32_t)align_up(prefix_chunk_len, 32);
    } else {
      // About one prefix workgroup per compute unit.
      int32_t want = cdiv(cus, hkv * mgroups);
      if (want < 1) want = 1;
      chunk = (int32_t)align_up(cdiv(P, want), 32);
    }
    n_chunks = cdiv(P, chunk);
  }
  const int32_t max_suffix = max_kv - P;
  const int32_t pass = aios::kSuffixPass;  // KV positions one suffix workgroup loads at once
  const int32_t tpg = pass / 4;             // per wavefront
  int32_t split;
  if (suffix_split_len > 0) {
    split = suffix_split_len;
  } else if (!cascade && max_suffix <= 2 * pass) {
    split = max_suffix > 0 ? max_suffix : 1;  // one item covers the whole row
  } else {
    split = pass;
  }
  int32_t n_splits = max_suffix > 0 ? cdiv(max_suffix, split) : 1;
  // Bound the parts per (row, kv-head) merged by the combine.
  while (n_chunks + n_splits > kMaxParts) {
    if (n_splits > n_chunks) {
      split *= 2;
      n_splits = max_suffix > 0 ? cdiv(max_suffix, split) : 1;
    } else {
      chunk = (int32_t)align_up((int64_t)chunk * 2, 32);
      n_chunks = cdiv(P, chunk);
    }
  }
  // With the cascade the combine runs anyway: each suffix wavefront then
  // writes its own part instead of merging the item's four states through
  // LDS first (the merge waits for the slowest wavefront and then runs on
  // one), as long as the part count stays within the bound.
  const int32_t per_item =
      (cascade && n_chunks + n_splits * aios::kSuffixWaves <= kMaxParts) ? aios::kSuffixWaves : 1;
  const int32_t n_parts = n_chunks + n_splits * per_item;
  p->suffix_parts_per_item = per_item;
  p->prefix_len = P;
  p->prefix_chunk_len = chunk;
  p->num_prefix_chunks = n_chunks;
  p->cascade_rows = m_rows;
  p->cascade_mgroups = mgroups;
  p->suffix_split_len = split;
  p->num_suffix_splits = n_splits;
  p->suffix_tpg = tpg;
  p->num_parts = n_parts;
  if (n_parts > 1) {
    p->ws_parts_o = 0;
    p->ws_parts_lse = align_up((int64_t)batch * hkv * n_parts * G * d * 2, 256);
    p->ws_bytes = p->ws_parts_lse + align_up((int64_t)batch * hkv * n_parts * G * 4, 256);
  }
  if (p->ws_bytes > ws_bytes)
    return fail(AIOS_ERR_WORKSPACE, "plan: workspace of %lld bytes is smaller than the %lld needed",
                (long long)ws_bytes, (long long)p->ws_bytes);
  return AIOS_OK;
}

static int check_plan(const aios_attn_plan_t* p, int phase) {
  if (!p) return fail(AIOS_ERR_INVALID, "null plan");
  if (p->phase != phase)
    return fail(AIOS_ERR_INVALID, "plan phase %d does not match the call", p->phase);
  if (!aios::head_dim_supported(p->head_dim) || !aios::group_supported(p->group))
    return fail(AIOS_ERR_UNSUPPORTED, "plan: unsupported head_dim/group");
  return AIOS_OK;
}

// The attention kernels address one layer's K (or V) cache with 32-bit byte
// offsets (buffer descriptors), so a layer's cache must stay below 4 GiB,
// and form a page's offset with a 24-bit multiply, so the pool holds fewer
// than 2^24 pages.
static int check_cache(int64_t kv_num_pages, int64_t tok_stride) {
  if (kv_num_pages < 0) return fail(AIOS_ERR_INVALID, "negative page count");
  if (kv_num_pages >= (1ll << 24))
    return fail(AIOS_ERR_UNSUPPORTED, "a pool of %lld pages exceeds the 2^24 - 1 the kernels address",
                (long long)kv_num_pages);
  const int64_t bytes = kv_num_pages * tok_stride * 2;
  if (bytes > 0xffff0000ll)
    return fail(AIOS_ERR_UNSUPPORTED,
                "per-layer KV cache of %lld bytes exceeds the 4 GiB the kernels address",
                (long long)bytes);
  return AIOS_OK;
}

int aios_attn_prefill(const aios_attn_plan_t* p, const void* q, int64_t q_tok_stride,
                      const void* k_cache, const void* v_cache, int64_t kv_num_pages,
                      const int32_t* indices, const int32_t* cu_q, const int32_t* cu_k, void* out,
                      float sm_scale, void* stream) {
  int rc = check_plan(p, AIOS_PHASE_PREFILL);
  if (rc) return rc;
  if (p->batch_size == 0 || p->total_q == 0) return AIOS_OK;
  const int D = p->head_dim;
  if (q_tok_stride < (int64_t)p->num_qo_heads * D || (q_tok_stride % 8) != 0)
    return fail(AIOS_ERR_INVALID, "prefill: q token stride %lld must be >= Hq*D and a multiple of 8",
                (long long)q_tok_stride);
  if (!q || !k_cache || !v_cache || !indices || !cu_q || !cu_k || !out)
    return fail(AIOS_ERR_INVALID, "prefill: null pointer");
  if ((((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15) != 0)
    return fail(AIOS_ERR_INVALID, "prefill: q, caches and out must be 16-byte aligned");
  if ((rc = check_cache(kv_num_pages, (int64_t)p->num_kv_heads * D))) return rc;
  aios::PrefillArgs a = {};
  a.q = static_cast<const aios::bf16*>(q);
  a.q_tok_stride = q_tok_stride;
  a.k_cache = static_cast<const aios::bf16*>(k_cache);
  a.v_cache = static_cast<const aios::bf16*>(v_cache);
  a.kv_tok_stride = (int64_t)p->num_kv_heads * D;
  a.num_pages = kv_num_pages;
  a.indices = indices;
  a.cu_q = cu_q;
  a.cu_k = cu_k;
  a.num_qo_heads = p->num_qo_heads;
  a.num_kv_heads = p->num_kv_heads;
  a.group = p->group;
  a.scale_log2 = sm_scale * aios::kLog2e;
  a.q_tile = p->prefill_q_tile;
  a.q_tiles = p->num_q_tiles;
  a.batch = p->batch_size;
  a.out = static_cast<aios::bf16*>(out);
  return check_hip(aios::launch_prefill(D, 4, a, p->num_q_tiles, p->batch_size,
                                        static_cast<hipStream_t>(stream)),
                   "prefill launch");
}

}  // extern "C"

namespace {

struct NewKV {
  const void* k;
  int64_t k_stride;
  const void* v;
  int64_t v_stride;
  const int32_t* out_loc;
};

// Per-head q / k RMSNorm + RoPE applied on load (aios_attn_append_decode_rope).
struct QkRopeIn {
  const void* q_norm;
  const void* k_norm;
  const void* cos;
  const void* sin;
  int64_t rows;
  const int32_t* positions;
  float eps;
};

int decode_impl(const aios_attn_plan_t* p, const void* q, int64_t q_tok_stride,
                const void* k_cache, const void* v_cache, int64_t kv_num_pages,
                const int32_t* indices, const int32_t* cu_k, void* out, void* workspace,
                int64_t workspace_bytes, float sm_scale, void* stream, const NewKV* nk,
                const QkRopeIn* ro = nullptr) {
  int rc = check_plan(p, AIOS_PHASE_DECODE);
  if (rc) return rc;
  if (p->batch_size == 0) return AIOS_OK;
  const int D = p->head_dim;
  if (q_tok_stride < (int64_t)p->num_qo_heads * D || (q_tok_stride % 8) != 0)
    return fail(AIOS_ERR_INVALID, "decode: q token stride %lld must be >= Hq*D and a multiple of 8",
                (long long)q_tok_stride);
  if (p->ws_bytes > workspace_bytes || (p->ws_bytes > 0 && !workspace))
    return fail(AIOS_ERR_WORKSPACE, "decode: workspace of %lld bytes is smaller than the %lld needed",
                (long long)workspace_bytes, (long long)p->ws_bytes);
  if (((uintptr_t)workspace & 255) != 0)
    return fail(AIOS_ERR_INVALID, "decode: workspace must be 256-byte aligned");
  if (!q || !k_cache || !v_cache || !indices || !cu_k || !out)
    return fail(AIOS_ERR_INVALID, "decode: null pointer");
  if ((((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15) != 0)
    return fail(AIOS_ERR_INVALID, "decode: q, caches and out must be 16-byte aligned");
  if ((rc = check_cache(kv_num_pages, (int64_t)p->num_kv_heads * D))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int32_t mask = p->stage_mask == 0 ? 3 : p->stage_mask;

  aios::DecodeArgs a = {};
  a.q = static_cast<const aios::bf16*>(q);
  a.q_tok_stride = q_tok_stride;
  a.k_cache = static_cast<const aios::bf16*>(k_cache);
  a.v_cache = static_cast<const aios::bf16*>(v_cache);
  a.kv_tok_stride = (int64_t)p->num_kv_heads * D;
  a.num_pages = kv_num_pages;
  a.indices = indices;
  a.cu_k = cu_k;
  a.batch = p->batch_size;
  a.num_qo_heads = p->num_qo_heads;
  a.num_kv_heads = p->num_kv_heads;
  a.group = p->group;
  a.scale_log2 = sm_scale * aios::kLog2e;
  a.prefix_len = p->prefix_len;
  a.chunk_len = p->prefix_chunk_len;
  a.n_chunks = p->num_prefix_chunks;
  a.m_rows = p->cascade_rows;
  a.m_groups = p->cascade_mgroups > 0 ? p->cascade_mgroups : 1;
  a.prefix_wgs = p->num_prefix_chunks * p->num_kv_heads * a.m_groups;
  a.split_len = p->suffix_split_len;
  a.n_splits = p->num_suffix_splits;
  a.suffix_items = p->batch_size * p->num_kv_heads * p->num_suffix_splits;
  a.final_out = p->num_parts == 1 ? 1 : 0;
  a.wave_parts = p->suffix_parts_per_item > 1 ? 1 : 0;
  a.parts.o = reinterpret_cast<aios::bf16*>(ws + p->ws_parts_o);
  a.parts.lse = reinterpret_cast<float*>(ws + p->ws_parts_lse);
  a.parts.n_parts = p->num_parts;
  a.parts.n_chunks = p->num_prefix_chunks;
  a.parts.rows = p->batch_size * p->group;
  a.out = static_cast<aios::bf16*>(out);
  if (nk) {
    if (!nk->k || !nk->v || !nk->out_loc)
      return fail(AIOS_ERR_INVALID, "append_decode: null pointer");
    if (nk->k_stride < a.kv_tok_stride || nk->v_stride < a.kv_tok_stride ||
        (nk->k_stride % 8) != 0 || (nk->v_stride % 8) != 0)
      return fail(AIOS_ERR_INVALID,
                  "append_decode: K/V token strides must be >= Hkv*D and multiples of 8");
    const int E = D / 16;
    const uintptr_t align = E == 8 ? 16 : (E == 4 ? 8 : 4);
    if (((uintptr_t)nk->k % align) != 0 || ((uintptr_t)nk->v % align) != 0)
      return fail(AIOS_ERR_INVALID, "append_decode: K/V rows must be %d-byte aligned", (int)align);
    if (p->min_kv_len < 1 || p->prefix_len >= p->min_kv_len)
      return fail(AIOS_ERR_INVALID,
                  "append_decode: every row's new token must lie after the shared prefix");
    a.k_new = static_cast<const aios::bf16*>(nk->k);
    a.v_new = static_cast<const aios::bf16*>(nk->v);
    a.k_new_stride = nk->k_stride;
    a.v_new_stride = nk->v_stride;
    a.out_loc = nk->out_loc;
  }
  if (ro) {
    if (!nk) return fail(AIOS_ERR_INVALID, "append_decode_rope: the rotation needs the new K rows");
    if (!ro->q_norm || !ro->k_norm || !ro->cos || !ro->sin || !ro->positions)
      return fail(AIOS_ERR_INVALID, "append_decode_rope: null pointer");
    if (ro->rows < 1) return fail(AIOS_ERR_INVALID, "append_decode_rope: empty rotation table");
    if ((((uintptr_t)ro->q_norm | (uintptr_t)ro->k_norm | (uintptr_t)ro->cos |
          (uintptr_t)ro->sin | (uintptr_t)nk->k) & 15) != 0)
      return fail(AIOS_ERR_INVALID,
                  "append_decode_rope: norm weights, tables and K rows must be 16-byte aligned");
    a.q_norm = static_cast<const aios::bf16*>(ro->q_norm);
    a.k_norm = static_cast<const aios::bf16*>(ro->k_norm);
    a.rope_cos = static_cast<const aios::bf16*>(ro->cos);
    a.rope_sin = static_cast<const aios::bf16*>(ro->sin);
    a.rope_rows = ro->rows;
    a.positions = ro->positions;
    a.norm_eps = ro->eps;
  }
  if (mask & 1) {
    rc = check_hip(aios::launch_decode_main(D, a, s), "decode launch");
    if (rc) return rc;
  }
  if (p->num_parts > 1 && (mask & 2))
    return check_hip(aios::launch_decode_combine(D, a, s), "combine launch");
  return AIOS_OK;
}

}  // namespace

extern "C" {

int aios_attn_decode(const aios_attn_plan_t* p, const void* q, int64_t q_tok_stride,
                     const void* k_cache, const void* v_cache, int64_t kv_num_pages,
                     const int32_t* indices, const int32_t* cu_k, void* out, void* workspace,
                     int64_t workspace_bytes, float sm_scale, void* stream) {
  return decode_impl(p, q, q_tok_stride, k_cache, v_cache, kv_num_pages, indices, cu_k, out,
                     workspace, workspace_bytes, sm_scale, stream, nullptr);
}

int aios_attn_append_decode(const aios_attn_plan_t* p, const void* q, int64_t q_tok_stride,
                            const void* k_new, int64_t k_tok_stride, const void* v_new,
                            int64_t v_tok_stride, const int32_t* out_loc, void* k_cache,
                            void* v_cache, int64_t kv_num_pages, const int32_t* indices,
                            const int32_t* cu_k, void* out, void* workspace,
                            int64_t workspace_bytes, float sm_scale, void* stream) {
  const NewKV nk = {k_new, k_tok_stride, v_new, v_tok_stride, out_loc};
  return decode_impl(p, q, q_tok_stride, k_cache, v_cache, kv_num_pages, indices, cu_k, out,
                     workspace, workspace_bytes, sm_scale, stream, &nk);
}

int aios_attn_append_decode_rope(const aios_attn_plan_t* p, const void* q, int64_t q_tok_stride,
                                 const void* k_new, int64_t k_tok_stride, const void* v_new,
                                 int64_t v_tok_stride, const int32_t* out_loc, void* k_cache,
                                 void* v_cache, int64_t kv_num_pages, const int32_t* indices,
                                 const int32_t* cu_k, const void* q_norm, const void* k_norm,
                                 const void* rope_cos, const void* rope_sin, int64_t rope_rows,
                                 const int32_t* positions, float norm_eps, void* out,
                                 void* workspace, int64_t workspace_bytes, float sm_scale,
                                 void* stream) {
  const NewKV nk = {k_new, k_tok_stride, v_new, v_tok_stride, out_loc};
  const QkRopeIn ro = {q_norm, k_norm, rope_cos, rope_sin, rope_rows, positions, norm_eps};
  return decode_impl(p, q, q_tok_stride, k_cache, v_cache, kv_num_pages, indices, cu_k, out,
                     workspace, workspace_bytes, sm_scale, stream, &nk, &ro);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free decode.  The partial softmax states live in this file-scope
// device array instead of a caller workspace: every GPU the library runs on
// holds its own copy until the process ends.  Host code never uses the
// array's name as an address (on the host it is only a stand-in); the
// device address of the current GPU's copy is looked up once per device with
// hipGetSymbolAddress and passed to the kernels like a workspace.
constexpr int64_t kNoAllocScratchBytes = AIOS_DECODE_NOALLOC_MAX_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address (looked up on its first use there).
// The stream must belong to the current device.
int scratch_for(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return check_hip(e, "decode_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(AIOS_ERR_UNSUPPORTED, "decode_noalloc: device %d beyond the %d supported", dev,
                kMaxDevices);
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return check_hip(e, "decode_noalloc: hipStreamGetDevice");
    if (sdev != dev)
      return fail(AIOS_ERR_INVALID, "decode_noalloc: stream of device %d, current device %d",
                  sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return check_hip(e, "decode_noalloc: hipGetSymbolAddress(scratch)");
    if (!p || ((uintptr_t)p & 255) != 0)
      return fail(AIOS_ERR_LAUNCH, "decode_noalloc: scratch address %p not 256-byte aligned", p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AIOS_OK;
}

}  // namespace

extern "C" {

int aios_attn_decode_noalloc(const aios_attn_plan_t* p, const void* q, int64_t q_tok_stride,
                             const void* k_cache, const void* v_cache, int64_t kv_num_pages,
                             const int32_t* indices, const int32_t* cu_k, void* out,
                             float sm_scale, void* stream) {
  int rc = check_plan(p, AIOS_PHASE_DECODE);
  if (rc) return rc;
  if (p->ws_bytes > kNoAllocScratchBytes)
    return fail(AIOS_ERR_WORKSPACE,
                "decode_noalloc: the batch needs %lld bytes of partial states, above the %lld "
                "of the built-in scratch (use aios_attn_decode with a workspace)",
                (long long)p->ws_bytes, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_for(stream, &ws))) return rc;
  return decode_impl(p, q, q_tok_stride, k_cache, v_cache, kv_num_pages, indices, cu_k, out, ws,
                     kNoAllocScratchBytes, sm_scale, stream, nullptr);
}

int aios_build_indices(const int32_t* page_table, int64_t page_table_stride,
                       const int32_t* row_ids, const int32_t* cu_k, int32_t batch,
                       int32_t total_kv, int32_t* indices_out, void* stream) {
  if (batch < 0 || total_kv < 0 || page_table_stride <= 0)
    return fail(AIOS_ERR_INVALID, "build_indices: bad sizes");
  if (batch == 0 || total_kv == 0) return AIOS_OK;
  if (!page_table || !row_ids || !cu_k || !indices_out)
    return fail(AIOS_ERR_INVALID, "build_indices: null pointer");
  return check_hip(aios::build_indices(page_table, page_table_stride, row_ids, cu_k, batch,
                                       total_kv, indices_out, static_cast<hipStream_t>(stream)),
                   "build_indices launch");
}

int aios_rmsnorm(const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
                 const void* weight, void* out, int64_t out_stride, int64_t rows, int32_t hidden,
                 float eps, void* stream) {
  if (rows < 0 || !aios::rmsnorm_supported(hidden))
    return fail(AIOS_ERR_INVALID, "rmsnorm: hidden %d must be a multiple of 8 up to 8192", hidden);
  if (rows == 0) return AIOS_OK;
  if (!x || !weight || !out) return fail(AIOS_ERR_INVALID, "rmsnorm: null pointer");
  if (x_stride < hidden || out_stride < hidden || (residual && residual_stride < hidden) ||
      (x_stride | out_stride | (residual ? residual_stride : 0)) % 8 != 0)
    return fail(AIOS_ERR_INVALID, "rmsnorm: row strides must be >= hidden and multiples of 8");
  if ((((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)residual) & 15) != 0)
    return fail(AIOS_ERR_INVALID, "rmsnorm: rows must be 16-byte aligned");
  return check_hip(aios::rmsnorm(x, x_stride, residual, residual_stride, weight, out, out_stride,
                                 rows, hidden, eps, static_cast<hipStream_t>(stream)),
                   "rmsnorm launch");
}

int aios_qk_norm_rope(const void* qkv, int64_t qkv_stride, int64_t tokens, int32_t num_qo_heads,
                      int32_t num_kv_heads, int32_t head_dim, const void* q_weight,
                      const void* k_weight, const float* cos_table, const float* sin_table,
                      int64_t table_rows, const int32_t* positions, void* q_out, void* k_out,
                      float eps, void* stream) {
  if (tokens < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || table_rows <= 0)
    return fail(AIOS_ERR_INVALID, "qk_norm_rope: bad sizes");
  if (!aios::head_dim_supported(head_dim))
    return fail(AIOS_ERR_UNSUPPORTED, "qk_norm_rope: head_dim %d is not built", head_dim);
  if (qkv_stride < (int64_t)(num_qo_heads + 2 * num_kv_heads) * head_dim || qkv_stride % 2 != 0)
    return fail(AIOS_ERR_INVALID, "qk_norm_rope: qkv row stride too small");
  if (tokens == 0) return AIOS_OK;
  if (!qkv || !q_weight || !k_weight || !cos_table || !sin_table || !positions || !q_out || !k_out)
    return fail(AIOS_ERR_INVALID, "qk_norm_rope: null pointer");
  if ((((uintptr_t)qkv | (uintptr_t)q_weight | (uintptr_t)k_weight) & 3) != 0)
    return fail(AIOS_ERR_INVALID, "qk_norm_rope: rows must be 4-byte aligned");
  return check_hip(aios::qk_norm_rope(qkv, qkv_stride, tokens, num_qo_heads, num_kv_heads, head_dim,
                                      q_weight, k_weight, cos_table, sin_table, table_rows,
                                      positions, q_out, k_out, eps,
                                      static_cast<hipStream_t>(stream)),
                   "qk_norm_rope launch");
}

int aios_silu_mul(const void* x, int64_t x_stride, int64_t rows, int32_t intermediate, void* out,
                  int64_t out_stride, void* stream) {
  if (rows < 0 || intermediate <= 0 || intermediate % 8 != 0)
    return fail(AIOS_ERR_INVALID, "silu_mul: intermediate size %d must be a multiple of 8",
                intermediate);
  if (x_stride < 2 * (int64_t)intermediate || out_stride < intermediate ||
      (x_stride | out_stride) % 8 != 0)
    return fail(AIOS_ERR_INVALID, "silu_mul: row strides too small or not multiples of 8");
  if (rows == 0) return AIOS_OK;
  if (!x || !out) return fail(AIOS_ERR_INVALID, "silu_mul: null pointer");
  if ((((uintptr_t)x | (uintptr_t)out) & 15) != 0)
    return fail(AIOS_ERR_INVALID, "silu_mul: rows must be 16-byte aligned");
  return check_hip(aios::silu_mul(x, x_stride, rows, intermediate, out, out_stride,
                                  static_cast<hipStream_t>(stream)),
                   "silu_mul launch");
}

int aios_linear_rows(const void* x, int64_t x_stride, const void* weight, int64_t w_stride,
                     void* y, int64_t y_stride, int64_t rows, int64_t out_features,
                     int64_t in_features, void* stream) {
  return aios_linear_rows_ex(x, x_stride, weight, w_stride, y, y_stride, rows, out_features,
                             in_features, AIOS_PROLOGUE_NONE, nullptr, 0, nullptr, 0.f, nullptr,
                             0, AIOS_EPILOGUE_NONE, stream);
}

int aios_linear_rows_ex(const void* x, int64_t x_stride, const void* weight, int64_t w_stride,
                        void* y, int64_t y_stride, int64_t rows, int64_t out_features,
                        int64_t in_features, int32_t prologue, const void* residual,
                        int64_t residual_stride, const void* norm_weight, float eps,
                        void* residual_out, int64_t residual_out_stride, int32_t epilogue,
                        void* stream) {
  if (!aios::skinny_gemm_supported(rows, out_features, in_features))
    return fail(AIOS_ERR_UNSUPPORTED,
                "linear_rows: needs 1..64 rows, out_features %% 16 == 0, in_features %% 128 == 0 "
                "(got %lld x %lld x %lld)",
                (long long)rows, (long long)out_features, (long long)in_features);
  if (prologue != AIOS_PROLOGUE_NONE && prologue != AIOS_PROLOGUE_ADD_RMSNORM)
    return fail(AIOS_ERR_INVALID, "linear_rows: unknown prologue %d", prologue);
  if (epilogue != AIOS_EPILOGUE_NONE && epilogue != AIOS_EPILOGUE_SILU_MUL)
    return fail(AIOS_ERR_INVALID, "linear_rows: unknown epilogue %d", epilogue);
  if (prologue == AIOS_PROLOGUE_ADD_RMSNORM && !aios::skinny_gemm_norm_supported(rows, in_features))
    return fail(AIOS_ERR_UNSUPPORTED, "linear_rows: RMSNorm prologue for %lld rows x %lld",
                (long long)rows, (long long)in_features);
  if (!x || !weight || !y) return fail(AIOS_ERR_INVALID, "linear_rows: null pointer");
  if (x_stride < in_features || w_stride < in_features || y_stride < out_features ||
      (x_stride | w_stride) % 8 != 0 || y_stride % 4 != 0)
    return fail(AIOS_ERR_INVALID, "linear_rows: bad row strides");
  if ((((uintptr_t)x | (uintptr_t)weight) & 15) != 0 || ((uintptr_t)y & 7) != 0)
    return fail(AIOS_ERR_INVALID, "linear_rows: misaligned rows");
  if (prologue == AIOS_PROLOGUE_ADD_RMSNORM) {
    if (!norm_weight || ((uintptr_t)norm_weight & 15) != 0)
      return fail(AIOS_ERR_INVALID, "linear_rows: norm weight missing or misaligned");
    if (residual && (residual_stride < in_features || residual_stride % 8 != 0 ||
                     ((uintptr_t)residual & 15) != 0))
      return fail(AIOS_ERR_INVALID, "linear_rows: bad residual rows");
    if (residual_out && (residual_out_stride < in_features || residual_out_stride % 8 != 0 ||
                         ((uintptr_t)residual_out & 15) != 0))
      return fail(AIOS_ERR_INVALID, "linear_rows: bad residual_out rows");
    if (residual_out && (residual_out == x || residual_out == residual))
      return fail(AIOS_ERR_INVALID, "linear_rows: residual_out must not alias the inputs");
  }
  aios::LinearArgs a = {};
  a.x = static_cast<const aios::bf16*>(x);
  a.x_stride = x_stride;
  a.w = static_cast<const aios::bf16*>(weight);
  a.w_stride = w_stride;
  a.y = static_cast<aios::bf16*>(y);
  a.y_stride = y_stride;
  a.M = (int32_t)rows;
  a.K = (int32_t)in_features;
  a.N = out_features;
  a.residual = static_cast<const aios::bf16*>(residual);
  a.r_stride = residual_stride;
  a.norm_w = static_cast<const aios::bf16*>(norm_weight);
  a.eps = eps;
  a.residual_out = static_cast<aios::bf16*>(residual_out);
  a.ro_stride = residual_out_stride;
  return check_hip(aios::skinny_gemm(a, prologue, epilogue, static_cast<hipStream_t>(stream)),
                   "linear_rows launch");
}

int aios_cg_step_begin(int64_t* step, const int32_t* pages, int32_t page_rows, int32_t rows,
                       int32_t* out_loc, int32_t* page_table, int64_t pt_stride, int32_t pt_cols,
                       int32_t* pos, void* stream) {
  if (rows <= 0 || page_rows <= 0 || pt_cols <= 0 || pt_stride < pt_cols)
    return fail(AIOS_ERR_INVALID, "cg_step_begin: bad sizes");
  if (!step || !pages || !out_loc || !page_table || !pos)
    return fail(AIOS_ERR_INVALID, "cg_step_begin: null pointer");
  aios::CgStepArgs a = {};
  a.rows = rows;
  a.step = step;
  a.pages = pages;
  a.page_rows = page_rows;
  a.out_loc = out_loc;
  a.page_table = page_table;
  a.pt_stride = pt_stride;
  a.pt_cols = pt_cols;
  a.pos = pos;
  return check_hip(aios::cg_step_begin(a, static_cast<hipStream_t>(stream)), "cg_step_begin launch");
}

int aios_cg_step_prepare(int64_t* step, const int32_t* pages, int32_t page_rows, int32_t rows,
                         int32_t* out_loc, int32_t* page_table, int64_t pt_stride, int32_t pt_cols,
                         int32_t* pos, int32_t* cu_k, int32_t* indices, int32_t max_kv_len,
                         int64_t* step_next, const int64_t* tokens, const void* embed,
                         int64_t vocab, int32_t hidden, void* h_out, void* stream) {
  if (rows <= 0 || page_rows <= 0 || pt_cols <= 0 || pt_stride < pt_cols)
    return fail(AIOS_ERR_INVALID, "cg_step_prepare: bad sizes");
  if (max_kv_len <= 0 || max_kv_len > pt_cols)
    return fail(AIOS_ERR_INVALID, "cg_step_prepare: max_kv_len %d outside [1, %d]", max_kv_len,
                pt_cols);
  if (!step || !pages || !out_loc || !page_table || !pos || !cu_k || !indices)
    return fail(AIOS_ERR_INVALID, "cg_step_prepare: null pointer");
  if (embed) {
    if (!tokens || !h_out) return fail(AIOS_ERR_INVALID, "cg_step_prepare: null pointer");
    if (vocab <= 0 || hidden <= 0 || (hidden % 8) != 0)
      return fail(AIOS_ERR_INVALID, "cg_step_prepare: embedding of %lld x %d (hidden must be a "
                                    "positive multiple of 8)", (long long)vocab, hidden);
    if ((((uintptr_t)embed | (uintptr_t)h_out) & 15) != 0)
      return fail(AIOS_ERR_INVALID, "cg_step_prepare: embedding table and rows must be 16-byte "
                                    "aligned");
  }
  aios::CgStepArgs a = {};
  a.rows = rows;
  a.step = step;
  a.pages = pages;
  a.page_rows = page_rows;
  a.out_loc = out_loc;
  a.page_table = page_table;
  a.pt_stride = pt_stride;
  a.pt_cols = pt_cols;
  a.pos = pos;
  a.cu_k = cu_k;
  a.indices = indices;
  a.max_kv_len = max_kv_len;
  a.step_next = step_next;
  a.tokens = const_cast<int64_t*>(tokens);
  a.embed = static_cast<const aios::bf16*>(embed);
  a.vocab = vocab;
  a.hidden = hidden;
  a.h_out = static_cast<aios::bf16*>(h_out);
  return check_hip(aios::cg_step_prepare(a, static_cast<hipStream_t>(stream)),
                   "cg_step_prepare launch");
}

int aios_cg_step_end(int64_t* step, int32_t rows, const int64_t* tok, const float* raw, int64_t eos,
                     uint8_t* finished, uint8_t* eos_hit, int64_t* out_ids, int64_t out_stride,
                     int32_t out_cols, float* logp_sum, int64_t* counts, int64_t* tokens,
                     int32_t* pos, int64_t* fed, void* stream) {
  if (rows <= 0 || out_cols <= 0 || out_stride < out_cols)
    return fail(AIOS_ERR_INVALID, "cg_step_end: bad sizes");
  if (!step || !tok || !raw || !finished || !eos_hit || !out_ids || !logp_sum || !counts ||
      !tokens || !pos || !fed)
    return fail(AIOS_ERR_INVALID, "cg_step_end: null pointer");
  aios::CgStepArgs a = {};
  a.rows = rows;
  a.step = step;
  a.tok = tok;
  a.raw = raw;
  a.eos = eos < 0 ? -1 : eos;
  a.finished = finished;
  a.eos_hit = eos_hit;
  a.out_ids = out_ids;
  a.out_stride = out_stride;
  a.out_cols = out_cols;
  a.logp_sum = logp_sum;
  a.counts = counts;
  a.tokens = tokens;
  a.pos = pos;
  a.fed = fed;
  return check_hip(aios::cg_step_end(a, static_cast<hipStream_t>(stream)), "cg_step_end launch");
}

int aios_greedy_select(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                       int32_t elem_bytes, int64_t* token_out, float* logprob_out,
                       void* stream) {
  if (rows < 0 || vocab <= 0 || row_stride < vocab)
    return fail(AIOS_ERR_INVALID, "greedy_select: bad sizes (rows=%d vocab=%d stride=%lld)", rows,
                vocab, (long long)row_stride);
  if (elem_bytes != 2 && elem_bytes != 4)
    return fail(AIOS_ERR_UNSUPPORTED, "greedy_select: elem_bytes %d", elem_bytes);
  if (rows == 0) return AIOS_OK;
  if (!logits || !token_out || !logprob_out)
    return fail(AIOS_ERR_INVALID, "greedy_select: null pointer");
  return check_hip(aios::greedy_select(logits, row_stride, rows, vocab, elem_bytes, token_out,
                                       logprob_out, static_cast<hipStream_t>(stream)),
                   "greedy_select launch");
}

int aios_stateless_uniforms(const int64_t* seeds, int32_t rows, int32_t steps, float* out,
                            void* stream) {
  if (rows < 0 || steps < 1)
    return fail(AIOS_ERR_INVALID, "stateless_uniforms: steps must be positive (rows=%d steps=%d)",
                rows, steps);
  if (rows == 0) return AIOS_OK;
  if (!seeds || !out) return fail(AIOS_ERR_INVALID, "stateless_uniforms: null pointer");
  return check_hip(aios::stateless_uniforms(seeds, rows, steps, out,
                                            static_cast<hipStream_t>(stream)),
                   "stateless_uniforms launch");
}

int aios_sample(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                int32_t elem_bytes, float temperature, int32_t top_k, float top_p,
                const float* uniforms, int64_t uniform_stride, int32_t uniform_count,
                const int64_t* step, const int32_t* forbidden, int32_t n_forbidden,
                int32_t forbid_before_step, const int64_t* forbidden_by_row,
                int32_t row_forbidden_count, int64_t* token_out, float* logprob_out,
                void* stream) {
  if (rows < 0 || vocab <= 0 || (row_stride != 0 && row_stride < vocab))
    return fail(AIOS_ERR_INVALID, "sample: bad sizes (rows=%d vocab=%d stride=%lld)", rows, vocab,
                (long long)row_stride);
  if (elem_bytes != 2 && elem_bytes != 4)
    return fail(AIOS_ERR_UNSUPPORTED, "sample: elem_bytes %d", elem_bytes);
  if (n_forbidden < 0 || row_forbidden_count < 0 ||
      n_forbidden + row_forbidden_count > aios::kSampleMaxForbidden)
    return fail(AIOS_ERR_INVALID, "sample: at most %d forbidden ids per row",
                aios::kSampleMaxForbidden);
  const bool greedy = (temperature <= 0.f || top_k == 1) && top_p == 1.f;
  if (!greedy) {
    if (!(temperature > 0.f)) return fail(AIOS_ERR_INVALID, "sample: temperature must be positive");
    if (!(top_p > 0.f && top_p <= 1.f)) return fail(AIOS_ERR_INVALID, "sample: top_p must be in (0, 1]");
    if (top_k > aios::kSampleMaxTopK)
      return fail(AIOS_ERR_UNSUPPORTED, "sample: top_k %d above %d is not built", top_k,
                  aios::kSampleMaxTopK);
    if (top_k <= 0 && top_p < 1.f)
      return fail(AIOS_ERR_UNSUPPORTED, "sample: top_p without top_k (a full-vocabulary sort) is not built");
    if (!uniforms || uniform_count < 1 || uniform_stride < uniform_count)
      return fail(AIOS_ERR_INVALID, "sample: uniforms are required to sample");
  }
  if (rows == 0) return AIOS_OK;
  if (!logits || !token_out || !logprob_out) return fail(AIOS_ERR_INVALID, "sample: null pointer");
  if (((uintptr_t)logits & 15) != 0 || (row_stride * elem_bytes) % 16 != 0)
    return fail(AIOS_ERR_INVALID, "sample: logits rows must be 16-byte aligned");
  if ((n_forbidden > 0 && !forbidden) || (row_forbidden_count > 0 && !forbidden_by_row))
    return fail(AIOS_ERR_INVALID, "sample: null forbidden list");
  aios::SampleArgs a;
  a.logits = logits;
  a.row_stride = row_stride;
  a.rows = rows;
  a.vocab = vocab;
  a.elem_bytes = elem_bytes;
  a.temperature = temperature;
  a.top_k = greedy ? 1 : (top_k > 0 ? top_k : 0);
  a.top_p = top_p;
  a.greedy = greedy ? 1 : 0;
  a.uniforms = greedy ? nullptr : uniforms;
  a.uniform_stride = uniform_stride;
  a.uniform_count = uniform_count;
  a.step = step;
  a.forbidden = n_forbidden > 0 ? forbidden : nullptr;
  a.n_forbidden = n_forbidden;
  a.forbid_before_step = forbid_before_step;
  a.forbidden_by_row = row_forbidden_count > 0 ? forbidden_by_row : nullptr;
  a.row_forbidden_count = row_forbidden_count;
  a.token_out = token_out;
  a.logprob_out = logprob_out;
  return check_hip(aios::sample_rows(a, static_cast<hipStream_t>(stream)), "sample launch");
}

static bool overlaps(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
  if (!a || !b) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)b_bytes && y < x + (uintptr_t)a_bytes;
}

int aios_attnres_mix_ex(const void* bank, int32_t bank_sources, int64_t num_tokens,
                        int32_t hidden, const void* partial, const void* delta,
                        void* partial_out, const float* weighted_query, float eps, float* scores,
                        void* out, void* stream) {
  if (bank_sources < 1 || num_tokens < 1 || hidden < 1)
    return fail(AIOS_ERR_INVALID, "attnres_mix: bank dimensions must be positive");
  if (num_tokens > 0x7fffffffll)
    return fail(AIOS_ERR_INVALID, "attnres_mix: num_tokens %lld too large", (long long)num_tokens);
  const int total = bank_sources + ((partial || delta) ? 1 : 0);
  if (!aios::attnres_supported(hidden, total))
    return fail(AIOS_ERR_UNSUPPORTED,
                "attnres_mix: hidden %d (multiple of 8 up to 8192) or %d sources (<= 64) not built",
                hidden, total);
  if (!bank || !weighted_query || !out) return fail(AIOS_ERR_INVALID, "attnres_mix: null pointer");
  if ((((uintptr_t)bank | (uintptr_t)partial | (uintptr_t)delta | (uintptr_t)partial_out |
        (uintptr_t)weighted_query | (uintptr_t)out) & 15) != 0)
    return fail(AIOS_ERR_INVALID, "attnres_mix: tensors must be 16-byte aligned");
  const int64_t plane = num_tokens * (int64_t)hidden * 2;
  if (overlaps(out, plane, bank, plane * bank_sources) ||
      overlaps(partial_out, plane, bank, plane * bank_sources) ||
      overlaps(out, plane, partial_out, plane) || overlaps(out, plane, partial, plane) ||
      overlaps(out, plane, delta, plane))
    return fail(AIOS_ERR_INVALID, "attnres_mix: out / partial_out overlap an input");
  aios::AttnResArgs a;
  a.bank = static_cast<const aios::bf16*>(bank);
  a.bank_sources = bank_sources;
  a.num_tokens = num_tokens;
  a.hidden = hidden;
  a.partial = static_cast<const aios::bf16*>(partial);
  a.delta = static_cast<const aios::bf16*>(delta);
  a.partial_out = static_cast<aios::bf16*>(partial_out);
  a.wq = weighted_query;
  a.eps = eps;
  a.scores = scores;
  a.out = static_cast<aios::bf16*>(out);
  return check_hip(aios::attnres_mix(a, static_cast<hipStream_t>(stream)), "attnres_mix launch");
}

int aios_attnres_mix(const void* bank, int32_t bank_sources, int64_t num_tokens, int32_t hidden,
                     const void* partial, const float* weighted_query, float eps, float* scores,
                     void* out, void* stream) {
  return aios_attnres_mix_ex(bank, bank_sources, num_tokens, hidden, partial, nullptr, nullptr,
                             weighted_query, eps, scores, out, stream);
}

}  // extern "C"
