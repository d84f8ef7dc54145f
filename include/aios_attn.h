/*
 * aios_attn.h — C ABI of the MI355X (gfx950) paged attention backend for
 * AIOS-IME.
 *
 * Every entry point takes plain device pointers, element strides and a HIP
 * stream handle (passed as void*), returns an int status (AIOS_OK == 0) and
 * never synchronises the host.  The library allocates no device memory:
 * the KV pool, page indices, outputs and the partial-softmax workspace all
 * belong to the caller.  On a non-zero status, aios_last_error() returns a
 * thread-local, NUL-terminated message.
 *
 * Reference interfaces replaced (paths relative to the 7155/aios tree):
 *   aios_kv_append     python/aios/kernel/store.py:32-61 (store_cache), the
 *                      op behind MHAKVCache.store_kv (python/aios/kvcache/
 *                      mha_pool.py:45-56)
 *   aios_attn_plan     FlashInferAttentionBackend._initialize_metadata_once
 *                      -> wrapper.plan(...) (python/aios/attention/
 *                      flashinfer.py:252-289)
 *   aios_attn_prefill  BatchPrefillWithPagedKVCacheWrapper.run and the
 *                      head_dim-96 SDPA fallback (python/aios/attention/
 *                      flashinfer.py:300-372, 33-91)
 *   aios_attn_decode   BatchDecodeWithPagedKVCacheWrapper.run (python/aios/
 *                      attention/flashinfer.py:374-394)
 *   aios_attn_append_decode  store_kv (flashinfer.py:389 -> store.py:32-61)
 *                      and the decode run above, in one launch
 *   aios_attn_append_decode_rope  the same with Qwen3Attention's q/k norm
 *                      and rotary embedding (python/aios/models/qwen3.py:
 *                      52-67) applied on load
 *   aios_build_indices the device half of prepare_metadata's
 *                      torch.cat([page_table[row, :device_len] ...])
 *                      (python/aios/attention/flashinfer.py:228-230)
 *   aios_rmsnorm, aios_qk_norm_rope, aios_silu_mul  the decoder-layer
 *                      elementwise ops that produce the backend's inputs
 *                      (python/aios/layers/norm.py:18-40, models/qwen3.py:
 *                      60-70, layers/attention.py:11-16, activation.py:9-12)
 *   aios_linear_rows   F.linear of the few-row decode projections
 *                      (python/aios/layers/linear.py:11-60)
 *   aios_greedy_select the greedy branch of Sampler.sample_with_logprobs
 *                      (python/aios/engine/sample.py:73, 115-117): argmax of
 *                      the logits plus the raw log_softmax value gathered
 *                      there, as called by the CandidateGroup decode loop
 *                      (python/aios/ime.py:998-1008)
 *   aios_stateless_uniforms, aios_sample  stateless_uniforms and the
 *                      uniforms path of Sampler.sample_with_logprobs
 *                      (python/aios/engine/sample.py:12-160)
 *   aios_attnres_mix, aios_attnres_mix_ex  triton_attnres_mix
 *                      (python/aios/kernel/attnres.py:130-223) behind
 *                      BlockAttnResMixer (python/aios/models/minimind_ime.py:
 *                      92-190), the latter with the block's partial update
 */
#ifndef AIOS_ATTN_H
#define AIOS_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define AIOS_OK 0
#define AIOS_ERR_INVALID 1     /* bad shape / stride / argument (ValueError)  */
#define AIOS_ERR_UNSUPPORTED 2 /* head_dim, group size or dtype not built     */
#define AIOS_ERR_WORKSPACE 3   /* caller workspace smaller than plan needs    */
#define AIOS_ERR_LAUNCH 4      /* HIP runtime error at launch (RuntimeError)  */

#define AIOS_PHASE_PREFILL 0
#define AIOS_PHASE_DECODE 1

/* Thread-local message for the last non-zero status of this thread. */
const char* aios_last_error(void);

/* Version string of the built library. */
const char* aios_version(void);

/*
 * Paged KV append (kernel (a)).  For t in [0, n_tokens):
 *   k_cache[out_loc[t] * cache_tok_stride + 0 .. width) = k[t * k_tok_stride + 0 .. width)
 *   v_cache[out_loc[t] * cache_tok_stride + 0 .. width) = v[t * v_tok_stride + 0 .. width)
 * Strides and width are in elements of elem_bytes bytes (2 for bf16/fp16).
 * k and v have independent token strides (v is usually a strided view into
 * the fused qkv projection).  out_loc entries outside [0, num_slots) are
 * skipped (never written).  Replaces kernel/store.py:8-61.
 */
int aios_kv_append(void* k_cache, void* v_cache, int64_t num_slots,
                   int64_t cache_tok_stride, const int32_t* out_loc,
                   const void* k, int64_t k_tok_stride, const void* v,
                   int64_t v_tok_stride, int64_t n_tokens, int64_t width,
                   int32_t elem_bytes, void* stream);

/*
 * Per-batch schedule, built on the host from host copies of cu_seqlens and
 * reused by every layer of the batch (the plan-once contract of
 * flashinfer.py:252-256).  Filled by aios_attn_plan; treat as opaque apart
 * from ws_bytes (workspace bytes the batch needs).
 */
typedef struct aios_attn_plan {
  int32_t phase;
  int32_t batch_size;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t group; /* num_qo_heads / num_kv_heads */
  int32_t total_q;
  int32_t total_kv;
  int32_t max_q_len;
  int32_t max_kv_len;
  /* decode */
  int32_t prefix_len;        /* shared prefix read once per kv-head (0 = not used) */
  int32_t prefix_chunk_len;  /* KV positions per prefix workgroup */
  int32_t num_prefix_chunks;
  int32_t cascade_rows;      /* batch_size * group */
  int32_t cascade_mgroups;   /* 128-row groups of cascade_rows */
  int32_t suffix_split_len;  /* KV positions per suffix item */
  int32_t num_suffix_splits; /* suffix items per (row, kv-head) */
  int32_t suffix_tpg;        /* KV positions a suffix wavefront gathers per pass */
  int32_t num_parts;         /* partial states per (row, kv-head); 1 = direct output */
  /* prefill */
  int32_t prefill_q_tile;    /* query tokens per workgroup */
  int32_t num_q_tiles;
  /* decode launches to issue: bit 0 the main kernel (prefix chunks and
   * suffix items), bit 1 the combine; 0 (the value aios_attn_plan writes)
   * issues both.  Lets a profiler bracket the two launches separately. */
  int32_t stage_mask;
  int32_t min_kv_len;        /* shortest row of the batch */
  int32_t suffix_parts_per_item; /* partial states one suffix item writes: 1 (its
                                  * wavefronts merge first) or 4 (one per wavefront) */
  /* workspace layout (byte offsets) */
  int64_t ws_parts_o;
  int64_t ws_parts_lse;
  int64_t ws_bytes;
} aios_attn_plan_t;

/*
 * Build the schedule for one batch.
 *   cu_q_host, cu_k_host : host int32 arrays of batch_size + 1 prefix sums of
 *                          per-request query / KV lengths (cu_seqlens_q/k).
 *   shared_prefix_len    : decode only.  Number of leading KV positions whose
 *                          page ids are identical in every row (the
 *                          CandidateGroup shares page_table[:, :P]); 0 = none.
 *                          Those positions are read once per kv-head.
 *   prefix_chunk_len, suffix_split_len : tuning overrides (0 = automatic).
 * Performs validation only on host data; touches no device memory.
 */
int aios_attn_plan(int32_t phase, const int32_t* cu_q_host,
                   const int32_t* cu_k_host, int32_t batch_size,
                   int32_t num_qo_heads, int32_t num_kv_heads,
                   int32_t head_dim, int32_t page_size,
                   int32_t shared_prefix_len, int64_t workspace_bytes,
                   int32_t prefix_chunk_len, int32_t suffix_split_len,
                   aios_attn_plan_t* plan_out);

/*
 * Varlen causal paged prefill (kernel (b)), bf16.  Request r owns query rows
 * [cu_q[r], cu_q[r+1]) and KV positions [0, kv_len_r) whose pages are
 * indices[cu_k[r] + pos]; query row i of r sits at absolute position
 * cached_len_r + i with cached_len_r = kv_len_r - q_len_r and attends to
 * positions <= cached_len_r + i.  q is [total_q, Hq, D] with token stride
 * q_tok_stride (elements; head stride D), the per-layer caches are
 * [kv_num_pages, Hkv, D] contiguous, out is [total_q, Hq, D] contiguous.
 * cu_q, cu_k and indices are device int32.  A page id outside
 * [0, kv_num_pages) is read as an all-zero K/V row (never dereferenced).
 * One layer's cache (kv_num_pages * Hkv * D * 2 bytes) must be below 4 GiB
 * (the kernels use 32-bit byte offsets) and kv_num_pages below 2^24 (a
 * 24-bit page multiply); AIOS_ERR_UNSUPPORTED otherwise.
 */
int aios_attn_prefill(const aios_attn_plan_t* plan, const void* q,
                      int64_t q_tok_stride, const void* k_cache,
                      const void* v_cache, int64_t kv_num_pages,
                      const int32_t* indices,
                      const int32_t* cu_q, const int32_t* cu_k, void* out,
                      float sm_scale, void* stream);

/*
 * Paged decode (kernels (c) + (d) + log-sum-exp combine), bf16.  Row b has
 * one query token q[b] and KV positions [0, kv_len_b) with pages
 * indices[cu_k[b] + pos].  Positions [0, plan->prefix_len) are read through
 * row 0's page ids (indices[0 .. prefix_len)) once per kv-head and shared by
 * all rows; the rest are read per row.  workspace holds the partial softmax
 * states (plan->ws_bytes bytes).  Page ids and the 4 GiB per-layer cache
 * limit as for aios_attn_prefill.
 */
int aios_attn_decode(const aios_attn_plan_t* plan, const void* q,
                     int64_t q_tok_stride, const void* k_cache,
                     const void* v_cache, int64_t kv_num_pages,
                     const int32_t* indices,
                     const int32_t* cu_k, void* out, void* workspace,
                     int64_t workspace_bytes, float sm_scale, void* stream);

/*
 * Paged KV append and decode in one launch: the same result as
 *   aios_kv_append(k_cache, v_cache, kv_num_pages, Hkv*D, out_loc, k_new,
 *                  k_tok_stride, v_new, v_tok_stride, batch_size, Hkv*D, 2)
 * followed by aios_attn_decode(...), for the decode step of
 * BatchDecodeWithPagedKVCacheWrapper after MHAKVCache.store_kv
 * (python/aios/attention/flashinfer.py:374-394 with :389, and
 * python/aios/kernel/store.py:32-61).  Row b's new token is its last KV
 * position: indices[cu_k[b+1] - 1] == out_loc[b]; its K/V rows k_new[b],
 * v_new[b] ([Hkv, D], token strides in elements) are attended to directly
 * and written to page out_loc[b] (an out_loc outside [0, kv_num_pages) is
 * not written, and that row then attends to zeros there, as the separate
 * calls would).  Needs plan->prefix_len < plan->min_kv_len (the new token
 * is never part of the shared prefix).
 */
int aios_attn_append_decode(const aios_attn_plan_t* plan, const void* q,
                            int64_t q_tok_stride, const void* k_new,
                            int64_t k_tok_stride, const void* v_new,
                            int64_t v_tok_stride, const int32_t* out_loc,
                            void* k_cache, void* v_cache, int64_t kv_num_pages,
                            const int32_t* indices, const int32_t* cu_k,
                            void* out, void* workspace, int64_t workspace_bytes,
                            float sm_scale, void* stream);

/*
 * aios_attn_append_decode with the per-head query/key RMSNorm and rotary
 * embedding of the decoder layer applied on load: q and k_new are the raw
 * projections (the q and k parts of the fused qkv rows), and the result -
 * attention output and the K row written to page out_loc[b] - is that of
 *   aios_qk_norm_rope(q/k rows, q_norm, k_norm, cos, sin, rope_rows,
 *                     positions, norm_eps)
 * followed by aios_attn_append_decode on its outputs (the fp32 sum of squares
 * of a head is taken in another order, so a normalised element can differ by
 * one bf16 unit where that sum rounds differently).  Replaces, for a decode
 * batch, the q_norm / k_norm + rotary embedding of Qwen3Attention.forward
 * (python/aios/models/qwen3.py:52-67) together with store_kv and the decode
 * run (python/aios/attention/flashinfer.py:374-394).  q_norm, k_norm: bf16
 * [D]; rope_cos, rope_sin: bf16 [rope_rows][D], the fp32 cos / sin tables
 * of aios_qk_norm_rope rounded to bf16 (nearest even: the rounding that
 * call applies to each entry it uses); positions: int32 [batch_size]
 * (clamped into the table); these and the k_new rows 16-byte aligned.
 */
int aios_attn_append_decode_rope(const aios_attn_plan_t* plan, const void* q,
                                 int64_t q_tok_stride, const void* k_new,
                                 int64_t k_tok_stride, const void* v_new,
                                 int64_t v_tok_stride, const int32_t* out_loc,
                                 void* k_cache, void* v_cache, int64_t kv_num_pages,
                                 const int32_t* indices, const int32_t* cu_k,
                                 const void* q_norm, const void* k_norm,
                                 const void* rope_cos, const void* rope_sin,
                                 int64_t rope_rows, const int32_t* positions,
                                 float norm_eps, void* out, void* workspace,
                                 int64_t workspace_bytes, float sm_scale, void* stream);

/*
 * aios_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The partial softmax states live in a device array built into the library
 * (AIOS_DECODE_NOALLOC_MAX_BYTES per GPU, held until the process ends); a
 * plan whose ws_bytes exceeds it returns AIOS_ERR_WORKSPACE.  The call
 * allocates nothing (no hipMalloc / hipFree); its first call on a device
 * looks up that device's array once.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (concurrent streams or
 * threads) race.  Nothing in the array needs to start at zero: every
 * partial the combine reads is written by the same call.  The stream must
 * belong to the current device.  Same results as aios_attn_decode.
 */
#define AIOS_DECODE_NOALLOC_MAX_BYTES (8ll << 20)
int aios_attn_decode_noalloc(const aios_attn_plan_t* plan, const void* q,
                             int64_t q_tok_stride, const void* k_cache,
                             const void* v_cache, int64_t kv_num_pages,
                             const int32_t* indices, const int32_t* cu_k,
                             void* out, float sm_scale, void* stream);

/*
 * Gather the flat page-index list of a batch on the device:
 *   indices_out[cu_k[b] + j] = page_table[row_ids[b] * page_table_stride + j]
 * for j in [0, cu_k[b+1] - cu_k[b]).  row_ids and cu_k are device int32.
 */
int aios_build_indices(const int32_t* page_table, int64_t page_table_stride,
                       const int32_t* row_ids, const int32_t* cu_k,
                       int32_t batch_size, int32_t total_kv,
                       int32_t* indices_out, void* stream);

/*
 * RMSNorm over rows of bf16 hidden states (hidden a multiple of 8, <= 8192;
 * rows 16-byte aligned), fp32 math:
 *   residual == NULL: out = x * rsqrt(mean(x^2) + eps) * weight
 *   otherwise:        r = x + residual; residual <- r (bf16);
 *                     out = r * rsqrt(mean(r^2) + eps) * weight
 * Replaces flashinfer rmsnorm / fused_add_rmsnorm behind RMSNorm and
 * RMSNormFused (python/aios/layers/norm.py:18-40).  out may alias x.
 */
int aios_rmsnorm(const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
                 const void* weight, void* out, int64_t out_stride, int64_t rows, int32_t hidden,
                 float eps, void* stream);

/*
 * Per-head query/key RMSNorm followed by rotary embedding, from the fused
 * qkv projection rows [tokens][(Hq + 2*Hkv) * D] (row stride qkv_stride):
 *   x' = bf16(x * rsqrt(mean(x^2) + eps) * w)                (q or k weight)
 *   out_i = bf16(bf16(x'_i * c_i) + bf16(rot(x')_i * s_i)),  rot = rotate_half
 * with c, s = bf16(cos/sin_table[positions[t]][i]) (fp32 tables of
 * table_rows x D; positions outside [0, table_rows) are clamped into it).
 * q_out is [tokens][Hq][D], k_out [tokens][Hkv][D].
 * Replaces q_norm / k_norm (python/aios/models/qwen3.py:65-66) and
 * apply_rotary_pos_emb (python/aios/layers/attention.py:11-16).
 */
int aios_qk_norm_rope(const void* qkv, int64_t qkv_stride, int64_t tokens, int32_t num_qo_heads,
                      int32_t num_kv_heads, int32_t head_dim, const void* q_weight,
                      const void* k_weight, const float* cos_table, const float* sin_table,
                      int64_t table_rows, const int32_t* positions, void* q_out, void* k_out,
                      float eps, void* stream);

/*
 * out[r][i] = bf16(bf16(silu(x[r][i])) * x[r][intermediate + i]) for the
 * merged gate/up rows x [rows][2 * intermediate].  Replaces silu_and_mul
 * (python/aios/layers/activation.py:9-12).
 */
int aios_silu_mul(const void* x, int64_t x_stride, int64_t rows, int32_t intermediate, void* out,
                  int64_t out_stride, void* stream);

/*
 * y[r][n] = sum_k x[r][k] * weight[n][k] (bf16 in, fp32 accumulate, bf16
 * out) for 1..64 rows, out_features a multiple of 16 and in_features a
 * multiple of 128: the projections of a decode step (F.linear behind
 * Linear / LinearQKVMerged / LinearColParallelMerged,
 * python/aios/layers/linear.py:11-60, and the tied LM head,
 * python/aios/layers/embedding.py:13-41).  Returns AIOS_ERR_UNSUPPORTED for
 * other shapes (callers use a library GEMM there).
 */
int aios_linear_rows(const void* x, int64_t x_stride, const void* weight, int64_t w_stride,
                     void* y, int64_t y_stride, int64_t rows, int64_t out_features,
                     int64_t in_features, void* stream);

#define AIOS_PROLOGUE_NONE 0
#define AIOS_PROLOGUE_ADD_RMSNORM 1
#define AIOS_EPILOGUE_NONE 0
#define AIOS_EPILOGUE_SILU_MUL 1

/*
 * aios_linear_rows with the ops around the projection folded in (same shape
 * limits):
 *   prologue AIOS_PROLOGUE_ADD_RMSNORM: the operand is bf16(RMSNorm(x +
 *     residual) * norm_weight) as aios_rmsnorm computes it (residual may be
 *     NULL), and residual_out (if not NULL; must not alias x or residual)
 *     receives bf16(x + residual) -- RMSNormFused.forward followed by the
 *     projection (python/aios/layers/norm.py:24-40, models/qwen3.py:
 *     112-130); supported for in_features / 128 * ceil(rows / 16) <= 8;
 *   epilogue AIOS_EPILOGUE_SILU_MUL: weight holds 2 * out_features rows
 *     (gate rows, then up rows: the merged gate/up projection) and
 *     y = silu_and_mul of the two bf16 halves
 *     (python/aios/layers/activation.py:9-12, models/qwen3.py:91-93).
 */
int aios_linear_rows_ex(const void* x, int64_t x_stride, const void* weight, int64_t w_stride,
                        void* y, int64_t y_stride, int64_t rows, int64_t out_features,
                        int64_t in_features, int32_t prologue, const void* residual,
                        int64_t residual_stride, const void* norm_weight, float eps,
                        void* residual_out, int64_t residual_out_stride, int32_t epilogue,
                        void* stream);

/*
 * The per-step bookkeeping of a captured CandidateGroup decode step (the
 * branch loop of python/aios/ime.py:1010-1054 around the model), all state
 * in device memory so that a graph replays it:
 *   aios_cg_step_begin: s = *step (clamped to [0, page_rows)); for every
 *     row r: out_loc[r] = pages[s][r] and page_table[r][pos[r]] = out_loc[r]
 *     (positions outside [0, pt_cols) are not written) -- the page the
 *     step's K/V goes to (ime.py:1219-1251);
 *   aios_cg_step_end: with the step's pick tok / raw: a row that is not
 *     finished is live; a live row whose token is eos (eos >= 0) finishes
 *     (eos_hit, finished set) and emits nothing; otherwise a live row emits:
 *     out_ids[r][*step + 1] = tok (or -1), logp_sum += raw, counts += 1;
 *     tokens = tok, pos += 1 for every row; fed += live rows; *step += 1.
 * bool flags are one byte.  No reference counterpart as a single call: the
 * reference runs these as torch ops on the host loop.
 */
int aios_cg_step_begin(int64_t* step, const int32_t* pages, int32_t page_rows, int32_t rows,
                       int32_t* out_loc, int32_t* page_table, int64_t pt_stride, int32_t pt_cols,
                       int32_t* pos, void* stream);
int aios_cg_step_end(int64_t* step, int32_t rows, const int64_t* tok, const float* raw, int64_t eos,
                     uint8_t* finished, uint8_t* eos_hit, int64_t* out_ids, int64_t out_stride,
                     int32_t out_cols, float* logp_sum, int64_t* counts, int64_t* tokens,
                     int32_t* pos, int64_t* fed, void* stream);

/*
 * aios_cg_step_begin and the rest of what a captured decode step reads
 * before the model, in one launch (the ime.py:1219-1251 page column, the
 * decode metadata of flashinfer.py:209-250 for a group whose rows share
 * their length, the sampler's step column and the embedding lookup of
 * embedding.py:13-41):
 *   the page-table column and out_loc as aios_cg_step_begin;
 *   L = pos[0] + 1 clamped to [0, max_kv_len]; cu_k[b] = b * L for
 *     b in [0, rows]; indices[b * L + j] = page_table[b][j] for j < L (the
 *     column written this step read as out_loc[b]); rows are page-table
 *     rows 0 .. rows-1;
 *   *step_next = *step + 1 (step_next may be null);
 *   embed non-null: h_out[r][:] = embed[tokens[r]][:] (bf16 [vocab][hidden],
 *     hidden a multiple of 8, 16-byte aligned; ids clamped to [0, vocab)).
 * cu_k holds rows + 1 and indices rows * max_kv_len entries; max_kv_len is
 * at most pt_cols.
 */
int aios_cg_step_prepare(int64_t* step, const int32_t* pages, int32_t page_rows, int32_t rows,
                         int32_t* out_loc, int32_t* page_table, int64_t pt_stride, int32_t pt_cols,
                         int32_t* pos, int32_t* cu_k, int32_t* indices, int32_t max_kv_len,
                         int64_t* step_next, const int64_t* tokens, const void* embed,
                         int64_t vocab, int32_t hidden, void* h_out, void* stream);

/*
 * Greedy selection over rows of logits (elem_bytes 2: bf16, 4: fp32):
 *   token_out[r]   = first index of the maximum of logits[r, 0 .. vocab)
 *   logprob_out[r] = logits[r, token] - logsumexp(logits[r, :])  (fp32)
 * Rows are row_stride elements apart.  token_out is device int64,
 * logprob_out device fp32.  Replaces sample.py:73, 115-117 (greedy).
 */
int aios_greedy_select(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                       int32_t elem_bytes, int64_t* token_out, float* logprob_out,
                       void* stream);

/*
 * out[r][t] = the stateless U(0, 1) of candidate seed seeds[r] at token
 * step t (fp32 [rows][steps]): SplitMix64 of seed + (t + 1) * 0x9E3779B97F4A7C15,
 * (high 53 bits + 0.5) / 2^53.  Replaces stateless_uniforms
 * (python/aios/engine/sample.py:12-47), computed on the device.
 */
int aios_stateless_uniforms(const int64_t* seeds, int32_t rows, int32_t steps, float* out,
                            void* stream);

/*
 * One token per row of logits (elem_bytes 2: bf16, 4: fp32; rows
 * row_stride elements apart, 16-byte aligned; row_stride 0: every row
 * samples the same logits, e.g. the prefix logits of a candidate group,
 * each with its own uniform) and its raw log-probability
 * log_softmax(logits)[token] (fp32), as Sampler.sample_with_logprobs with
 * stateless uniforms (python/aios/engine/sample.py:50-160):
 *   - sampling logits = logits with the forbidden ids at -inf: forbidden
 *     (n_forbidden ids, applied while *step < forbid_before_step) and row
 *     r's forbidden_by_row[r][0 .. row_forbidden_count) (at most 256 ids in
 *     all; ids outside the vocabulary are ignored);
 *   - greedy ((temperature <= 0 or top_k == 1) and top_p == 1): the first
 *     index of the maximum;
 *   - otherwise logits / temperature; the top_k largest (ties: lower id
 *     first; top_k <= 1024) or, for top_k <= 0 with top_p == 1, every id in
 *     id order; softmax; for top_p < 1 the ids whose preceding cumulative
 *     probability exceeds top_p are removed (the first is kept) and the
 *     softmax is taken again; the chosen candidate is the number of
 *     cumulative probabilities below u, clamped to the last one, with u =
 *     uniforms[r * uniform_stride + min(*step, uniform_count - 1)] (step
 *     NULL: column 0).
 * top_k <= 0 with top_p < 1 (a full-vocabulary sort) returns
 * AIOS_ERR_UNSUPPORTED.  token_out int64, logprob_out fp32, both [rows].
 */
int aios_sample(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                int32_t elem_bytes, float temperature, int32_t top_k, float top_p,
                const float* uniforms, int64_t uniform_stride, int32_t uniform_count,
                const int64_t* step, const int32_t* forbidden, int32_t n_forbidden,
                int32_t forbid_before_step, const int64_t* forbidden_by_row,
                int32_t row_forbidden_count, int64_t* token_out, float* logprob_out,
                void* stream);

/*
 * Block-AttnRes depth mix.  bank is contiguous bf16 [bank_sources]
 * [num_tokens][hidden]; partial (may be NULL) a contiguous bf16
 * [num_tokens][hidden] plane appended as the last source;
 * weighted_query fp32 [hidden] = query * key_norm.weight.  Per token:
 *   score_s = <x_s, wq> * rsqrt(mean(x_s^2) + eps)       (fp32)
 *   w_s     = bf16(softmax over s of score)
 *   out     = bf16(sum_s w_s * x_s)                      (fp32 sum)
 * scores (may be NULL) receives score_s at [s * num_tokens + token].
 * hidden a multiple of 8 up to 8192, at most 64 sources (UNSUPPORTED
 * otherwise); every pointer 16-byte aligned; out must not overlap an input.
 * Replaces triton_attnres_mix (python/aios/kernel/attnres.py:130-223; the
 * mixer of python/aios/models/minimind_ime.py:92-190): one launch that reads
 * the bank once.
 */
int aios_attnres_mix(const void* bank, int32_t bank_sources, int64_t num_tokens, int32_t hidden,
                     const void* partial, const float* weighted_query, float eps, float* scores,
                     void* out, void* stream);

/*
 * aios_attnres_mix with the block's running-partial update folded in: when
 * delta is not NULL the partial source is bf16(partial + delta) (delta
 * alone when partial is NULL) -- the `partial + attention_delta` and
 * `partial + mlp_delta` adds of python/aios/models/minimind_ime.py:233-252 --
 * and partial_out (if not NULL) receives it.  partial_out may equal partial
 * (in-place update) or be the bank's next slot bank + bank_sources *
 * num_tokens * hidden (the block's new depth source, minimind_ime.py:
 * 305-315); it must not overlap the bank or out.
 */
int aios_attnres_mix_ex(const void* bank, int32_t bank_sources, int64_t num_tokens,
                        int32_t hidden, const void* partial, const void* delta,
                        void* partial_out, const float* weighted_query, float eps, float* scores,
                        void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AIOS_ATTN_H */
