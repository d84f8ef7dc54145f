// Internal launch interface shared by the kernel translation units and the
// C ABI in api.hip.
#pragma once

#include "common.hpp"

namespace aios {

// Partial softmax states of a decode batch live in one workspace array.
// Rows are the batch * G query rows m = b * G + g; for kv-head h and part j
// (slot j < n_chunks: prefix chunk j; n_chunks + s: suffix split s):
//   o   [Hkv][n_parts][D/16][rows][16] bf16 (normalised o = acc / l)
//   lse [Hkv][n_parts][rows]           fp32 (log2-domain m + log2 l; -inf = empty)
// so the 16 rows x 16 dims an MFMA accumulator tile holds are one
// contiguous 512-byte run, and the G rows of one (b, h, j) are adjacent.
struct PartsArgs {
  bf16* o;
  float* lse;
  int32_t n_parts;
  int32_t n_chunks;
  int32_t rows;  // batch * G
  // The struct's last word, named so that the prefix part can read it:
  // the decode kernel loads the struct with one 8-word scalar load, and a
  // loaded word that no code reads leaves its register free for reuse
  // while the load is in flight, which makes the wave wait for the whole
  // load at that reuse (ahead of the page-id loads).  Unused otherwise.
  int32_t spare;

  // Element (h, j, m, d) of o for head dimension D.
  __host__ __device__ int64_t o_index(int D, int h, int j, int m, int d) const {
    return ((((int64_t)h * n_parts + j) * (D >> 4) + (d >> 4)) * rows + m) * 16 + (d & 15);
  }
  __host__ __device__ int64_t lse_index(int h, int j, int m) const {
    return ((int64_t)h * n_parts + j) * rows + m;
  }
};

struct DecodeArgs {
  const bf16* q;
  int64_t q_tok_stride;  // elements
  const bf16* k_cache;
  const bf16* v_cache;
  int64_t kv_tok_stride;  // elements (= Hkv * D)
  int64_t num_pages;      // rows of the per-layer caches; other page ids read as zeros
  const int32_t* indices;
  const int32_t* cu_k;
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t group;
  float scale_log2;
  // shared prefix (cascade) work: chunks x kv-heads x row groups
  int32_t prefix_len;
  int32_t chunk_len;
  int32_t n_chunks;
  int32_t m_rows;      // batch * group
  int32_t m_groups;
  int32_t prefix_wgs;  // n_chunks * Hkv * m_groups
  // per-row suffix work: (row, kv-head, split) items, one wavefront each
  int32_t split_len;
  int32_t n_splits;
  int32_t suffix_items;  // batch * Hkv * n_splits
  int32_t final_out;     // 1: a single part per (row, head): write bf16 out directly
  int32_t wave_parts;    // 1: each suffix wavefront writes its own part (no merge)
  PartsArgs parts;
  bf16* out;  // [B][Hq][D]
  // Fused KV append (null k_new: none).  Row b's last KV position is its new
  // token: read from k_new / v_new and written to page out_loc[b].
  const bf16* k_new;
  const bf16* v_new;
  int64_t k_new_stride;  // elements per token
  int64_t v_new_stride;
  const int32_t* out_loc;
  // Per-head q / k RMSNorm + RoPE on load (null q_norm: q and k_new are
  // final).  q and k_new are then the raw projections; row b is rotated by
  // the rows of rope_cos / rope_sin [rope_rows][D] (bf16) at positions[b]
  // (clamped).
  const bf16* q_norm;
  const bf16* k_norm;
  const bf16* rope_cos;
  const bf16* rope_sin;
  int64_t rope_rows;
  const int32_t* positions;
  float norm_eps;
};

struct PrefillArgs {
  const bf16* q;
  int64_t q_tok_stride;
  const bf16* k_cache;
  const bf16* v_cache;
  int64_t kv_tok_stride;
  int64_t num_pages;
  const int32_t* indices;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t group;
  float scale_log2;
  int32_t q_tile;   // query tokens per workgroup
  int32_t q_tiles;  // query tiles of the longest request
  int32_t batch;
  bf16* out;
};

hipError_t kv_append(void* k_cache, void* v_cache, int64_t num_slots, int64_t cache_stride_b,
                     const int32_t* out_loc, const void* k, int64_t k_stride_b, const void* v,
                     int64_t v_stride_b, int64_t n_tokens, int64_t row_bytes,
                     hipStream_t stream);

hipError_t build_indices(const int32_t* page_table, int64_t pt_stride, const int32_t* row_ids,
                         const int32_t* cu_k, int32_t batch, int32_t max_len,
                         int32_t* indices, hipStream_t stream);

hipError_t rmsnorm(const void* x, int64_t x_stride, void* residual, int64_t r_stride,
                   const void* w, void* out, int64_t out_stride, int64_t rows, int hidden,
                   float eps, hipStream_t stream);
bool rmsnorm_supported(int hidden);

hipError_t qk_norm_rope(const void* qkv, int64_t stride, int64_t tokens, int hq, int hkv, int D,
                        const void* qw, const void* kw, const float* cos_t, const float* sin_t,
                        int64_t table_rows, const int32_t* positions, void* q_out, void* k_out,
                        float eps, hipStream_t stream);

hipError_t silu_mul(const void* x, int64_t x_stride, int64_t rows, int inter, void* out,
                    int64_t out_stride, hipStream_t stream);

// Few-row GEMM y = x W^T with an optional prologue producing x and an
// optional epilogue (see gemm_skinny.hip): prologue 0 plain, 1 residual-add
// RMSNorm; epilogue 0 store, 1 SiLU of the gate half times the up half.
struct LinearArgs {
  const bf16* x;
  int64_t x_stride;
  const bf16* w;  // [N][K], or [2N][K] (gate rows, then up rows) for the SiLU pair
  int64_t w_stride;
  bf16* y;        // [M][N]
  int64_t y_stride;
  int32_t M;
  int32_t K;
  int64_t N;
  const bf16* residual;  // prologue 1 (may be null)
  int64_t r_stride;
  const bf16* norm_w;    // prologue 1
  float eps;
  bf16* residual_out;    // prologue 1: bf16(x + residual) (may be null)
  int64_t ro_stride;
};
// Device state of a captured CandidateGroup decode step.
struct CgStepArgs {
  int32_t rows;
  int64_t* step;            // [1] step index (device)
  const int32_t* pages;     // [page_rows][rows] page of each row per step
  int32_t page_rows;
  int32_t* out_loc;         // [rows]
  int32_t* page_table;      // [rows][pt_stride]
  int64_t pt_stride;
  int32_t pt_cols;
  int32_t* pos;             // [rows]
  const int64_t* tok;       // [rows] the step's pick
  const float* raw;         // [rows] its raw log-prob
  int64_t eos;              // -1: none
  uint8_t* finished;        // [rows] bool
  uint8_t* eos_hit;         // [rows] bool
  int64_t* out_ids;         // [rows][out_stride]
  int64_t out_stride;
  int32_t out_cols;
  float* logp_sum;          // [rows]
  int64_t* counts;          // [rows]
  int64_t* tokens;          // [rows] next input ids
  int64_t* fed;             // [1] live rows fed so far
  // cg_step_prepare: the step's decode metadata and inputs
  int32_t* cu_k;            // [rows + 1]
  int32_t* indices;         // [rows * max_kv_len]
  int32_t max_kv_len;
  int64_t* step_next;       // [1] *step + 1 (may be null)
  const bf16* embed;        // [vocab][hidden] (null: no embedding gather)
  int64_t vocab;
  int32_t hidden;
  bf16* h_out;              // [rows][hidden]
};
hipError_t cg_step_begin(const CgStepArgs& a, hipStream_t stream);
hipError_t cg_step_prepare(const CgStepArgs& a, hipStream_t stream);
hipError_t cg_step_end(const CgStepArgs& a, hipStream_t stream);
bool skinny_gemm_supported(int64_t M, int64_t N, int64_t K);
bool skinny_gemm_norm_supported(int64_t M, int64_t K);
hipError_t skinny_gemm(const LinearArgs& a, int prologue, int epilogue, hipStream_t stream);

hipError_t greedy_select(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                         int32_t elem_bytes, int64_t* token_out, float* logprob_out,
                         hipStream_t stream);

// Stateless candidate sampling (sampling.hip).  One workgroup per row.
struct SampleArgs {
  const void* logits;
  int64_t row_stride;  // elements
  int32_t rows;
  int32_t vocab;
  int32_t elem_bytes;  // 2: bf16, 4: fp32
  float temperature;
  int32_t top_k;       // 0: every id (then top_p must be 1)
  float top_p;
  int32_t greedy;      // argmax of the sampling logits
  const float* uniforms;   // u of row r at uniforms[r * uniform_stride + step]
  int64_t uniform_stride;
  int32_t uniform_count;   // columns of the table (the step is clamped into them)
  const int64_t* step;     // device scalar (may be null: step 0)
  const int32_t* forbidden;  // ids blocked while step < forbid_before_step
  int32_t n_forbidden;
  int32_t forbid_before_step;
  const int64_t* forbidden_by_row;  // [rows][row_forbidden_count] (may be null)
  int32_t row_forbidden_count;
  int64_t* token_out;
  float* logprob_out;
};
constexpr int kSampleMaxTopK = 1024;
constexpr int kSampleMaxForbidden = 256;
hipError_t sample_rows(const SampleArgs& a, hipStream_t stream);
hipError_t stateless_uniforms(const int64_t* seeds, int32_t rows, int32_t steps, float* out,
                              hipStream_t stream);

// Block-AttnRes depth mix (attnres.hip).  bank [bank_sources][num_tokens]
// [hidden] and every [num_tokens][hidden] plane contiguous bf16.
struct AttnResArgs {
  const bf16* bank;
  int32_t bank_sources;
  int64_t num_tokens;
  int32_t hidden;
  const bf16* partial;  // may be null
  const bf16* delta;    // may be null: partial source = bf16(partial + delta)
  bf16* partial_out;    // receives the formed partial (may be null)
  const float* wq;      // [hidden] query * key-norm weight
  float eps;
  float* scores;  // [total sources][num_tokens] (may be null)
  bf16* out;
};
bool attnres_supported(int hidden, int total_sources);
hipError_t attnres_mix(const AttnResArgs& a, hipStream_t stream);

// Wavefronts of a suffix workgroup, and the KV positions it gathers per pass
// (one 32-position engine sub-tile per wavefront).
constexpr int kSuffixWaves = 4;
constexpr int kSuffixPass = 128;

// One launch: prefix-chunk workgroups (MFMA tile engine) followed by suffix
// workgroups (one (row, head, split) item per workgroup).
hipError_t launch_decode_main(int D, const DecodeArgs& a, hipStream_t stream);

// Log-sum-exp merge of every part of each (row, kv-head) into bf16 out.
hipError_t launch_decode_combine(int D, const DecodeArgs& a, hipStream_t stream);

hipError_t launch_prefill(int D, int NW, const PrefillArgs& a, int q_tiles, int batch,
                          hipStream_t stream);

bool head_dim_supported(int D);
bool group_supported(int G);

}  // namespace aios
