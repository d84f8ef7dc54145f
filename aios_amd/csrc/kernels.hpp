// Internal launch interface shared by the kernel translation units and the
// C ABI in api.hip.
#pragma once

#include "common.hpp"

namespace aios {

struct TileArgs {
  const bf16* q;
  int64_t q_tok_stride;  // elements
  const bf16* k_cache;
  const bf16* v_cache;
  int64_t kv_tok_stride;  // elements (= Hkv * D)
  int64_t num_pages;      // rows of the per-layer caches; other page ids read as zeros
  const int32_t* indices;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t group;
  float scale_log2;
  // cascade
  int32_t prefix_len;
  int32_t chunk_len;
  int32_t m_rows;   // batch * group
  float* part_o;    // [chunks][Hkv][m_rows][D]
  float* part_lse;  // [chunks][Hkv][m_rows]
  // prefill
  bf16* out;
  int32_t q_tile;  // query tokens per workgroup
};

struct SuffixArgs {
  const bf16* q;
  int64_t q_tok_stride;
  const bf16* k_cache;
  const bf16* v_cache;
  int64_t kv_tok_stride;
  int64_t num_pages;
  const int32_t* indices;
  const int32_t* cu_k;
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  float scale_log2;
  int32_t prefix_len;
  int32_t split_len;
  int32_t num_splits;
  // prefix partials (read when finalising)
  const float* pre_o;
  const float* pre_lse;
  int32_t pre_chunks;
  int32_t m_rows;
  // suffix partials (written when num_splits > 1)
  float* suf_o;    // [batch][num_splits][Hq][D]
  float* suf_lse;  // [batch][num_splits][Hq]
  bf16* out;       // [batch][Hq][D]
};

hipError_t kv_append(void* k_cache, void* v_cache, int64_t num_slots, int64_t cache_stride_b,
                     const int32_t* out_loc, const void* k, int64_t k_stride_b, const void* v,
                     int64_t v_stride_b, int64_t n_tokens, int64_t row_bytes,
                     hipStream_t stream);

hipError_t build_indices(const int32_t* page_table, int64_t pt_stride, const int32_t* row_ids,
                         const int32_t* cu_k, int32_t batch, int32_t max_len,
                         int32_t* indices, hipStream_t stream);

hipError_t launch_cascade(int D, int NW, const TileArgs& a, int chunks, int mgroups,
                          hipStream_t stream);

hipError_t launch_prefill(int D, int NW, const TileArgs& a, int q_tiles, int batch,
                          hipStream_t stream);

// finalize: merge prefix partials and write bf16 output (num_splits == 1);
// otherwise write suffix partials for launch_combine.
hipError_t launch_suffix(int D, int G, bool finalize, const SuffixArgs& a, hipStream_t stream);

hipError_t launch_combine(int D, int G, const SuffixArgs& a, hipStream_t stream);

bool tile_supported(int D);
bool suffix_supported(int D, int G);

}  // namespace aios
