// Per-step state of a captured CandidateGroup decode step, on the device:
// the bookkeeping around the model of ImeCompletionEngine's branch loop
// (python/aios/ime.py:1010-1054) in one launch before and one after the
// model instead of a dozen elementwise launches.
#include "kernels.hpp"

namespace aios {
namespace {

constexpr int kStateThreads = 256;

// out_loc[r] = pages[step][r]; page_table[r][pos[r]] = out_loc[r].
__global__ __launch_bounds__(kStateThreads) void cg_step_begin_kernel(CgStepArgs a) {
  const int64_t s = min(max(*a.step, (int64_t)0), (int64_t)a.page_rows - 1);
  for (int r = threadIdx.x; r < a.rows; r += kStateThreads) {
    const int32_t loc = a.pages[s * a.rows + r];
    a.out_loc[r] = loc;
    const int32_t p = a.pos[r];
    if (p >= 0 && p < a.pt_cols) a.page_table[(int64_t)r * a.pt_stride + p] = loc;
  }
}

// cg_step_begin's page-table column, then everything else the step reads
// before the model, in one launch: with L = pos[0] + 1 (every row of the
// group sits at the same position; clamped to [0, max_kv_len]),
// cu_k[b] = b * L, indices[b * L + j] = page_table[b][j] (the column being
// written this step taken from out_loc directly, so no thread reads what
// another writes), *step_next = *step + 1, and the embedding rows
// h_out[r] = embed[tokens[r]] (ids clamped to the table).  One thread per
// output element; the grid covers the largest of the three ranges.
__global__ __launch_bounds__(kStateThreads) void cg_step_prepare_kernel(CgStepArgs a) {
  const int64_t step = *a.step;
  const int64_t s = min(max(step, (int64_t)0), (int64_t)a.page_rows - 1);
  const int32_t L = min(max(a.pos[0] + 1, 0), a.max_kv_len);
  const int64_t tid = (int64_t)blockIdx.x * kStateThreads + threadIdx.x;
  const int64_t nth = (int64_t)gridDim.x * kStateThreads;
  for (int64_t r = tid; r < a.rows; r += nth) {
    const int32_t loc = a.pages[s * a.rows + r];
    a.out_loc[r] = loc;
    const int32_t p = a.pos[r];
    if (p >= 0 && p < a.pt_cols) a.page_table[r * a.pt_stride + p] = loc;
  }
  for (int64_t b = tid; b <= a.rows; b += nth) a.cu_k[b] = (int32_t)(b * L);
  const int64_t n_idx = (int64_t)a.rows * L;
  for (int64_t i = tid; i < n_idx; i += nth) {
    const int64_t b = i / L;
    const int32_t j = (int32_t)(i - b * L);
    a.indices[i] = j == a.pos[b] ? a.pages[s * a.rows + b] : a.page_table[b * a.pt_stride + j];
  }
  if (tid == 0 && a.step_next != nullptr) *a.step_next = step + 1;
  if (a.embed != nullptr) {
    const int32_t cpr = a.hidden / 8;  // 16-byte chunks per row
    const int64_t n_ch = (int64_t)a.rows * cpr;
    for (int64_t c = tid; c < n_ch; c += nth) {
      const int64_t r = c / cpr;
      const int64_t k = c - r * cpr;
      const int64_t t = min(max(a.tokens[r], (int64_t)0), a.vocab - 1);
      *reinterpret_cast<uint4*>(a.h_out + r * a.hidden + k * 8) =
          *reinterpret_cast<const uint4*>(a.embed + t * a.hidden + k * 8);
    }
  }
}

// Row r of the step's pick (tok, raw): emitted unless finished or EOS;
// out_ids[r][step + 1], the score sum and count take it; EOS finishes the
// row; tokens / positions advance; fed counts the rows that were live; the
// step counter advances last.
__global__ __launch_bounds__(kStateThreads) void cg_step_end_kernel(CgStepArgs a) {
  __shared__ int live_rows;
  if (threadIdx.x == 0) live_rows = 0;
  __syncthreads();
  const int64_t step = *a.step;
  const int64_t col = step + 1;
  int live_here = 0;
  for (int r = threadIdx.x; r < a.rows; r += kStateThreads) {
    const int64_t t = a.tok[r];
    const bool live = a.finished[r] == 0;
    live_here += live ? 1 : 0;
    const bool hit = live && a.eos >= 0 && t == a.eos;
    const bool emitted = live && !hit;
    if (col >= 0 && col < a.out_cols) a.out_ids[(int64_t)r * a.out_stride + col] = emitted ? t : -1;
    if (emitted) {
      a.logp_sum[r] += a.raw[r];
      a.counts[r] += 1;
    }
    if (hit) {
      a.eos_hit[r] = 1;
      a.finished[r] = 1;
    }
    a.tokens[r] = t;
    a.pos[r] += 1;
  }
  if (live_here) atomicAdd(&live_rows, live_here);
  __syncthreads();
  if (threadIdx.x == 0) {
    *a.fed += live_rows;
    *a.step = step + 1;
  }
}

}  // namespace

hipError_t cg_step_begin(const CgStepArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(cg_step_begin_kernel, dim3(1), dim3(kStateThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t cg_step_prepare(const CgStepArgs& a, hipStream_t stream) {
  int64_t work = (int64_t)a.rows * a.max_kv_len;
  if (a.rows + 1 > work) work = a.rows + 1;
  if (a.embed != nullptr && (int64_t)a.rows * (a.hidden / 8) > work) work = (int64_t)a.rows * (a.hidden / 8);
  int64_t blocks = (work + kStateThreads - 1) / kStateThreads;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(cg_step_prepare_kernel, dim3((unsigned)blocks), dim3(kStateThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t cg_step_end(const CgStepArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(cg_step_end_kernel, dim3(1), dim3(kStateThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace aios
