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

hipError_t cg_step_end(const CgStepArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(cg_step_end_kernel, dim3(1), dim3(kStateThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace aios
