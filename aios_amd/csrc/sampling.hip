// Greedy token selection with the raw log-probability of the chosen token.
//
// One workgroup per row.  token = the first index of the row maximum of the
// logits as stored (torch's argmax on the sampling logits); logprob =
// x[token] - logsumexp(x) in fp32 (log_softmax of the fp32-widened logits,
// gathered at the token).  Each lane keeps an online (max, first index,
// sum of exp(x - max)) state over a strided slice of the row; states merge
// across the wavefront with shuffles and across waves through LDS.
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

template <typename T>
__global__ __launch_bounds__(kGreedyThreads) void greedy_kernel(
    const T* __restrict__ logits, int64_t row_stride, int32_t vocab,
    int64_t* __restrict__ token_out, float* __restrict__ logprob_out) {
  const int row = blockIdx.x;
  const T* x = logits + (int64_t)row * row_stride;
  ArgState st = {kNegInf, 0x7fffffff, 0.f};
  for (int32_t j = threadIdx.x; j < vocab; j += kGreedyThreads) {
    const float v = load_logit(x + j) * kLog2e;
    if (v > st.m) {
      st.s = (st.m == kNegInf ? 0.f : st.s * fast_exp2(st.m - v)) + 1.f;
      st.m = v;
      st.i = j;
    } else if (v != kNegInf) {
      st.s += fast_exp2(v - st.m);
    }
  }
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

}  // namespace

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
