// The learned per-row scale of a binary layer and its gradient
// (src/qste/surface.py:84-85):
//
//   e = exp(log_scale),  s = clamp(e, lo, hi)
//   d log_scale = (lo <= e <= hi ? ds : 0) * e
//
// torch evaluates the forward as two launches (exp, clamp) and its autograd
// as six (a zero fill, two comparisons, their logical and, the where, the
// product with exp's result); here each direction is one launch over the
// rows.  Values are rounded as torch rounds them: exp is the device
// library's expf, the function torch's fp32 exp kernel calls; clamp keeps a
// NaN and is min(max(e, lo), hi) otherwise; the comparisons are fp32 against
// the bounds rounded to fp32, as torch compares an fp32 tensor with a Python
// float.  The forward also writes e, which the backward reads (torch's
// exp backward reads its saved result, not log_scale, so an in-place update
// of log_scale between forward and backward changes neither).
#include "common.hpp"

namespace qste {
namespace rowscale {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void forward_kernel(const float* __restrict__ log_scale,
                                                           float* __restrict__ scale, float* __restrict__ e_out,
                                                           int64_t n, float lo, float hi) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float e = expf(log_scale[i]);
  e_out[i] = e;
  scale[i] = e != e ? e : fminf(fmaxf(e, lo), hi);
}

__global__ __launch_bounds__(kThreads) void backward_kernel(const float* __restrict__ e_in,
                                                            const float* __restrict__ grad,
                                                            float* __restrict__ grad_log, int64_t n, float lo,
                                                            float hi) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float e = e_in[i];
  const float pass = (e >= lo && e <= hi) ? grad[i] : 0.0f;
  grad_log[i] = pass * e;
}

}  // namespace rowscale

int launch_row_scale(const float* log_scale, float* scale, float* e, int64_t n, float lo, float hi,
                     hipStream_t stream) {
  if (n == 0) return 0;
  rowscale::forward_kernel<<<ceil_div(n, rowscale::kThreads), rowscale::kThreads, 0, stream>>>(log_scale, scale,
                                                                                             e, n, lo, hi);
  return static_cast<int>(hipGetLastError());
}

int launch_row_scale_backward(const float* e, const float* grad, float* grad_log, int64_t n, float lo, float hi,
                              hipStream_t stream) {
  if (n == 0) return 0;
  rowscale::backward_kernel<<<ceil_div(n, rowscale::kThreads), rowscale::kThreads, 0, stream>>>(e, grad, grad_log,
                                                                                              n, lo, hi);
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
