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
// library's expf, the function torch's exp kernels call (for bf16 / fp16
// tensors on the fp32 value, rounded once to the dtype); clamp keeps a NaN
// and is min(max(e, lo), hi) otherwise, rounded to the dtype; the
// backward's comparisons are against the bounds rounded to the dtype, as
// torch compares a tensor with a Python float; its product is fp32, rounded
// to the dtype.  The forward also writes e, which the backward reads (torch's
// exp backward reads its saved result, not log_scale, so an in-place update
// of log_scale between forward and backward changes neither).
#include "common.hpp"

namespace qste {
namespace rowscale {

constexpr int kThreads = 256;

template <int DT>
__global__ __launch_bounds__(kThreads) void forward_kernel(const typename Elem<DT>::T* __restrict__ log_scale,
                                                           typename Elem<DT>::T* __restrict__ scale,
                                                           typename Elem<DT>::T* __restrict__ e_out, int64_t n,
                                                           float lo, float hi) {
  using E = Elem<DT>;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float e = E::round(expf(E::load(log_scale, i)));
  E::store(e_out, i, e);
  E::store(scale, i, e != e ? e : fminf(fmaxf(e, lo), hi));
}

template <int DT>
__global__ __launch_bounds__(kThreads) void backward_kernel(const typename Elem<DT>::T* __restrict__ e_in,
                                                            const typename Elem<DT>::T* __restrict__ grad,
                                                            typename Elem<DT>::T* __restrict__ grad_log, int64_t n,
                                                            float lo, float hi) {
  using E = Elem<DT>;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float e = E::load(e_in, i);
  // torch compares a tensor with a Python float in the tensor's dtype: the
  // bounds rounded to it
  const float pass = (e >= E::round(lo) && e <= E::round(hi)) ? E::load(grad, i) : 0.0f;
  E::store(grad_log, i, pass * e);
}

}  // namespace rowscale

#define QSTE_SCALE_DT_SWITCH(dtype, ...)                                  \
  switch (dtype) {                                                       \
    case QSTE_F32: { constexpr int DT = QSTE_F32; __VA_ARGS__; } break;  \
    case QSTE_F16: { constexpr int DT = QSTE_F16; __VA_ARGS__; } break;  \
    case QSTE_BF16: { constexpr int DT = QSTE_BF16; __VA_ARGS__; } break; \
    default: return QSTE_E_DTYPE;                                        \
  }

int launch_row_scale(const void* log_scale, int dtype, void* scale, void* e, int64_t n, float lo, float hi,
                     hipStream_t stream) {
  if (n == 0) return 0;
  QSTE_SCALE_DT_SWITCH(dtype, {
    using T = typename Elem<DT>::T;
    rowscale::forward_kernel<DT><<<ceil_div(n, rowscale::kThreads), rowscale::kThreads, 0, stream>>>(
        static_cast<const T*>(log_scale), static_cast<T*>(scale), static_cast<T*>(e), n, lo, hi);
  });
  return static_cast<int>(hipGetLastError());
}

int launch_row_scale_backward(const void* e, const void* grad, int dtype, void* grad_log, int64_t n, float lo,
                              float hi, hipStream_t stream) {
  if (n == 0) return 0;
  QSTE_SCALE_DT_SWITCH(dtype, {
    using T = typename Elem<DT>::T;
    rowscale::backward_kernel<DT><<<ceil_div(n, rowscale::kThreads), rowscale::kThreads, 0, stream>>>(
        static_cast<const T*>(e), static_cast<const T*>(grad), static_cast<T*>(grad_log), n, lo, hi);
  });
  return static_cast<int>(hipGetLastError());
}
#undef QSTE_SCALE_DT_SWITCH

}  // namespace qste
