// extern "C" entry points declared in include/qste_hip.h: argument checks,
// workspace carving and kernel dispatch.  Nothing here allocates or
// synchronizes; every launch goes on the caller's stream.
#include "common.hpp"

namespace qste {
int launch_pack_coordinate(const int8_t*, uint8_t*, int64_t, int64_t, hipStream_t);
int launch_unpack_rows(const uint8_t*, const float*, void*, int, int64_t, int64_t, hipStream_t);
int launch_pack_affine_rows(const void*, int, uint8_t*, float*, float*, int64_t, int64_t, hipStream_t);
int simt_linear_forward(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t,
                        int64_t, int64_t, hipStream_t);
int simt_linear_dgrad(const void*, int, const uint8_t*, const float*, void*, int64_t, int64_t, int64_t,
                      hipStream_t);
int simt_evidence(const void*, int, const uint8_t*, const float*, float*, int64_t, int64_t, int64_t,
                  const float*, const float*, const uint8_t*, float*, hipStream_t);
int simt_evidence_tiles(int64_t cols);
int launch_row_inner(const float*, const uint8_t*, float*, int64_t, int64_t, hipStream_t);
int launch_sum_partials(const float*, int64_t, int64_t, float*, hipStream_t);
int colsum_chunks(int64_t samples);
int launch_colsums(const void*, int, const float*, int64_t, int64_t, float*, float*, float*, float*,
                   hipStream_t);
size_t coordinate_update_workspace(int64_t, int64_t, int64_t);
size_t coordinate_update_scalars_offset(int64_t, int64_t, int64_t);
size_t coordinate_update_static_limit();
int coordinate_update_one_launch(int64_t, int64_t, int64_t);
int launch_stream_read(const void*, int64_t, uint32_t*, int64_t, hipStream_t);
int launch_clock_probe(int64_t*, int64_t, hipStream_t);
int device_info(int64_t*);
int launch_coordinate_update_static(const float*, int8_t*, uint8_t*, int8_t*, uint16_t*, uint16_t*, uint16_t*,
                                    int64_t, int64_t, double, double, double, double, int64_t, int64_t, int64_t,
                                    const int64_t*, int64_t*, const uint8_t*, hipStream_t);
int launch_coordinate_update(const float*, int8_t*, uint8_t*, int8_t*, uint16_t*, uint16_t*, uint16_t*,
                             int64_t, int64_t, double, double, double, double, int64_t, int64_t, int64_t,
                             const int64_t*, int64_t*, const uint8_t*, void*, size_t, hipStream_t);
// MFMA paths (gemm_mfma.hip): return 1 when the shape/dtype is not theirs.
int mfma_linear_forward(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t,
                        int64_t, int64_t, hipStream_t);
int mfma_linear_dgrad(const void*, int, const uint8_t*, const float*, void*, int64_t, int64_t, int64_t,
                      hipStream_t);
int mfma_linear_dgrad_t(const void*, int, const uint8_t*, int64_t, const uint16_t*, void*, int64_t, int64_t,
                        int64_t, hipStream_t);
int mfma_evidence(const void*, int, const uint8_t*, const float*, float*, int64_t, int64_t, int64_t,
                  const float*, const float*, const uint8_t*, float*, const EvidencePlan*, float*, hipStream_t);
int mfma_evidence_t(const void*, int, const uint8_t*, int64_t, const uint16_t*, float*, int64_t, int64_t, int64_t,
                    const float*, const float*, const uint8_t*, float*, const EvidencePlan*, float*, hipStream_t);
int64_t mfma_evidence_tiles(int64_t cols);
bool mfma_pair_ok(const void*, int, int64_t, int64_t, int64_t);
EvidencePlan mfma_evidence_plan(int64_t, int64_t, int64_t, bool);
int mfma_backward_pair(const void*, int, const uint8_t*, int64_t, const uint16_t*, float*, const uint8_t*, int64_t,
                       const uint16_t*, const uint8_t*, void*, int64_t, int64_t, int64_t, const float*,
                       const float*, float*, const EvidencePlan&, float*, hipStream_t);
int launch_transpose_bits(const uint8_t*, uint8_t*, int64_t, int64_t, int64_t, int64_t, hipStream_t);
int launch_f32_to_16(const float*, uint16_t*, int64_t, int64_t, int, hipStream_t);
int gemv_linear_forward(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t,
                        int64_t, int64_t, hipStream_t);
int launch_swiglu_forward(const void*, const void*, int, void*, uint8_t*, float*, float*, int64_t, int64_t,
                          hipStream_t);
int launch_swiglu_backward(const void*, const void*, const void*, int, void*, void*, int64_t, hipStream_t);
int launch_row_scale(const void*, int, void*, void*, int64_t, float, float, hipStream_t);
size_t swiglu_backward_sums_workspace(int64_t, int64_t);
int launch_swiglu_backward_sums(const void*, const void*, const void*, int, void*, void*, const float*, const float*,
                                int64_t, int64_t, float*, float*, hipStream_t, int64_t);
int launch_row_scale_backward(const void*, const void*, int, void*, int64_t, float, float, hipStream_t);
// fp32 products through bf16 limbs (gemm_mfma.hip): 0 bytes / return 1 when
// the shape is not for them
size_t f32_forward_workspace(int64_t, int64_t, int64_t);
size_t mfma_forward_split_workspace(int64_t, int64_t, int64_t, int);
int mfma_linear_forward_split(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t, int64_t,
                              int64_t, void*, size_t, hipStream_t);
int mfma_f32_forward(const float*, const uint8_t*, const float*, const float*, float*, int64_t, int64_t, int64_t,
                     void*, size_t, hipStream_t);
size_t f32_dgrad_workspace(int64_t, int64_t, int64_t);
int mfma_f32_dgrad(const float*, const uint8_t*, const float*, float*, int64_t, int64_t, int64_t, void*, size_t,
                   hipStream_t);
size_t f32_evidence_workspace(int64_t, int64_t, int64_t);
int mfma_f32_evidence(const float*, const uint8_t*, const float*, float*, int64_t, int64_t, int64_t, const float*,
                      const float*, const uint8_t*, float*, void*, size_t, hipStream_t);
}  // namespace qste

using namespace qste;

namespace {

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }
inline bool dtype_ok(int d) { return d == QSTE_F32 || d == QSTE_F16 || d == QSTE_BF16; }
inline size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

struct BackwardLayout {
  size_t v_part, db_part, v, gs_part, w_t, x_t, s16, xs16, partial, limbs, limb_bytes, total;
  int64_t chunks, tiles;
  int64_t w_t_pitch, x_t_pitch;  // bytes per row of the transposed sign copies
};

// with_limbs: room for fp32 dy's bf16 limbs (the dX and evidence products
// take turns in it)
BackwardLayout backward_layout(int64_t samples, int64_t rows, int64_t cols, bool with_limbs = false) {
  BackwardLayout l{};
  l.chunks = colsum_chunks(samples);
  int64_t tiles = simt_evidence_tiles(cols);
  const int64_t mt = mfma_evidence_tiles(cols);
  if (mt > tiles) tiles = mt;
  l.tiles = tiles;
  size_t at = 0;
  l.v_part = at; at += align_up(sizeof(float) * static_cast<size_t>((l.chunks > 0 ? l.chunks : 1) * rows));
  l.db_part = at; at += align_up(sizeof(float) * static_cast<size_t>((l.chunks > 0 ? l.chunks : 1) * rows));
  l.v = at; at += align_up(sizeof(float) * static_cast<size_t>(rows));
  l.gs_part = at; at += align_up(sizeof(float) * static_cast<size_t>(tiles * rows));
  // transposed signs (bits along K, rows padded to 64-bit words) and bf16
  // scales for the grouped MFMA products
  l.w_t_pitch = (rows + 63) / 64 * 8;
  l.x_t_pitch = (samples + 63) / 64 * 8;
  l.w_t = at; at += align_up(static_cast<size_t>(cols * l.w_t_pitch));
  l.x_t = at; at += align_up(static_cast<size_t>(cols * l.x_t_pitch));
  l.s16 = at; at += align_up(sizeof(uint16_t) * static_cast<size_t>((rows + 63) / 64 * 64));
  l.xs16 = at; at += align_up(sizeof(uint16_t) * static_cast<size_t>((samples + 63) / 64 * 64));
  // split-K partials of the evidence: room for the larger of the plans with
  // and without the input gradient
  int64_t partial = mfma_evidence_plan(samples, rows, cols, true).partial_bytes;
  const int64_t alone = mfma_evidence_plan(samples, rows, cols, false).partial_bytes;
  if (alone > partial) partial = alone;
  l.partial = at; at += align_up(static_cast<size_t>(partial));
  l.limb_bytes = 0;
  if (with_limbs) {
    const size_t d = f32_dgrad_workspace(samples, rows, cols), e = f32_evidence_workspace(samples, rows, cols);
    l.limb_bytes = d > e ? d : e;
  }
  l.limbs = at; at += align_up(l.limb_bytes);
  l.total = at;
  return l;
}

int forward_dispatch(const void* x, int dtype, const uint8_t* packed, const float* scale,
                     const float* bias, void* y, int64_t m, int64_t rows, int64_t cols, hipStream_t s) {
  int rc = gemv_linear_forward(x, dtype, packed, scale, bias, y, m, rows, cols, s);
  if (rc != 1) return rc;
  rc = mfma_linear_forward(x, dtype, packed, scale, bias, y, m, rows, cols, s);
  if (rc != 1) return rc;
  return simt_linear_forward(x, dtype, packed, scale, bias, y, m, rows, cols, s);
}

int dgrad_dispatch(const void* dy, int dtype, const uint8_t* packed, const float* row_scale, void* dx,
                   int64_t m, int64_t rows, int64_t cols, hipStream_t s) {
  int rc = mfma_linear_dgrad(dy, dtype, packed, row_scale, dx, m, rows, cols, s);
  if (rc != 1) return rc;
  return simt_linear_dgrad(dy, dtype, packed, row_scale, dx, m, rows, cols, s);
}

int evidence_dispatch(const void* dy, int dtype, const uint8_t* packed_x, const float* x_scale,
                      float* ev, int64_t samples, int64_t rows, int64_t cols, const float* m_add,
                      const float* m_scale, const uint8_t* w_bits, float* gs_part, const EvidencePlan* plan,
                      float* partial, int64_t* tiles, hipStream_t s) {
  int rc = mfma_evidence(dy, dtype, packed_x, x_scale, ev, samples, rows, cols, m_add, m_scale, w_bits,
                         gs_part, plan, partial, s);
  if (rc != 1) {
    *tiles = mfma_evidence_tiles(cols);
    return rc;
  }
  *tiles = simt_evidence_tiles(cols);
  return simt_evidence(dy, dtype, packed_x, x_scale, ev, samples, rows, cols, m_add, m_scale, w_bits,
                       gs_part, s);
}

// A zero-fill that is a kernel, so the library records no memset node when
// a caller captures it into a graph.
__global__ void fill_zero_kernel(float* p, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}
__global__ void set_i64_kernel(int64_t* p, int64_t v) { *p = v; }

int fill_zero(float* p, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  fill_zero_kernel<<<ceil_div(n, 256), 256, 0, s>>>(p, n);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

extern "C" {

int qste_version(void) { return 2; }

const char* qste_error_string(int code) {
  switch (code) {
    case 0: return "success";
    case QSTE_E_DTYPE: return "qste: unsupported dtype code";
    case QSTE_E_SHAPE: return "qste: invalid shape (negative size or inconsistent dimensions)";
    case QSTE_E_NULL: return "qste: required pointer is NULL";
    case QSTE_E_WORKSPACE: return "qste: workspace missing or smaller than the *_workspace_bytes query";
    case QSTE_E_BLOCK: return "qste: momentum block size must be positive";
    case QSTE_E_ALIGN: return "qste: pointer alignment not supported";
    case QSTE_E_SCRATCH:
      return "qste: surface too large for the library's static scratch (qste_coordinate_update_static_limit)";
    default: return hipGetErrorString(static_cast<hipError_t>(code));
  }
}

int qste_pack_coordinate(const int8_t* coordinate, uint8_t* packed, int64_t rows, int64_t cols,
                         void* stream) {
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows * cols > 0 && (!coordinate || !packed)) return QSTE_E_NULL;
  return launch_pack_coordinate(coordinate, packed, rows, cols, as_stream(stream));
}

int qste_unpack_rows(const uint8_t* packed, const float* row_scale, void* out, int out_dtype, int64_t rows,
                     int64_t cols, void* stream) {
  if (!dtype_ok(out_dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows * cols > 0 && (!packed || !out)) return QSTE_E_NULL;
  return launch_unpack_rows(packed, row_scale, out, out_dtype, rows, cols, as_stream(stream));
}

int qste_pack_affine_rows(const void* x, int dtype, uint8_t* packed, float* offset, float* scale,
                          int64_t rows, int64_t cols, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols <= 0) return QSTE_E_SHAPE;
  if (rows > 0 && (!x || !packed || !offset || !scale)) return QSTE_E_NULL;
  return launch_pack_affine_rows(x, dtype, packed, offset, scale, rows, cols, as_stream(stream));
}

int qste_packed_linear_affine(const void* x, int dtype, const uint8_t* packed, const float* scale,
                              const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                              void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (m < 0 || rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (m * rows == 0) return 0;
  if (!y || !scale || (cols > 0 && (!x || !packed))) return QSTE_E_NULL;
  return forward_dispatch(x, dtype, packed, scale, bias, y, m, rows, cols, as_stream(stream));
}

size_t qste_packed_linear_affine_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int dtype) {
  return dtype == QSTE_F32 ? f32_forward_workspace(m, rows, cols) : mfma_forward_split_workspace(m, rows, cols, dtype);
}

int qste_packed_linear_affine_ws(const void* x, int dtype, const uint8_t* packed, const float* scale,
                                 const float* bias, void* y, int64_t m, int64_t rows, int64_t cols, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (m < 0 || rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (m * rows == 0) return 0;
  if (!y || !scale || (cols > 0 && (!x || !packed))) return QSTE_E_NULL;
  if (dtype == QSTE_F32 && cols > 0) {
    const int rc = mfma_f32_forward(static_cast<const float*>(x), packed, scale, bias, static_cast<float*>(y), m,
                                    rows, cols, workspace, workspace_bytes, as_stream(stream));
    if (rc != 1) return rc;
  } else if (cols > 0) {
    const int rc = mfma_linear_forward_split(x, dtype, packed, scale, bias, y, m, rows, cols, workspace,
                                             workspace_bytes, as_stream(stream));
    if (rc != 1) return rc;
  }
  return forward_dispatch(x, dtype, packed, scale, bias, y, m, rows, cols, as_stream(stream));
}

size_t qste_packed_transpose_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int dtype) {
  return dtype == QSTE_F32 ? f32_dgrad_workspace(m, rows, cols) : 0;
}

int qste_packed_transpose_ws(const void* dy, int dtype, const uint8_t* packed, const float* row_scale, void* dx,
                             int64_t m, int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                             void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (m < 0 || rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (m * cols == 0) return 0;
  if (!dx || (rows > 0 && (!dy || !packed))) return QSTE_E_NULL;
  if (dtype == QSTE_F32 && rows > 0 && row_scale) {
    const int rc = mfma_f32_dgrad(static_cast<const float*>(dy), packed, row_scale, static_cast<float*>(dx), m, rows,
                                  cols, workspace, workspace_bytes, as_stream(stream));
    if (rc != 1) return rc;
  }
  return dgrad_dispatch(dy, dtype, packed, row_scale, dx, m, rows, cols, as_stream(stream));
}

int qste_packed_transpose(const void* dy, int dtype, const uint8_t* packed, const float* row_scale,
                          void* dx, int64_t m, int64_t rows, int64_t cols, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (m < 0 || rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (m * cols == 0) return 0;
  if (!dx || (rows > 0 && (!dy || !packed))) return QSTE_E_NULL;
  return dgrad_dispatch(dy, dtype, packed, row_scale, dx, m, rows, cols, as_stream(stream));
}

size_t qste_evidence_from_packed_workspace_bytes(int64_t samples, int64_t rows, int64_t cols) {
  if (samples <= 0 || rows <= 0 || cols <= 0) return 0;
  return static_cast<size_t>(mfma_evidence_plan(samples, rows, cols, false).partial_bytes);
}

size_t qste_evidence_from_packed_workspace_bytes_dtype(int64_t samples, int64_t rows, int64_t cols, int dtype) {
  if (dtype == QSTE_F32) return f32_evidence_workspace(samples, rows, cols);
  return qste_evidence_from_packed_workspace_bytes(samples, rows, cols);
}

int qste_evidence_from_packed(const void* dy, int dtype, const uint8_t* packed_x, const float* row_scale,
                              float* evidence, int64_t samples, int64_t rows, int64_t cols, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (samples < 0 || rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows * cols == 0) return 0;
  if (!evidence || (samples > 0 && (!dy || !packed_x))) return QSTE_E_NULL;
  if (dtype == QSTE_F32 && samples > 0 && workspace) {
    const int rc = mfma_f32_evidence(static_cast<const float*>(dy), packed_x, row_scale, evidence, samples, rows, cols,
                                     nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes,
                                     as_stream(stream));
    if (rc != 1) return rc;
    workspace = nullptr;  // what remains for fp32 is the unsplit SIMT kernel
  }
  // without a workspace the evidence runs unsplit
  EvidencePlan plan = mfma_evidence_plan(samples, rows, cols, false);
  if (!workspace) plan.splits = 1;
  else if (workspace_bytes < static_cast<size_t>(plan.partial_bytes)) return QSTE_E_WORKSPACE;
  int64_t tiles = 0;
  return evidence_dispatch(dy, dtype, packed_x, row_scale, evidence, samples, rows, cols, nullptr, nullptr,
                           nullptr, nullptr, &plan, static_cast<float*>(workspace), &tiles, as_stream(stream));
}

int qste_packed_row_inner(const float* matrix, const uint8_t* packed, float* out, int64_t rows,
                          int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows == 0) return 0;
  if (!out || (cols > 0 && (!matrix || !packed))) return QSTE_E_NULL;
  return launch_row_inner(matrix, packed, out, rows, cols, as_stream(stream));
}

size_t qste_linear_backward_workspace_bytes(int64_t samples, int64_t rows, int64_t cols) {
  if (samples < 0 || rows < 0 || cols < 0) return 0;
  return backward_layout(samples, rows, cols).total;
}

size_t qste_linear_backward_workspace_bytes_dtype(int64_t samples, int64_t rows, int64_t cols, int dtype) {
  if (samples < 0 || rows < 0 || cols < 0) return 0;
  return backward_layout(samples, rows, cols, dtype == QSTE_F32).total;
}

namespace {

// offset_dot: sum_t dy[t, r] * x_offset[t] when the caller has it (then dy
// is not read for it), or NULL
int linear_backward_impl(const void* dy, int dtype, const uint8_t* packed_x, const float* x_offset,
                         const float* x_scale, const uint8_t* packed_w, const float* scale, void* dx,
                         float* evidence, float* grad_scale, float* grad_bias, const float* offset_dot,
                         int64_t samples, int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                         void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (samples < 0 || rows <= 0 || cols <= 0) return QSTE_E_SHAPE;
  if (!evidence || !grad_scale || !scale || !packed_w) return QSTE_E_NULL;
  if (samples > 0 && (!dy || !packed_x || !x_offset || !x_scale)) return QSTE_E_NULL;
  // fp32 takes its products through bf16 limbs when the workspace has room
  // for them (qste_linear_backward_workspace_bytes_dtype), the SIMT kernels
  // otherwise
  BackwardLayout l = backward_layout(samples, rows, cols, dtype == QSTE_F32);
  if (workspace_bytes < l.total) l = backward_layout(samples, rows, cols);
  if (!workspace || workspace_bytes < l.total) return QSTE_E_WORKSPACE;
  hipStream_t s = as_stream(stream);
  char* base = static_cast<char*>(workspace);
  float* v_part = reinterpret_cast<float*>(base + l.v_part);
  float* db_part = reinterpret_cast<float*>(base + l.db_part);
  float* v = reinterpret_cast<float*>(base + l.v);
  float* gs_part = reinterpret_cast<float*>(base + l.gs_part);
  int rc;
  if (samples > 0) {
    // the offset correction's column sums, unless the caller brings them
    // (with a bias gradient to form, dy is read for both anyway)
    if (offset_dot && !grad_bias) {
      v = const_cast<float*>(offset_dot);  // only read from here on
    } else if ((rc = launch_colsums(dy, dtype, x_offset, samples, rows, v_part, grad_bias ? db_part : nullptr, v,
                                    grad_bias, s))) {
      return rc;
    }
    // MFMA path: the plan runs evidence and dgrad in one launch (from
    // transposed copies of the signs and bf16 copies of the scales) or as
    // two, and splits evidence tiles over K where that shortens the work
    bool dgrad_done = false;
    if (mfma_pair_ok(dy, dtype, samples, rows, cols)) {
      const EvidencePlan plan = mfma_evidence_plan(samples, rows, cols, dx != nullptr);
      float* partial = reinterpret_cast<float*>(base + l.partial);
      uint8_t* w_t = reinterpret_cast<uint8_t*>(base + l.w_t);
      uint16_t* s16 = reinterpret_cast<uint16_t*>(base + l.s16);
      const int64_t pb = (cols + 7) / 8;
      if (plan.pair) {
        uint8_t* x_t = reinterpret_cast<uint8_t*>(base + l.x_t);
        uint16_t* xs16 = reinterpret_cast<uint16_t*>(base + l.xs16);
        if ((rc = launch_transpose_bits(packed_w, w_t, rows, cols, pb, l.w_t_pitch, s))) return rc;
        if ((rc = launch_transpose_bits(packed_x, x_t, samples, cols, pb, l.x_t_pitch, s))) return rc;
        if ((rc = launch_f32_to_16(scale, s16, rows, (rows + 63) / 64 * 64, dtype, s))) return rc;
        if ((rc = launch_f32_to_16(x_scale, xs16, samples, (samples + 63) / 64 * 64, dtype, s))) return rc;
        rc = mfma_backward_pair(dy, dtype, x_t, l.x_t_pitch, xs16, evidence, w_t, l.w_t_pitch, s16, packed_w, dx,
                                samples, rows, cols, v, scale, gs_part, plan, partial, s);
        if (rc == 0) return launch_sum_partials(gs_part, mfma_evidence_tiles(cols), rows, grad_scale, s);
        if (rc != 1) return rc;
      } else {
        if (dx) {
          // dgrad from transposed signs (bits along K, bf16 scales)
          if ((rc = launch_transpose_bits(packed_w, w_t, rows, cols, pb, l.w_t_pitch, s))) return rc;
          if ((rc = launch_f32_to_16(scale, s16, rows, (rows + 63) / 64 * 64, dtype, s))) return rc;
          rc = mfma_linear_dgrad_t(dy, dtype, w_t, l.w_t_pitch, s16, dx, samples, rows, cols, s);
          if (rc == 1) rc = dgrad_dispatch(dy, dtype, packed_w, scale, dx, samples, rows, cols, s);
          if (rc) return rc;
        }
        dgrad_done = true;
        // the evidence from a transposed copy of x's signs (bits along K,
        // bf16 scales), as the pair reads them
        uint8_t* x_t = reinterpret_cast<uint8_t*>(base + l.x_t);
        uint16_t* xs16 = reinterpret_cast<uint16_t*>(base + l.xs16);
        if ((rc = launch_transpose_bits(packed_x, x_t, samples, cols, pb, l.x_t_pitch, s))) return rc;
        if ((rc = launch_f32_to_16(x_scale, xs16, samples, (samples + 63) / 64 * 64, dtype, s))) return rc;
        rc = mfma_evidence_t(dy, dtype, x_t, l.x_t_pitch, xs16, evidence, samples, rows, cols, v, scale, packed_w,
                             gs_part, &plan, partial, s);
        if (rc == 0) return launch_sum_partials(gs_part, mfma_evidence_tiles(cols), rows, grad_scale, s);
        if (rc != 1) return rc;
        int64_t tiles = 0;
        if ((rc = evidence_dispatch(dy, dtype, packed_x, x_scale, evidence, samples, rows, cols, v, scale,
                                    packed_w, gs_part, &plan, partial, &tiles, s)))
          return rc;
        return launch_sum_partials(gs_part, tiles, rows, grad_scale, s);
      }
    }
    if (dtype == QSTE_F32 && l.limb_bytes > 0) {
      // the dX and evidence products take turns in the limbs' space
      void* lw = base + l.limbs;
      if (dx) {
        rc = mfma_f32_dgrad(static_cast<const float*>(dy), packed_w, scale, static_cast<float*>(dx), samples, rows,
                            cols, lw, l.limb_bytes, s);
        if (rc == 1) rc = dgrad_dispatch(dy, dtype, packed_w, scale, dx, samples, rows, cols, s);
        if (rc) return rc;
      }
      dgrad_done = true;
      rc = mfma_f32_evidence(static_cast<const float*>(dy), packed_x, x_scale, evidence, samples, rows, cols, v,
                             scale, packed_w, gs_part, lw, l.limb_bytes, s);
      if (rc == 0) return launch_sum_partials(gs_part, mfma_evidence_tiles(cols), rows, grad_scale, s);
      if (rc != 1) return rc;
    }
    if (dx && !dgrad_done && (rc = dgrad_dispatch(dy, dtype, packed_w, scale, dx, samples, rows, cols, s)))
      return rc;
  } else {
    if ((rc = fill_zero(v, rows, s))) return rc;
    if (grad_bias && (rc = fill_zero(grad_bias, rows, s))) return rc;
  }
  int64_t tiles = 0;
  if ((rc = evidence_dispatch(dy, dtype, packed_x, x_scale, evidence, samples, rows, cols, v, scale, packed_w,
                              gs_part, nullptr, nullptr, &tiles, s)))
    return rc;
  return launch_sum_partials(gs_part, tiles, rows, grad_scale, s);
}

}  // namespace

int qste_linear_backward(const void* dy, int dtype, const uint8_t* packed_x, const float* x_offset,
                         const float* x_scale, const uint8_t* packed_w, const float* scale, void* dx,
                         float* evidence, float* grad_scale, float* grad_bias, int64_t samples,
                         int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                         void* stream) {
  return linear_backward_impl(dy, dtype, packed_x, x_offset, x_scale, packed_w, scale, dx, evidence, grad_scale,
                              grad_bias, nullptr, samples, rows, cols, workspace, workspace_bytes, stream);
}

int qste_linear_backward_offset_dot(const void* dy, int dtype, const uint8_t* packed_x, const float* x_offset,
                                    const float* x_scale, const uint8_t* packed_w, const float* scale, void* dx,
                                    float* evidence, float* grad_scale, float* grad_bias, const float* offset_dot,
                                    int64_t samples, int64_t rows, int64_t cols, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!offset_dot) return QSTE_E_NULL;
  return linear_backward_impl(dy, dtype, packed_x, x_offset, x_scale, packed_w, scale, dx, evidence, grad_scale,
                              grad_bias, offset_dot, samples, rows, cols, workspace, workspace_bytes, stream);
}

size_t qste_swiglu_backward_sums_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return swiglu_backward_sums_workspace(rows, cols);
}

int qste_swiglu_backward_sums(const void* grad, const void* gate, const void* up, int dtype, void* grad_gate,
                              void* grad_up, const float* offset_gate, const float* offset_up, float* sums,
                              int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (cols == 0) return 0;
  if (!sums) return QSTE_E_NULL;
  hipStream_t s = as_stream(stream);
  if (rows == 0) return fill_zero(sums, 2 * cols, s);
  if (!grad || !gate || !up || !grad_gate || !grad_up || !offset_gate || !offset_up) return QSTE_E_NULL;
  if (!workspace || workspace_bytes < swiglu_backward_sums_workspace(rows, cols)) return QSTE_E_WORKSPACE;
  return launch_swiglu_backward_sums(grad, gate, up, dtype, grad_gate, grad_up, offset_gate, offset_up, rows, cols,
                                     sums, static_cast<float*>(workspace), s, cols);
}

int qste_swiglu_backward_sums_into(const void* grad, const void* gate, const void* up, int dtype, void* grads,
                                   const float* offset_gate, const float* offset_up, float* sums, int64_t rows,
                                   int64_t cols, void* workspace, size_t workspace_bytes, void* stream) {
  if (dtype != QSTE_BF16 && dtype != QSTE_F16) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (cols == 0) return 0;
  if (!sums) return QSTE_E_NULL;
  hipStream_t s = as_stream(stream);
  if (rows == 0) return fill_zero(sums, 2 * cols, s);
  if (!grad || !gate || !up || !grads || !offset_gate || !offset_up) return QSTE_E_NULL;
  if (!workspace || workspace_bytes < swiglu_backward_sums_workspace(rows, cols)) return QSTE_E_WORKSPACE;
  uint16_t* out = static_cast<uint16_t*>(grads);
  return launch_swiglu_backward_sums(grad, gate, up, dtype, out, out + cols, offset_gate, offset_up, rows, cols, sums,
                                     static_cast<float*>(workspace), s, 2 * cols);
}

size_t qste_coordinate_update_workspace_bytes(int64_t rows, int64_t cols, int64_t block_size) {
  return coordinate_update_workspace(rows, cols, block_size);
}

size_t qste_coordinate_update_scalars_offset(int64_t rows, int64_t cols, int64_t block_size) {
  return coordinate_update_scalars_offset(rows, cols, block_size);
}

int qste_coordinate_update_one_launch(int64_t rows, int64_t cols, int64_t block_size) {
  return coordinate_update_one_launch(rows, cols, block_size);
}

int qste_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t groups, void* stream) {
  return launch_stream_read(src, bytes, sink, groups, as_stream(stream));
}

int qste_clock_probe(int64_t* out, int64_t spins, void* stream) {
  return launch_clock_probe(out, spins, as_stream(stream));
}

int qste_device_info(int64_t* out) {
  if (!out) return QSTE_E_NULL;
  return device_info(out);
}

int qste_coordinate_update(const float* evidence, int8_t* coordinate, uint8_t* packed, int8_t* moment_q,
                           uint16_t* moment_scale, uint16_t* row_v, uint16_t* col_v, int64_t rows,
                           int64_t cols, double beta1, double beta2, double update_clip,
                           double coordinate_lr, int64_t block_size, int64_t seed, int64_t step,
                           const int64_t* step_device, int64_t* flips_out, const uint8_t* update_enabled,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (block_size <= 0) return QSTE_E_BLOCK;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  hipStream_t s = as_stream(stream);
  if (rows == 0 || cols == 0) {
    if (!flips_out) return 0;
    set_i64_kernel<<<1, 1, 0, s>>>(flips_out, 0);
    return static_cast<int>(hipGetLastError());
  }
  if (!evidence || !coordinate || !packed || !moment_q || !moment_scale || !row_v || !col_v)
    return QSTE_E_NULL;
  return launch_coordinate_update(evidence, coordinate, packed, moment_q, moment_scale, row_v, col_v, rows,
                                  cols, beta1, beta2, update_clip, coordinate_lr, block_size, seed, step,
                                  step_device, flips_out, update_enabled, workspace, workspace_bytes, s);
}

int qste_swiglu_forward(const void* gate, const void* up, int dtype, void* out, uint8_t* packed, float* offset,
                        float* scale, int64_t rows, int64_t cols, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows * cols == 0) return 0;
  if (!gate || !up || !out) return QSTE_E_NULL;
  if (packed && (!offset || !scale)) return QSTE_E_NULL;
  return launch_swiglu_forward(gate, up, dtype, out, packed, offset, scale, rows, cols, as_stream(stream));
}

int qste_swiglu_backward(const void* grad, const void* gate, const void* up, int dtype, void* grad_gate,
                         void* grad_up, int64_t count, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (count < 0) return QSTE_E_SHAPE;
  if (count == 0) return 0;
  if (!grad || !gate || !up || !grad_gate || !grad_up) return QSTE_E_NULL;
  return launch_swiglu_backward(grad, gate, up, dtype, grad_gate, grad_up, count, as_stream(stream));
}

int qste_row_scale(const void* log_scale, int dtype, void* scale, void* exp_value, int64_t n, float lo, float hi,
                   void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (n < 0) return QSTE_E_SHAPE;
  if (n == 0) return 0;
  if (!log_scale || !scale || !exp_value) return QSTE_E_NULL;
  return launch_row_scale(log_scale, dtype, scale, exp_value, n, lo, hi, as_stream(stream));
}

int qste_row_scale_backward(const void* exp_value, const void* grad, int dtype, void* grad_log_scale, int64_t n,
                            float lo, float hi, void* stream) {
  if (!dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (n < 0) return QSTE_E_SHAPE;
  if (n == 0) return 0;
  if (!exp_value || !grad || !grad_log_scale) return QSTE_E_NULL;
  return launch_row_scale_backward(exp_value, grad, dtype, grad_log_scale, n, lo, hi, as_stream(stream));
}

size_t qste_coordinate_update_static_limit(void) { return coordinate_update_static_limit(); }

int qste_coordinate_update_static(const float* evidence, int8_t* coordinate, uint8_t* packed,
                                  int8_t* moment_q, uint16_t* moment_scale, uint16_t* row_v, uint16_t* col_v,
                                  int64_t rows, int64_t cols, double beta1, double beta2, double update_clip,
                                  double coordinate_lr, int64_t block_size, int64_t seed, int64_t step,
                                  const int64_t* step_device, int64_t* flips_out,
                                  const uint8_t* update_enabled, void* stream) {
  if (block_size <= 0) return QSTE_E_BLOCK;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  hipStream_t s = as_stream(stream);
  if (rows == 0 || cols == 0) {
    if (!flips_out) return 0;
    set_i64_kernel<<<1, 1, 0, s>>>(flips_out, 0);
    return static_cast<int>(hipGetLastError());
  }
  if (!evidence || !coordinate || !packed || !moment_q || !moment_scale || !row_v || !col_v)
    return QSTE_E_NULL;
  return launch_coordinate_update_static(evidence, coordinate, packed, moment_q, moment_scale, row_v, col_v,
                                         rows, cols, beta1, beta2, update_clip, coordinate_lr, block_size, seed,
                                         step, step_device, flips_out, update_enabled, s);
}

}  // extern "C"
