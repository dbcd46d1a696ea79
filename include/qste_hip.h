/*
 * qste_hip.h -- C ABI of the MI355X (gfx950) binary-linear kernels.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream
 * (passed as `void*`, i.e. a hipStream_t; NULL is the default stream), runs
 * asynchronously on that stream, never synchronizes the host and never
 * allocates: scratch space, where an operation needs it, is passed in by the
 * caller through `workspace` / `workspace_bytes`, sized by the matching
 * `*_workspace_bytes` query.  Every entry returns 0 on success, a positive
 * hipError_t when a launch fails, or a negative QSTE_E_* code for an argument
 * the kernels cannot take (qste_error_string() names it).  Nothing is
 * written on an argument error.
 *
 * Layouts (the reference's own, src/qste/surface.py:67-79):
 *   packed sign  uint8 [rows, (cols + 7) / 8], bit j of byte b is column
 *                8b + j, set means +1 (value >= 0); pad bits are zero.
 *   coordinate / moment_q     int8  [rows, cols] row-major
 *   moment_scale              fp16  [ceil(rows * cols / block_size)]
 *   row_v / col_v             fp16  [rows] / [cols]
 *   activations and gradients row-major [samples, features] in `dtype`.
 *
 * Each declaration names the reference interface it replaces (file:line in
 * BleedingXiko/QSTE).  The Python binding is qste_amd/kernels/_lib.py.
 */
#ifndef QSTE_HIP_H
#define QSTE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of activations / gradients / outputs */
#define QSTE_F32 0
#define QSTE_F16 1
#define QSTE_BF16 2

/* argument errors (negative so they never collide with hipError_t) */
#define QSTE_E_DTYPE (-1)
#define QSTE_E_SHAPE (-2)
#define QSTE_E_NULL (-3)
#define QSTE_E_WORKSPACE (-4)
#define QSTE_E_BLOCK (-5)
#define QSTE_E_ALIGN (-6)
#define QSTE_E_SCRATCH (-7)

/* Library version; bumps when an entry point's contract changes. */
int qste_version(void);

/* Text for a return code of any entry point. */
const char* qste_error_string(int code);

/* Sign bits of an int8 coordinate matrix (coord >= 0 -> 1).
 * Replaces qste.kernels.pack_coordinate (src/qste/kernels/loader.py:285-289;
 * spec fallback.py:91-92). */
int qste_pack_coordinate(const int8_t* coordinate, uint8_t* packed, int64_t rows,
                         int64_t cols, void* stream);

/* Expand packed signs to +-1 (times row_scale[r] when row_scale != NULL) in
 * out_dtype, pad columns dropped: out [rows, cols].
 * Replaces qste.kernels.unpack_rows (loader.py:247-254; fallback.py:27-29). */
int qste_unpack_rows(const uint8_t* packed, const float* row_scale, void* out,
                     int out_dtype, int64_t rows, int64_t cols, void* stream);

/* One-bit affine encoding of each row of x [rows, cols] (fp32 arithmetic on
 * the dtype's values): offset = mean, bits = (x - offset >= 0),
 * scale = mean |x - offset|.
 * Replaces qste.kernels.pack_affine_rows (loader.py:278-282;
 * fallback.py:77-88), called by encode_activation (functional.py:98-115). */
int qste_pack_affine_rows(const void* x, int dtype, uint8_t* packed, float* offset,
                          float* scale, int64_t rows, int64_t cols, void* stream);

/* y [m, rows] = (x [m, cols] @ sign^T) * scale + bias, output in x's dtype,
 * fp32 accumulation, scale (fp32 [rows]) and bias (fp32 [rows] or NULL)
 * applied in fp32 after the product.  Skinny m (decode) and large m share
 * this entry.
 * Replaces qste.kernels.packed_linear_affine (loader.py:292-297;
 * fallback.py:95-108; PackedLinear.forward modules.py:114-120). */
int qste_packed_linear_affine(const void* x, int dtype, const uint8_t* packed,
                              const float* scale, const float* bias, void* y, int64_t m,
                              int64_t rows, int64_t cols, void* stream);

/* qste_packed_linear_affine with a workspace of
 * qste_packed_linear_affine_workspace_bytes(m, rows, cols, dtype) bytes
 * (0: none is used).  fp32 x then runs on the bf16 MFMA path: x splits
 * exactly into three bf16 limbs (hi + mid + lo) along K, the signs repeat
 * for each, every product is exact and the sums are the MFMA's fp32
 * accumulators -- an fp32 product, where the plain entry runs fp32 SIMT
 * code.  Where a product has few output tiles against its K (fp32 at small
 * m; bf16 / fp16 with 16 < m and at most a round of 256-row tiles), K is
 * cut into ranges whose fp32 accumulators the workspace holds, summed in
 * range order before the scale, bias and one rounding.  Other dtypes and
 * shapes behave as the plain entry.  Replaces
 * qste.kernels.packed_linear_affine (loader.py:292-297); the reference's
 * route for fp32 inputs is torch's fp32 mm on expanded signs
 * (cuda.py:1531-1597). */
size_t qste_packed_linear_affine_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int dtype);
int qste_packed_linear_affine_ws(const void* x, int dtype, const uint8_t* packed, const float* scale,
                                 const float* bias, void* y, int64_t m, int64_t rows, int64_t cols, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* dx [m, cols] = dy [m, rows] @ (row_scale (*) sign), output in dy's dtype.
 * row_scale (fp32 [rows], may be NULL) is folded into the expanded operand
 * and rounded to dy's dtype there, as the reference GPU path does
 * (src/qste/kernels/cuda.py:1585-1586).
 * Replaces qste.kernels.packed_transpose (loader.py:299-304;
 * fallback.py:111-123). */
int qste_packed_transpose(const void* dy, int dtype, const uint8_t* packed,
                          const float* row_scale, void* dx, int64_t m, int64_t rows,
                          int64_t cols, void* stream);

/* qste_packed_transpose with a workspace of
 * qste_packed_transpose_workspace_bytes(m, rows, cols, dtype) bytes: fp32 dy
 * times the row scale (one fp32 rounding) runs through bf16 limbs on the
 * MFMA path as above.  Replaces qste.kernels.packed_transpose
 * (loader.py:299-304) for fp32 inputs. */
size_t qste_packed_transpose_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int dtype);
int qste_packed_transpose_ws(const void* dy, int dtype, const uint8_t* packed, const float* row_scale, void* dx,
                             int64_t m, int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                             void* stream);

/* evidence fp32 [rows, cols] = dy[samples, rows]^T @ (row_scale (*) sign_x),
 * sign_x from packed_x uint8 [samples, (cols+7)/8]; row_scale (fp32
 * [samples], may be NULL) is rounded to dy's dtype as in cuda.py:1625.
 * workspace: NULL, or at least qste_evidence_from_packed_workspace_bytes()
 * bytes, with which output tiles whose K (= samples) chain is long against
 * the launch are split over K and summed in a fixed order (the query
 * returns 0 where no split pays).
 * Replaces qste.kernels.evidence_from_packed (loader.py:306-313;
 * fallback.py:126-138). */
size_t qste_evidence_from_packed_workspace_bytes(int64_t samples, int64_t rows, int64_t cols);
/* The workspace for a given dtype: for fp32 dy, room for its bf16 limbs
 * (dy times the sample scale, one fp32 rounding, then split as above),
 * which qste_evidence_from_packed then uses for the MFMA path. */
size_t qste_evidence_from_packed_workspace_bytes_dtype(int64_t samples, int64_t rows, int64_t cols, int dtype);
int qste_evidence_from_packed(const void* dy, int dtype, const uint8_t* packed_x,
                              const float* row_scale, float* evidence, int64_t samples,
                              int64_t rows, int64_t cols, void* workspace,
                              size_t workspace_bytes, void* stream);

/* out fp32 [rows] = sum_c matrix[r, c] * sign[r, c], matrix fp32 [rows, cols].
 * Replaces qste.kernels.packed_row_inner (loader.py:315-320;
 * fallback.py:141-148). */
int qste_packed_row_inner(const float* matrix, const uint8_t* packed, float* out,
                          int64_t rows, int64_t cols, void* stream);

/* The whole backward of one binary linear layer (QSTELinearFn.backward,
 * src/qste/functional.py:173-194) in one call:
 *   dx       [samples, cols] = dy @ (scale (*) sign_w)             (dy dtype)
 *   E0       = dy^T @ (x_scale (*) sign_x) + (dy^T @ x_offset) 1^T
 *              (decoded_evidence, functional.py:118-145)
 *   grad_scale fp32 [rows] = sum_c E0 * sign_w         (packed_row_inner)
 *   evidence fp32 [rows, cols] = E0 * scale[r]           (functional.py:190)
 *   grad_bias fp32 [rows] = sum_t dy  (written when grad_bias != NULL)
 * x_offset / x_scale are the fp32 [samples] rows of the saved aux.
 * dx may be NULL when no input gradient is wanted (autograd's
 * needs_input_grad); then that product is not computed.
 * Per shape, evidence and dx run in one launch or as two, and evidence
 * tiles whose K (= samples) chain is long against the launch are split over
 * K and summed in a fixed order in the workspace, so results do not depend
 * on scheduling.
 * Needs qste_linear_backward_workspace_bytes() bytes of workspace.
 * No counterpart as a single call in the reference: it fuses five of its
 * calls (cuda.py:1568-1688, functional.py:143, 193). */
size_t qste_linear_backward_workspace_bytes(int64_t samples, int64_t rows, int64_t cols);
/* The workspace for a given dtype: for fp32 dy it includes room for the
 * bf16 limbs of dX's and the evidence's dense operands, with which
 * qste_linear_backward runs both products on the MFMA path; given only
 * qste_linear_backward_workspace_bytes() it runs them in fp32 SIMT code. */
size_t qste_linear_backward_workspace_bytes_dtype(int64_t samples, int64_t rows, int64_t cols, int dtype);
int qste_linear_backward(const void* dy, int dtype, const uint8_t* packed_x,
                         const float* x_offset, const float* x_scale,
                         const uint8_t* packed_w, const float* scale, void* dx,
                         float* evidence, float* grad_scale, float* grad_bias,
                         int64_t samples, int64_t rows, int64_t cols, void* workspace,
                         size_t workspace_bytes, void* stream);

/* qste_linear_backward with the offset correction's column sums brought by
 * the caller: offset_dot fp32 [rows] = sum_t dy[t, r] * x_offset[t], which
 * the entry then uses instead of reading dy for it (when grad_bias is
 * requested dy is read for the bias sums anyway, and offset_dot is ignored).
 * Same outputs as qste_linear_backward when offset_dot holds what that entry
 * would sum (qste_swiglu_backward_sums produces it so).  Replaces
 * QSTELinearFn.backward (src/qste/functional.py:173-194), as that entry does;
 * the reference has no split of its column sums. */
int qste_linear_backward_offset_dot(const void* dy, int dtype, const uint8_t* packed_x, const float* x_offset,
                                    const float* x_scale, const uint8_t* packed_w, const float* scale, void* dx,
                                    float* evidence, float* grad_scale, float* grad_bias, const float* offset_dot,
                                    int64_t samples, int64_t rows, int64_t cols, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* One fused QSTE coordinate step on one surface
 * (qste.kernels.coordinate_update, loader.py:329-368; spec
 * fallback.py:158-242): factored second moment, global RMS clip, block
 * momentum through fp16 scales, hash-seeded stochastic rounding of the int8
 * coordinate, momentum requantization, sign repack and flip count.
 *   evidence      fp32 [rows, cols], read only (the reference consumes it as
 *                 scratch; this implementation does not write it)
 *   step          used when step_device == NULL, else *step_device (int64 on
 *                 the device) is read at run time (graph replay)
 *   flips_out     device int64, set to the number of sign flips (NULL: skip)
 *   update_enabled device uint8 or NULL; when it holds 0, no state is
 *                 written and flips_out is set to 0 (cuda.py:1724-1729)
 * block_size is any positive size (powers of two take the vector paths).  Needs
 * qste_coordinate_update_workspace_bytes() bytes of workspace. */
size_t qste_coordinate_update_workspace_bytes(int64_t rows, int64_t cols, int64_t block_size);
/* Diagnostics of the step above: the byte offset, inside its workspace, of
 * four fp32 values a completed call leaves there -- sqrt of the mean clamped
 * row statistic, the RMS-clip divisor, the step size (reciprocal(rms(m)) *
 * fp32(coordinate_lr), fallback.py:204-206) and rms(m).  Tests compare them
 * with the specification's.  No counterpart in the reference. */
size_t qste_coordinate_update_scalars_offset(int64_t rows, int64_t cols, int64_t block_size);
/* Diagnostics of the step above: 1 when a surface of this shape and block
 * size takes the one-launch step on the current device (every pass in one
 * kernel with grid barriers: columns a multiple of 2048, block_size a power
 * of two in 8..256, at most 256 rows per compute unit's strip), 0 when it
 * takes the multi-launch path (vector-aligned operands are needed too).
 * Both give the same results bit for bit.  No counterpart in the reference. */
int qste_coordinate_update_one_launch(int64_t rows, int64_t cols, int64_t block_size);

/* Measurement probes; no counterpart in the reference (bench.py and
 * qste_amd.device_profile() use them).
 * qste_stream_read: a plain streaming read of `bytes` (a multiple of 16, from
 * a 16-byte aligned device pointer) by `groups` workgroups of 256 threads,
 * each reading a contiguous share with eight 16-byte loads in flight per
 * thread -- the time any kernel that reads those bytes once can approach.
 * `sink` (groups * 256 words) is written only in an unlikely case.
 * qste_clock_probe: one wave runs `spins` dependent integer steps and stores
 * the shader-clock cycles (s_memtime) and 100 MHz real-time ticks
 * (s_memrealtime) they took in out[0], out[1] (device int64[3]). */
int qste_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t groups, void* stream);
int qste_clock_probe(int64_t* out, int64_t spins, void* stream);
/* What the runtime reports for the current device, into host int64[4]:
 * compute units, maximum shader clock (kHz), memory clock (kHz), LDS bytes
 * per compute unit.  No counterpart in the reference. */
int qste_device_info(int64_t* out);
int qste_coordinate_update(const float* evidence, int8_t* coordinate, uint8_t* packed,
                           int8_t* moment_q, uint16_t* moment_scale, uint16_t* row_v,
                           uint16_t* col_v, int64_t rows, int64_t cols, double beta1,
                           double beta2, double update_clip, double coordinate_lr,
                           int64_t block_size, int64_t seed, int64_t step,
                           const int64_t* step_device, int64_t* flips_out,
                           const uint8_t* update_enabled, void* workspace,
                           size_t workspace_bytes, void* stream);

/* qste_coordinate_update without a caller workspace: it allocates nothing
 * and takes no workspace argument.  No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving or training loops, harnesses that forbid
 * hipMalloc).  Its scratch is a static device array of
 * qste_coordinate_update_static_limit() bytes (16 MiB) per GPU, held until
 * the process ends; a surface whose qste_coordinate_update_workspace_bytes()
 * exceeds it is refused with QSTE_E_SCRATCH (14336 x 4096 at block 256 needs
 * about 10 MiB).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race and must not be
 * issued.  Results equal qste_coordinate_update's bit for bit. */
size_t qste_coordinate_update_static_limit(void);
int qste_coordinate_update_static(const float* evidence, int8_t* coordinate, uint8_t* packed,
                                  int8_t* moment_q, uint16_t* moment_scale, uint16_t* row_v,
                                  uint16_t* col_v, int64_t rows, int64_t cols, double beta1,
                                  double beta2, double update_clip, double coordinate_lr,
                                  int64_t block_size, int64_t seed, int64_t step,
                                  const int64_t* step_device, int64_t* flips_out,
                                  const uint8_t* update_enabled, void* stream);

/* ---- packed activations (src/qste/nn.py) ------------------------------- */

/* masked-activation kinds of qste_masked_activation */
#define QSTE_MASK_CLAMP 0    /* ReLU, ReLU6, Hardtanh: out = clamp(x), bit = lower < out (< upper) */
#define QSTE_MASK_LEAKY 1    /* LeakyReLU: out = x > 0 ? x : x * slope, bit = x > 0 */
#define QSTE_MASK_INTERVAL 2 /* Hardsigmoid: bit = lower < x (< upper) only; out unused */

/* smooth-activation kinds of qste_smooth_activation */
#define QSTE_ACT_GELU 0
#define QSTE_ACT_GELU_TANH 1
#define QSTE_ACT_SILU 2
#define QSTE_ACT_TANH 3
#define QSTE_ACT_SIGMOID 4
#define QSTE_ACT_ELU 5        /* param = alpha */
#define QSTE_ACT_CELU 6       /* param = alpha */
#define QSTE_ACT_SELU 7
#define QSTE_ACT_SOFTPLUS 8   /* param = beta (threshold 20) */
#define QSTE_ACT_MISH 9
#define QSTE_ACT_HARDSWISH 10
#define QSTE_ACT_RELU_SQUARE 11 /* relu(x)^2; uint8 payload of relu(x) */
#define QSTE_ACT_PROVIDED 12  /* derivative handed in as fp32 [rows, cols] */

/* One bit per element of a byte mask (nonzero -> 1), LSB first:
 * mask uint8 [rows, cols] -> packed uint8 [rows, (cols+7)/8], pad bits 0.
 * Replaces qste.kernels.pack_bits (src/qste/kernels/loader.py:256-260;
 * fallback.py:32-47). */
int qste_pack_bits(const uint8_t* mask, uint8_t* packed, int64_t rows, int64_t cols,
                   void* stream);

/* The 0/1 companion of unpack_rows: out [rows, cols] in out_dtype.
 * Replaces qste.kernels.unpack_bits (loader.py:270-273; fallback.py:50-54). */
int qste_unpack_bits(const uint8_t* packed, void* out, int out_dtype, int64_t rows,
                     int64_t cols, void* stream);

/* out = values where the bit is set, +0 where it is not (the GPU
 * reference's select, cuda.py:158-178).
 * Replaces qste.kernels.apply_bits (loader.py:263-267; fallback.py:57-70). */
int qste_apply_bits(const void* values, int dtype, const uint8_t* packed, void* out,
                    int64_t rows, int64_t cols, void* stream);

/* Backward of every one-bit activation: kept = bit ? grad : 0, then
 * out = kept * inside when outside == 0, else
 * out = grad * outside + kept * diff (each product and the sum rounded to the
 * dtype).  Replaces the backward bodies of _MaskedFn, _PiecewiseFn, _LeakyFn
 * and _DropoutFn (src/qste/nn.py:133-136, 168-181, 278-282, 364-368), which
 * call apply_bits and then scale in torch. */
int qste_masked_backward(const void* grad, int dtype, const uint8_t* packed, void* out,
                         int64_t rows, int64_t cols, float inside, float outside, float diff,
                         void* stream);

/* Forward of a one-bit activation and its mask in one pass (kind
 * QSTE_MASK_*; upper ignored unless has_upper).  out and x may not overlap.
 * Replaces the forward bodies of _MaskedFn, _LeakyFn and _PiecewiseFn
 * (src/qste/nn.py:119-131, 152-166, 271-276): torch's clamp / leaky_relu
 * followed by pack_bits. */
int qste_masked_activation(const void* x, int dtype, int kind, float lower, float upper,
                           int has_upper, float slope, void* out, uint8_t* packed,
                           int64_t rows, int64_t cols, void* stream);

/* Smooth activation with its derivative retained as a row-quantized byte.
 * Per row r: d = f'(x) in fp32 (from x and from y = f(x) rounded to the
 * dtype), scale[r] = max(amax_c |d|, 1e-8) / 127, payload int8 =
 * clamp(round_half_even(d / scale), -127, 127).
 *   y_given == 0: y = f(x) is computed here and written to y (y may be NULL)
 *   y_given != 0: y holds the forward output already and is read
 *   kind QSTE_ACT_PROVIDED: `derivative` (fp32 [rows, cols]) is quantized;
 *                 x and y are unused
 *   kind QSTE_ACT_RELU_SQUARE: y = relu(x)^2; the payload is uint8 of relu(x)
 *                 against max(amax, 1e-8) / 255, that arithmetic in the dtype
 * Replaces _SmoothFn.forward, _ReluSquareFn.forward and
 * _AnyElementwiseFn.forward (src/qste/nn.py:487-502, 315-323, 531-548). */
int qste_smooth_activation(const void* x, int dtype, int kind, float param, void* y,
                           int y_given, const float* derivative, void* payload, float* scale,
                           int64_t rows, int64_t cols, void* stream);

/* out = grad * (payload * scale[r]) (products rounded to the dtype); with
 * unsigned_payload, out = grad * 2 * (payload * scale[r]) (relu(x)^2).
 * Replaces _SmoothFn.backward / _ReluSquareFn.backward /
 * _AnyElementwiseFn.backward (src/qste/nn.py:504-507, 325-330, 550-555). */
int qste_smooth_backward(const void* grad, int dtype, const void* payload,
                         int unsigned_payload, const float* scale, void* out, int64_t rows,
                         int64_t cols, void* stream);

/* ---- the SwiGLU gate (no counterpart in the reference) ------------------ */

/* out = silu(gate) * up elementwise over [rows, cols] in `dtype`, each step
 * rounded where torch's F.silu(gate) * up rounds (silu rounded to the dtype,
 * then the product), so the values equal torch's.  When `packed` is not
 * NULL, every row of `out` is also given the one-bit affine encoding of
 * qste_pack_affine_rows (packed uint8 [rows, (cols+7)/8], offset and scale
 * fp32 [rows]), byte-identical to that entry on the same rows: the saved
 * activation of a binary layer that reads `out` next.
 * No counterpart in the reference, which runs torch's silu and mul (a
 * SwiGLU MLP's gate: down(silu(gate(x)) * up(x))). */
int qste_swiglu_forward(const void* gate, const void* up, int dtype, void* out, uint8_t* packed,
                        float* offset, float* scale, int64_t rows, int64_t cols, void* stream);

/* The gradients of out = silu(gate) * up over `count` elements, rounded as
 * torch's autograd of that expression rounds them: a = dtype(silu(gate)),
 * grad_up = dtype(grad * a), da = dtype(grad * up),
 * grad_gate = dtype((da * s) * (1 + gate * (1 - s))), s = sigmoid(gate).
 * No counterpart in the reference (see qste_swiglu_forward). */
int qste_swiglu_backward(const void* grad, const void* gate, const void* up, int dtype, void* grad_gate,
                         void* grad_up, int64_t count, void* stream);

/* qste_swiglu_backward over [rows, cols] that also sums its outputs for the
 * two binary layers that produced gate and up:
 *   sums[c]        = sum_t grad_gate[t, c] * offset_gate[t]
 *   sums[cols + c] = sum_t grad_up[t, c] * offset_up[t]
 * (fp32, offsets fp32 [rows]: those layers' saved input offsets), each
 * summed in the order qste_linear_backward sums its dy, so the sums are what
 * that entry would compute from grad_gate and grad_up, bit for bit: the
 * offset_dot of qste_linear_backward_offset_dot.  grad_gate and grad_up are
 * those of qste_swiglu_backward.  Needs
 * qste_swiglu_backward_sums_workspace_bytes(rows, cols) bytes of workspace.
 * No counterpart in the reference (see qste_swiglu_forward). */
size_t qste_swiglu_backward_sums_workspace_bytes(int64_t rows, int64_t cols);
int qste_swiglu_backward_sums(const void* grad, const void* gate, const void* up, int dtype, void* grad_gate,
                              void* grad_up, const float* offset_gate, const float* offset_up, float* sums,
                              int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes, void* stream);

/* qste_swiglu_backward_sums with both gradients in one [rows, 2 cols]
 * tensor, grad_gate in columns 0 .. cols-1 and grad_up in cols .. 2cols-1
 * of each row (bf16 or fp16; cols a multiple of 8, 16-byte aligned
 * operands).  Two layers that read one input then run their backward as
 * one (qste_linear_backward_offset_dot over the concatenated signs and
 * scales): their input gradients summed in one product, their evidence and
 * scale gradients as one product's row blocks, with sums as its offset_dot.
 * No counterpart in the reference (see qste_swiglu_forward). */
int qste_swiglu_backward_sums_into(const void* grad, const void* gate, const void* up, int dtype, void* grads,
                                   const float* offset_gate, const float* offset_up, float* sums, int64_t rows,
                                   int64_t cols, void* workspace, size_t workspace_bytes, void* stream);

/* ---- the learned row scale (src/qste/surface.py:84-85) ------------------- */

/* scale = clamp(exp(log_scale), lo, hi) over n rows, and exp_value = the
 * exp before the clamp (what the backward reads), all three in `dtype`
 * (fp32, fp16 or bf16, the log-scale parameter's), rounded as torch's
 * log_scale.exp().clamp(lo, hi) rounds on a tensor of that dtype (exp on
 * the fp32 value, rounded once; lo and hi as fp32; a NaN stays NaN).
 * Replaces the Surface.scale property's two torch operators
 * (src/qste/surface.py:84-85). */
int qste_row_scale(const void* log_scale, int dtype, void* scale, void* exp_value, int64_t n, float lo, float hi,
                   void* stream);

/* grad_log_scale = (lo <= exp_value <= hi ? grad : 0) * exp_value, all in
 * `dtype` (the bounds rounded to it for the comparisons): torch's autograd of exp().clamp(lo, hi) (clamp_backward, then
 * exp's backward by its result), bit for bit.  Replaces that autograd chain
 * of src/qste/surface.py:84-85. */
int qste_row_scale_backward(const void* exp_value, const void* grad, int dtype, void* grad_log_scale, int64_t n,
                            float lo, float hi, void* stream);

/* ---- binary embedding (src/qste/modules.py:68-100) ---------------------- */

/* out [count, cols] (out_dtype) = sign(packed[ids[n]]) * scale[ids[n]];
 * ids int64 [count] must lie in [0, rows) (an id outside gives a zero row;
 * the Python layer rejects such ids before the call).
 * Replaces qste.kernels.packed_embedding (cuda.py:1691-1702;
 * fallback.py:151-155). */
int qste_packed_embedding(const int64_t* ids, int64_t count, const uint8_t* packed,
                          const float* scale, void* out, int out_dtype, int64_t rows,
                          int64_t cols, void* stream);

/* Backward of the embedding (QSTEEmbeddingFn.backward,
 * src/qste/functional.py:274-286) in one call:
 *   E0 [rows, cols] = zeros.index_add_(0, ids, grad), each row summed in
 *                     ascending token order (a sequential index_add_'s fp32
 *                     sums, bit for bit)
 *   grad_scale fp32 [rows] = sum_c E0 * sign
 *   evidence fp32 [rows, cols] = E0 * scale[r]  (every row written)
 * grad [count, cols] in dtype.  Needs
 * qste_embedding_backward_workspace_bytes(count, rows) bytes of workspace.
 * No single counterpart in the reference: it fuses index_add_, packed_row_inner
 * and the scaling. */
size_t qste_embedding_backward_workspace_bytes(int64_t count, int64_t rows);
int qste_embedding_backward(const int64_t* ids, int64_t count, const void* grad, int dtype,
                            const uint8_t* packed, const float* scale, float* evidence,
                            float* grad_scale, int64_t rows, int64_t cols, void* workspace,
                            size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QSTE_HIP_H */
