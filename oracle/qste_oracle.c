/*
 * qste_oracle.c -- CPU restatement of QSTE's binary-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP kernels are
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; no product code path calls it.
 *
 * Every function restates the specification of the reference, which is its
 * pure-torch backend (src/qste/kernels/fallback.py, declared "the
 * specification" in CONTRIBUTING.md:26-27), with the hash taken from
 * src/qste/kernels/stream.py.  Citations are file:line in the reference.
 *
 * Float conventions, chosen so the restatement is a pure function of its
 * inputs rather than of a BLAS or thread count:
 *   - element-wise fp32 arithmetic is spelled out operation by operation and
 *     compiled with -ffp-contract=off, so every product and sum rounds where
 *     torch's does.  torch's `add_(other, alpha=a)` is a fused multiply-add on
 *     CPU (ATen ufunc add: fmadd(other, alpha, self)); it is written fmaf here.
 *   - torch reductions (`sum`, `mean`) accumulate in fp32 in an order that
 *     depends on the host's vector width.  Here every reduction accumulates in
 *     double and rounds once to fp32, i.e. the correctly rounded sum in almost
 *     every case.  `mean` is then fp32(sum) / fp32(n), which is how ATen's CPU
 *     mean is built (sum followed by div_).  Reduction-order differences are
 *     why the tests compare integer outputs with a declared rounding-margin
 *     band (see qo_coordinate_update's margin outputs).
 *   - the dense products (forward, input gradient, evidence, row inner) are
 *     accumulated in double: they are the exact-arithmetic oracle the float
 *     tolerances are stated against.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QO_SALT 0x2545F491u
#define QO_MULTIPLIER 0x27D4EB2Du

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32 with round-to-nearest-even (torch's .to(torch.float16)).    */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float qo_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24, exact in fp32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t qo_float_to_half(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t abs = u & 0x7FFFFFFFu;
  if (abs > 0x7F800000u) return (uint16_t)(sign | 0x7E00u); /* NaN */
  if (abs >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
  if (abs < 0x38800000u) {
    /* result is subnormal (or zero): units of 2^-24, RNE */
    float a = u2f(abs);
    float scaled = a * 16777216.0f; /* exact: power of two */
    float r = rintf(scaled);
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t mant = abs & 0x7FFFFFu;
  uint32_t exp = (abs >> 23) - 112u;
  uint32_t half = (exp << 10) | (mant >> 13);
  uint32_t rest = mant & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) half += 1u;
  return (uint16_t)(sign | half);
}

/* bf16 with RNE, for operand-rounded float oracles */
float qo_round_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return f;
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return u2f(u & 0xFFFF0000u);
}

/* ------------------------------------------------------------------------ */
/* The rounding stream: stream.py:41-66 (scramble, seed_hash, step_hash),   */
/* per-element draw fallback.py:210-223 / stream.py:69-83.                  */
/* ------------------------------------------------------------------------ */

uint32_t qo_scramble(uint32_t v) {
  v = (v ^ 61u) ^ (v >> 16);
  v = v + (v << 3);
  v = v ^ (v >> 4);
  v = v * QO_MULTIPLIER;
  v = v ^ (v >> 15);
  return v;
}

uint32_t qo_seed_hash(int64_t seed) { return qo_scramble((uint32_t)(uint64_t)seed); }

uint32_t qo_step_hash(int64_t step) {
  return qo_scramble(((uint32_t)(uint64_t)step) ^ QO_SALT);
}

static inline float draw(uint32_t combined, int64_t index) {
  uint32_t raw = qo_scramble(((uint32_t)(uint64_t)index) ^ combined);
  /* int -> fp32 rounds to nearest even, then an exact scale by 2^-32 */
  return (float)raw * (1.0f / 4294967296.0f);
}

void qo_uniform(int64_t seed, int64_t step, const int64_t* index, int64_t n, float* out) {
  uint32_t combined = qo_seed_hash(seed) ^ qo_step_hash(step);
  for (int64_t i = 0; i < n; ++i) out[i] = draw(combined, index[i]);
}

void qo_scramble_many(const uint32_t* v, int64_t n, uint32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = qo_scramble(v[i]);
}

/* ------------------------------------------------------------------------ */
/* Packing: fallback.py:31-48 (pack_bits, LSB first), 73-92                 */
/* ------------------------------------------------------------------------ */

void qo_pack_coordinate(const int8_t* coord, int64_t rows, int64_t cols, uint8_t* out) {
  int64_t stride = (cols + 7) / 8;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < stride; ++b) {
      uint8_t byte = 0;
      for (int64_t j = 0; j < 8; ++j) {
        int64_t c = b * 8 + j;
        if (c < cols && coord[r * cols + c] >= 0) byte |= (uint8_t)(1u << j);
      }
      out[r * stride + b] = byte;
    }
  }
}

/* unpack_rows: fallback.py:27-29 -- bit -> +1, clear -> -1, pad dropped */
void qo_unpack_rows(const uint8_t* packed, int64_t rows, int64_t cols, float* out) {
  int64_t stride = (cols + 7) / 8;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = ((packed[r * stride + c / 8] >> (c % 8)) & 1) ? 1.0f : -1.0f;
}

/* pack_affine_rows: fallback.py:77-88; used by functional.py:98-115.
 * offset = mean(x), bits = (x - offset >= 0), scale = mean |x - offset|.   */
void qo_pack_affine_rows(const float* x, int64_t rows, int64_t cols, uint8_t* bits,
                         float* offset, float* scale) {
  int64_t stride = (cols + 7) / 8;
  float n = (float)cols;
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    double sum = 0.0;
    for (int64_t c = 0; c < cols; ++c) sum += (double)row[c];
    float mean = (float)sum / n;
    double dev = 0.0;
    memset(bits + r * stride, 0, (size_t)stride);
    for (int64_t c = 0; c < cols; ++c) {
      float centered = row[c] - mean;
      dev += (double)fabsf(centered);
      if (centered >= 0.0f) bits[r * stride + c / 8] |= (uint8_t)(1u << (c % 8));
    }
    offset[r] = mean;
    scale[r] = (float)dev / n;
  }
}

/* ------------------------------------------------------------------------ */
/* Dense products in double (exact-arithmetic references).                   */
/* ------------------------------------------------------------------------ */

static inline double sign_at(const uint8_t* packed, int64_t stride, int64_t r, int64_t c) {
  return ((packed[r * stride + c / 8] >> (c % 8)) & 1) ? 1.0 : -1.0;
}

/* packed_linear_affine: fallback.py:95-108  y = (x @ sign^T) * scale + bias */
void qo_linear_fwd(const float* x, int64_t m, const uint8_t* packed, int64_t rows,
                   int64_t cols, const float* scale, const float* bias, double* y) {
  int64_t stride = (cols + 7) / 8;
  for (int64_t i = 0; i < m; ++i) {
    const float* xi = x + i * cols;
    for (int64_t r = 0; r < rows; ++r) {
      double acc = 0.0;
      const uint8_t* w = packed + r * stride;
      for (int64_t c = 0; c < cols; ++c)
        acc += ((w[c / 8] >> (c % 8)) & 1) ? (double)xi[c] : -(double)xi[c];
      acc *= (double)scale[r];
      if (bias) acc += (double)bias[r];
      y[i * rows + r] = acc;
    }
  }
}

/* packed_transpose: fallback.py:111-123  dx = dy @ (row_scale * sign)        */
void qo_linear_dgrad(const float* dy, int64_t m, const uint8_t* packed, int64_t rows,
                     int64_t cols, const float* row_scale, double* dx) {
  int64_t stride = (cols + 7) / 8;
  for (int64_t i = 0; i < m * cols; ++i) dx[i] = 0.0;
  for (int64_t i = 0; i < m; ++i) {
    double* out = dx + i * cols;
    for (int64_t r = 0; r < rows; ++r) {
      double g = (double)dy[i * rows + r];
      if (row_scale) g *= (double)row_scale[r];
      for (int64_t c = 0; c < cols; ++c) out[c] += g * sign_at(packed, stride, r, c);
    }
  }
}

/* evidence_from_packed: fallback.py:126-138
 *   E[r, c] = sum_t dy[t, r] * xs[t] * sign_x[t, c]                          */
void qo_evidence(const float* dy, int64_t samples, int64_t rows, const uint8_t* packed_x,
                 int64_t cols, const float* row_scale, double* ev) {
  int64_t stride = (cols + 7) / 8;
  for (int64_t i = 0; i < rows * cols; ++i) ev[i] = 0.0;
  for (int64_t t = 0; t < samples; ++t) {
    double s = row_scale ? (double)row_scale[t] : 1.0;
    for (int64_t r = 0; r < rows; ++r) {
      double g = (double)dy[t * rows + r] * s;
      double* out = ev + r * cols;
      for (int64_t c = 0; c < cols; ++c) out[c] += g * sign_at(packed_x, stride, t, c);
    }
  }
}

/* The rank-one offset correction of functional.py:139-144:
 *   v[r] = sum_t dy[t, r] * offset[t]                                        */
void qo_offset_correction(const float* dy, int64_t samples, int64_t rows, const float* offset,
                          double* v) {
  for (int64_t r = 0; r < rows; ++r) v[r] = 0.0;
  for (int64_t t = 0; t < samples; ++t)
    for (int64_t r = 0; r < rows; ++r) v[r] += (double)dy[t * rows + r] * (double)offset[t];
}

/* packed_row_inner: fallback.py:141-148  gs[r] = sum_c E[r, c] * sign[r, c] */
void qo_row_inner(const float* mat, const uint8_t* packed, int64_t rows, int64_t cols,
                  double* out) {
  int64_t stride = (cols + 7) / 8;
  for (int64_t r = 0; r < rows; ++r) {
    double acc = 0.0;
    for (int64_t c = 0; c < cols; ++c)
      acc += (double)mat[r * cols + c] * sign_at(packed, stride, r, c);
    out[r] = acc;
  }
}

/* ------------------------------------------------------------------------ */
/* The step size of fallback.py:204-206, `coordinate_lr / moment_rms`, with  */
/* a Python float over a 0-dim fp32 tensor.  Python hands that division to   */
/* Tensor.__rtruediv__, which torch defines as `self.reciprocal() * other`:  */
/* a correctly rounded fp32 reciprocal, then an fp32 product with the float  */
/* cast to fp32.  Two roundings; for a learning rate that is not a power of  */
/* two this differs from one fp32 division in about a quarter of cases.      */
/* ------------------------------------------------------------------------ */
float qo_step_size(float moment_rms, double coordinate_lr) {
  const float inverse = 1.0f / moment_rms;
  return inverse * (float)coordinate_lr;
}

/* ------------------------------------------------------------------------ */
/* coordinate_update: fallback.py:158-242, operation by operation.           */
/*                                                                           */
/* State arrays are updated in place exactly as the reference mutates them:  */
/* coord (int8), packed (uint8), moment_q (int8), moment_scale / row_v /     */
/* col_v (fp16 bit patterns).  `grad` is consumed as scratch (it ends up     */
/* holding the clipped update, as fallback.py:190-192 leaves it).            */
/*                                                                           */
/* Optional diagnostics (may be NULL), one float per element:                */
/*   target_margin[i] = |target - floor(target) - u|, the distance of the    */
/*                      stochastic-rounding decision from its threshold;     */
/*   moment_margin[i] = | |m/S| - floor(|m/S|) - 0.5 |, the distance of the  */
/*                      momentum requantization from a rounding tie.         */
/* They let a test prove that an integer mismatch against another           */
/* implementation sits exactly where a one-ulp difference in a reduction can */
/* move the decision.                                                        */
/*   scalars_out[0..3] = sqrt(mean clamped row statistic), RMS-clip divisor, */
/*                      step size (qo_step_size), momentum RMS.              */
/*   scale_margin[b]  = the distance, in fp16 ulps, of block b's fp32 scale  */
/*                      amax / 127 from the midpoint between its two fp16    */
/*                      neighbours: the tie a one-ulp difference in amax can */
/*                      cross, moving the stored scale (and so every q of    */
/*                      the block) by one.                                   */
/* ------------------------------------------------------------------------ */

int64_t qo_coordinate_update(float* grad, int8_t* coord, uint8_t* packed, int8_t* moment_q,
                             uint16_t* moment_scale, uint16_t* row_v, uint16_t* col_v,
                             int64_t rows, int64_t cols, double beta1, double beta2,
                             double update_clip, double coordinate_lr, int64_t block_size,
                             int64_t seed, int64_t step, float* target_margin,
                             float* moment_margin, float* scalars_out, float* scale_margin) {
  const int64_t count = rows * cols;
  const int64_t blocks = (count + block_size - 1) / block_size;
  const int64_t padded = blocks * block_size;
  const int64_t stride = (cols + 7) / 8;
  /* python scalars as torch applies them to fp32 tensors */
  const float b1 = (float)beta1, a1 = (float)(1.0 - beta1);
  const float b2 = (float)beta2, a2 = (float)(1.0 - beta2);
  const float clip = (float)update_clip;
  const float eps_sq = (float)1e-12, eps_stat = (float)1e-10;

  double* row_sum = (double*)calloc((size_t)rows, sizeof(double));
  double* col_sum = (double*)calloc((size_t)cols, sizeof(double));
  float* new_row = (float*)malloc(sizeof(float) * (size_t)rows);
  float* new_col = (float*)malloc(sizeof(float) * (size_t)cols);
  float* row_factor = (float*)malloc(sizeof(float) * (size_t)rows);
  float* col_factor = (float*)malloc(sizeof(float) * (size_t)cols);
  float* moment = (float*)malloc(sizeof(float) * (size_t)padded);
  uint8_t* previous_bits = (uint8_t*)malloc((size_t)(rows * stride) + 1);

  /* fallback.py:178-187: square = g^2 + 1e-12; factored EMA, stored fp16 */
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      float g = grad[r * cols + c];
      float sq = g * g;
      sq = sq + eps_sq;
      row_sum[r] += (double)sq;
      col_sum[c] += (double)sq;
    }
  }
  for (int64_t r = 0; r < rows; ++r) {
    float mean = (float)row_sum[r] / (float)cols;
    float decayed = qo_half_to_float(row_v[r]) * b2;
    new_row[r] = fmaf(mean, a2, decayed);
  }
  for (int64_t c = 0; c < cols; ++c) {
    float mean = (float)col_sum[c] / (float)rows;
    float decayed = qo_half_to_float(col_v[c]) * b2;
    new_col[c] = fmaf(mean, a2, decayed);
  }
  for (int64_t r = 0; r < rows; ++r) row_v[r] = qo_float_to_half(new_row[r]);
  for (int64_t c = 0; c < cols; ++c) col_v[c] = qo_float_to_half(new_col[c]);

  /* fallback.py:188-190: row/col factors, U = g * rf * cf (in place) */
  double clamped_sum = 0.0;
  for (int64_t r = 0; r < rows; ++r) clamped_sum += (double)fmaxf(new_row[r], eps_stat);
  const float sqrt_mean = sqrtf((float)clamped_sum / (float)rows);
  for (int64_t r = 0; r < rows; ++r) row_factor[r] = sqrt_mean / sqrtf(fmaxf(new_row[r], eps_stat));
  for (int64_t c = 0; c < cols; ++c) col_factor[c] = 1.0f / sqrtf(fmaxf(new_col[c], eps_stat));

  double usq = 0.0;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      float u = grad[r * cols + c] * row_factor[r];
      u = u * col_factor[c];
      grad[r * cols + c] = u;
      float s = u * u;
      usq += (double)s;
    }
  }
  /* fallback.py:191-192: global RMS clip */
  float rms = sqrtf((float)usq / (float)count);
  rms = fmaxf(rms, (float)1e-8);
  float ratio = rms / clip;
  float divisor = ratio > 1.0f ? ratio : 1.0f;
  for (int64_t i = 0; i < count; ++i) grad[i] = grad[i] / divisor;

  /* fallback.py:194-202: block momentum, decoded through its fp16 scale */
  double msq = 0.0;
  for (int64_t b = 0; b < blocks; ++b) {
    float s_old = qo_half_to_float(moment_scale[b]);
    for (int64_t j = 0; j < block_size; ++j) {
      int64_t i = b * block_size + j;
      float prev = i < count ? (float)moment_q[i] : 0.0f;
      float u = i < count ? grad[i] : 0.0f;
      float decoded = prev * s_old;
      decoded = decoded * b1;
      float m = fmaf(u, a1, decoded);
      moment[i] = m;
      float s = m * m;
      msq += (double)s;
    }
  }
  float mrms = sqrtf((float)msq / (float)padded);
  mrms = fmaxf(mrms, (float)1e-8);
  const float step_size = qo_step_size(mrms, coordinate_lr);
  if (scalars_out) {
    scalars_out[0] = sqrt_mean;
    scalars_out[1] = divisor;
    scalars_out[2] = step_size;
    scalars_out[3] = mrms;
  }

  /* fallback.py:204-225: stochastic rounding of the coordinate target */
  const uint32_t combined = qo_seed_hash(seed) ^ qo_step_hash(step);
  memcpy(previous_bits, packed, (size_t)(rows * stride));
  for (int64_t i = 0; i < count; ++i) {
    float delta = moment[i] * step_size;
    float target = (float)coord[i] - delta;
    float lower = floorf(target);
    float u = draw(combined, i);
    float frac = target - lower;
    float rounded = lower + (u < frac ? 1.0f : 0.0f);
    if (rounded > 127.0f) rounded = 127.0f;
    if (rounded < -127.0f) rounded = -127.0f;
    coord[i] = (int8_t)rounded;
    if (target_margin) target_margin[i] = fabsf(frac - u);
  }

  /* fallback.py:228-232: new fp16 block scale; requantize against it */
  for (int64_t b = 0; b < blocks; ++b) {
    float amax = 0.0f;
    for (int64_t j = 0; j < block_size; ++j) amax = fmaxf(amax, fabsf(moment[b * block_size + j]));
    float s_new = fmaxf(amax, (float)1e-6) / 127.0f;
    uint16_t h = qo_float_to_half(s_new);
    moment_scale[b] = h;
    if (scale_margin) {
      /* fp16 keeps 11 significant bits; below 2^-14 its spacing is 2^-24 */
      int e;
      frexpf(s_new, &e);
      const double ulp = ldexp(1.0, (e - 11) < -24 ? -24 : (e - 11));
      const double pos = (double)s_new / ulp - floor((double)s_new / ulp);
      scale_margin[b] = (float)fabs(pos - 0.5);
    }
    float decode = fmaxf(qo_half_to_float(h), (float)1e-12);
    for (int64_t j = 0; j < block_size; ++j) {
      int64_t i = b * block_size + j;
      if (i >= count) break;
      float ratio_q = moment[i] / decode;
      float q = rintf(ratio_q);
      if (q > 127.0f) q = 127.0f;
      if (q < -127.0f) q = -127.0f;
      moment_q[i] = (int8_t)q;
      if (moment_margin) {
        float a = fabsf(ratio_q);
        moment_margin[i] = fabsf(a - floorf(a) - 0.5f);
      }
    }
  }

  /* fallback.py:234-242: repack and count flips over valid columns */
  qo_pack_coordinate(coord, rows, cols, packed);
  int64_t flips = 0;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < stride; ++b) {
      int64_t valid = cols - b * 8;
      uint32_t mask = valid >= 8 ? 0xFFu : ((1u << valid) - 1u);
      flips += __builtin_popcount((previous_bits[r * stride + b] ^ packed[r * stride + b]) & mask);
    }
  }

  free(row_sum); free(col_sum); free(new_row); free(new_col);
  free(row_factor); free(col_factor); free(moment); free(previous_bits);
  return flips;
}
