/*
 * cpu_port.c -- the work of the reference's native CPU backend
 * (src/qste/kernels/cpu.cpp) on a multi-core host, for timing only.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it on the GPU
 * box's host cores.  It is not the checker (qste_oracle.c is) and no product
 * code path calls it.
 *
 * What it computes is what cpu.cpp computes, with cpu.cpp's numerics where
 * they differ from the specification backend (fallback.py): fp32 sums, 1e-12
 * added after each mean of squares, the momentum gain folded with the clip
 * divisor, the step size as one division, requantization as rint(m * (1/S)).
 * How it computes it is this file's own, laid out for a many-core host:
 *
 *   cp_expand             packed signs -> +-1 floats by bit arithmetic (the
 *                         tile operand of the fp32 BLAS products the caller
 *                         runs, as cpu.cpp:342-456 does)
 *   cp_scale_rows         a row scale folded into an expanded tile
 *   cp_pack_affine_rows   one-bit affine encoding of fp32 rows
 *   cp_row_inner          sum_c m[r,c] * sign[r,c] per row
 *   cp_coordinate_update  the coordinate step (cpu.cpp:578-808) as four
 *                         phases, each a parallel loop over tasks of its own
 *                         shape:
 *     squares   tiles of SQ_ROWS x SQ_COLS: each tile's row and column sums
 *               of squares land in partial arrays, summed in tile order
 *     unitize   the same tiles: E scaled in place to U = E * rf * cf, and
 *               each tile's sum of U^2
 *     momentum  runs of whole momentum blocks: m = q * (s * b1) + U * gain
 *               in place of U, the new fp16 block scale, sum of m^2
 *     settle    rows: per group of eight columns the stochastic rounding,
 *               the requantization and the packed byte with its flips
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int cp_threads(void) { return omp_get_max_threads(); }
void cp_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

/* ---- sign expansion ------------------------------------------------------ */

/* bit set -> +1.0f, clear -> -1.0f: the sign bit of 1.0f set where the bit
 * is clear */
static inline float sign_of_bit(uint32_t byte, int bit) {
  const uint32_t word = 0x3F800000u | ((~byte >> bit) & 1u) << 31;
  float f;
  memcpy(&f, &word, 4);
  return f;
}

/* out [rows, stride * 8] floats; pad columns decode to -1 (the caller
 * narrows them away) */
void cp_expand(const uint8_t* packed, int64_t rows, int64_t stride, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t* from = packed + r * stride;
    float* to = out + r * stride * 8;
    for (int64_t b = 0; b < stride; ++b) {
      const uint32_t byte = from[b];
      for (int bit = 0; bit < 8; ++bit) to[8 * b + bit] = sign_of_bit(byte, bit);
    }
  }
}

/* tile[r, :width] *= scale[r] */
void cp_scale_rows(float* tile, int64_t rows, int64_t width, const float* scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float* line = tile + r * width;
    const float s = scale[r];
    for (int64_t c = 0; c < width; ++c) line[c] = line[c] * s;
  }
}

/* ---- one-bit affine encoding ---------------------------------------------- */

/* fp32 sum of n values, eight running sums added pairwise at the end */
static float sum8(const float* v, int64_t n) {
  float lane[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) lane[j] += v[i + j];
  for (int j = 0; i < n; ++i, ++j) lane[j] += v[i];
  return ((lane[0] + lane[1]) + (lane[2] + lane[3])) + ((lane[4] + lane[5]) + (lane[6] + lane[7]));
}

void cp_pack_affine_rows(const float* x, int64_t rows, int64_t cols, uint8_t* bits, float* offset,
                         float* scale) {
  const int64_t stride = (cols + 7) / 8;
  const float per = 1.0f / (float)(cols > 0 ? cols : 1);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    const float centre = sum8(row, cols) * per;
    float spread = 0.f;
    for (int64_t b = 0; b < stride; ++b) {
      const int64_t c0 = 8 * b, n = cols - c0 < 8 ? cols - c0 : 8;
      uint32_t byte = 0;
      float part = 0.f;
      for (int64_t j = 0; j < n; ++j) {
        const float d = row[c0 + j] - centre;
        byte |= (uint32_t)(d >= 0.0f) << j;
        part += fabsf(d);
      }
      bits[r * stride + b] = (uint8_t)byte;
      spread += part;
    }
    offset[r] = centre;
    scale[r] = spread * per;
  }
}

void cp_row_inner(const float* mat, const uint8_t* packed, int64_t rows, int64_t cols, float* out) {
  const int64_t stride = (cols + 7) / 8;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = mat + r * cols;
    const uint8_t* signs = packed + r * stride;
    float pos = 0.f, all = 0.f;
    for (int64_t c = 0; c < cols; ++c) {
      all += row[c];
      if ((signs[c >> 3] >> (c & 7)) & 1) pos += row[c];
    }
    out[r] = 2.0f * pos - all;  /* sum over +1 columns minus sum over -1 columns */
  }
}

/* ---- fp16 <-> fp32 (round to nearest even) --------------------------------- */

static float f16_value(uint16_t h) {
  const int e = (h >> 10) & 0x1F;
  const float frac = (float)(h & 0x3FF);
  float v;
  if (e == 0) v = ldexpf(frac, -24);
  else if (e == 31) v = (h & 0x3FF) ? NAN : INFINITY;
  else v = ldexpf(1024.0f + frac, e - 25);
  return (h & 0x8000) ? -v : v;
}

static uint16_t f16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const float a = fabsf(f);
  if (a != a) return (uint16_t)(sign | 0x7E00u);
  if (a >= 65520.0f) return (uint16_t)(sign | 0x7C00u);  /* rounds past the largest finite half */
  int e;
  frexpf(a, &e);  /* a = m * 2^e, m in [0.5, 1) */
  /* the half's unit in the last place: 2^(e - 11), not below 2^-24 */
  const int ulp_exp = e - 11 < -24 ? -24 : e - 11;
  const float q = rintf(ldexpf(a, -ulp_exp));  /* multiples of the unit, ties to even */
  const float v = ldexpf(q, ulp_exp);
  if (v == 0.0f) return sign;
  int ve;
  const float vm = frexpf(v, &ve);
  if (ve <= -14) return (uint16_t)(sign | (uint16_t)ldexpf(v, 24));  /* subnormal: v / 2^-24 */
  const uint16_t mant = (uint16_t)(ldexpf(vm, 11) - 1024.0f);
  return (uint16_t)(sign | (uint16_t)((ve + 14) << 10) | mant);
}

/* ---- the rounding stream (the reference's hash, steps in the specification) */

static inline uint32_t mix32(uint32_t v) {
  v = (v ^ 61u) ^ (v >> 16);
  v = v * 9u;
  v = v ^ (v >> 4);
  v = v * 0x27D4EB2Du;
  return v ^ (v >> 15);
}

/* ---- the coordinate step ------------------------------------------------------ */

enum { SQ_ROWS = 64, SQ_COLS = 1024, RUN_BLOCKS = 64 };

typedef struct {
  int64_t rows, cols, count, block, blocks;
  int64_t row_tiles, col_tiles;
  float b1, b2, clip, lr;
} Shape;

static void tile_span(const Shape* s, int64_t t, int64_t* r0, int64_t* r1, int64_t* c0, int64_t* c1) {
  const int64_t tr = t / s->col_tiles, tc = t % s->col_tiles;
  *r0 = tr * SQ_ROWS;
  *r1 = *r0 + SQ_ROWS < s->rows ? *r0 + SQ_ROWS : s->rows;
  *c0 = tc * SQ_COLS;
  *c1 = *c0 + SQ_COLS < s->cols ? *c0 + SQ_COLS : s->cols;
}

/* squares: row_part[tc][r] and col_part[tr][c], the tile's fp32 sums */
static void phase_squares(const Shape* s, const float* e, float* row_part, float* col_part) {
  const int64_t tiles = s->row_tiles * s->col_tiles;
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t t = 0; t < tiles; ++t) {
    int64_t r0, r1, c0, c1;
    tile_span(s, t, &r0, &r1, &c0, &c1);
    float* cp = col_part + (t / s->col_tiles) * s->cols;
    for (int64_t c = c0; c < c1; ++c) cp[c] = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
      const float* row = e + r * s->cols;
      float acc = 0.f;
      for (int64_t c = c0; c < c1; ++c) {
        const float q = row[c] * row[c];
        acc += q;
        cp[c] += q;
      }
      row_part[(t % s->col_tiles) * s->rows + r] = acc;
    }
  }
}

/* the second-moment EMA of one statistic, in place; returns the new value */
static float ema_update(uint16_t* stat, float sum, int64_t n, float b2) {
  const float v = f16_value(*stat) * b2 + (sum / (float)n + 1e-12f) * (1.0f - b2);
  *stat = f16_bits(v);
  return v;
}

/* unitize: U = E * rf[r] * cf[c] in place; returns sum U^2 */
static double phase_unitize(const Shape* s, float* e, const float* rf, const float* cf) {
  const int64_t tiles = s->row_tiles * s->col_tiles;
  double total = 0.0;
#pragma omp parallel for schedule(dynamic, 4) reduction(+ : total)
  for (int64_t t = 0; t < tiles; ++t) {
    int64_t r0, r1, c0, c1;
    tile_span(s, t, &r0, &r1, &c0, &c1);
    double tile_sum = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
      float* row = e + r * s->cols;
      const float f = rf[r];
      float acc = 0.f;
      for (int64_t c = c0; c < c1; ++c) {
        const float u = row[c] * f * cf[c];
        row[c] = u;
        acc += u * u;
      }
      tile_sum += (double)acc;
    }
    total += tile_sum;
  }
  return total;
}

/* momentum: m in place of U over runs of whole blocks; returns sum m^2 */
static double phase_momentum(const Shape* s, float* e, const int8_t* q, uint16_t* qscale, float gain) {
  const int64_t runs = (s->blocks + RUN_BLOCKS - 1) / RUN_BLOCKS;
  double total = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : total)
  for (int64_t k = 0; k < runs; ++k) {
    const int64_t b0 = k * RUN_BLOCKS, b1 = b0 + RUN_BLOCKS < s->blocks ? b0 + RUN_BLOCKS : s->blocks;
    double run_sum = 0.0;
    for (int64_t b = b0; b < b1; ++b) {
      const int64_t i0 = b * s->block, i1 = i0 + s->block < s->count ? i0 + s->block : s->count;
      const float keep = f16_value(qscale[b]) * s->b1;
      float peak = 1e-6f, acc = 0.f;
      for (int64_t i = i0; i < i1; ++i) {
        const float m = (float)q[i] * keep + e[i] * gain;
        e[i] = m;
        acc += m * m;
        peak = peak < fabsf(m) ? fabsf(m) : peak;
      }
      qscale[b] = f16_bits(peak / 127.0f);
      run_sum += (double)acc;
    }
    total += run_sum;
  }
  return total;
}

/* min(127, max(-127, v)) with the comparisons of std::max / std::min, as
 * cpu.cpp's clamps compile (a NaN gives -127), not the libm calls fminf and
 * fmaxf become without fast math */
static inline float clamp127(float v) {
  const float lo = -127.0f < v ? v : -127.0f;
  return lo < 127.0f ? lo : 127.0f;
}

/* settle: coordinates by stochastic rounding, momentum requantized against
 * the new block scales, packed signs and flips, eight columns at a time */
static int64_t phase_settle(const Shape* s, const float* m, int8_t* coord, int8_t* q, const uint16_t* qscale,
                            uint8_t* bits, float step_size, uint32_t key) {
  const int64_t stride = (s->cols + 7) / 8;
  int64_t flips = 0;
#pragma omp parallel for schedule(static) reduction(+ : flips)
  for (int64_t r = 0; r < s->rows; ++r) {
    int64_t blk = -1;
    float inv = 0.f;
    for (int64_t g = 0; g < stride; ++g) {
      const int64_t c0 = 8 * g, n = s->cols - c0 < 8 ? s->cols - c0 : 8;
      uint32_t byte = 0;
      for (int64_t j = 0; j < n; ++j) {
        const int64_t i = r * s->cols + c0 + j;
        if (i / s->block != blk) {
          blk = i / s->block;
          const float sc = f16_value(qscale[blk]);
          inv = 1.0f / (sc > 1e-12f ? sc : 1e-12f);
        }
        const float target = (float)coord[i] - m[i] * step_size;
        const float below = floorf(target);
        const float draw = (float)mix32((uint32_t)i ^ key) * (1.0f / 4294967296.0f);
        const float next = clamp127(below + (draw < target - below ? 1.0f : 0.0f));
        coord[i] = (int8_t)next;
        q[i] = (int8_t)clamp127(rintf(m[i] * inv));
        byte |= (uint32_t)(next >= 0.0f) << j;
      }
      const uint32_t keep_mask = n == 8 ? 0u : (0xFFu << n) & 0xFFu;
      const uint32_t old = bits[r * stride + g];
      flips += __builtin_popcount((old ^ byte) & ~keep_mask & 0xFFu);
      bits[r * stride + g] = (uint8_t)((old & keep_mask) | byte);
    }
  }
  return flips;
}

/* One coordinate step; `grad` is consumed as scratch (U, then m). */
int64_t cp_coordinate_update(float* grad, int8_t* coord, uint8_t* bits, int8_t* moment_int,
                             uint16_t* moment_block, uint16_t* row_stat, uint16_t* col_stat, int64_t rows,
                             int64_t columns, double beta1, double beta2, double clip, double lr,
                             int64_t block_size, int64_t seed, int64_t step) {
  Shape s;
  s.rows = rows;
  s.cols = columns;
  s.count = rows * columns;
  s.block = block_size;
  s.blocks = (s.count + block_size - 1) / block_size;
  s.row_tiles = (rows + SQ_ROWS - 1) / SQ_ROWS;
  s.col_tiles = (columns + SQ_COLS - 1) / SQ_COLS;
  s.b1 = (float)beta1;
  s.b2 = (float)beta2;
  s.clip = (float)clip;
  s.lr = (float)lr;

  float* row_part = (float*)malloc(sizeof(float) * (size_t)(s.col_tiles * rows));
  float* col_part = (float*)malloc(sizeof(float) * (size_t)(s.row_tiles * columns));
  float* rf = (float*)malloc(sizeof(float) * (size_t)rows);
  float* cf = (float*)malloc(sizeof(float) * (size_t)columns);

  phase_squares(&s, grad, row_part, col_part);
  /* row statistics, their mean, and the row factors sqrt(mean) / sqrt(R) */
  double row_total = 0.0;
  for (int64_t r = 0; r < rows; ++r) {
    float sum = 0.f;
    for (int64_t t = 0; t < s.col_tiles; ++t) sum += row_part[t * rows + r];
    rf[r] = ema_update(&row_stat[r], sum, columns, s.b2);
    row_total += rf[r];
  }
  const float row_mean = (float)(row_total / (double)rows);
  const float root_mean = sqrtf(row_mean > 1e-10f ? row_mean : 1e-10f);
  for (int64_t r = 0; r < rows; ++r) rf[r] = root_mean / sqrtf(rf[r] > 1e-10f ? rf[r] : 1e-10f);
  for (int64_t c = 0; c < columns; ++c) {
    float sum = 0.f;
    for (int64_t t = 0; t < s.row_tiles; ++t) sum += col_part[t * columns + c];
    const float v = ema_update(&col_stat[c], sum, rows, s.b2);
    cf[c] = 1.0f / sqrtf(v > 1e-10f ? v : 1e-10f);
  }

  const double u_sq = phase_unitize(&s, grad, rf, cf);
  const float u_ms = (float)(u_sq / (double)s.count);
  const float u_rms = sqrtf(u_ms > 1e-16f ? u_ms : 1e-16f);
  const float divisor = u_rms / s.clip > 1.0f ? u_rms / s.clip : 1.0f;

  const double m_sq = phase_momentum(&s, grad, moment_int, moment_block, (1.0f - s.b1) * (1.0f / divisor));
  const float m_ms = (float)(m_sq / (double)(s.blocks * block_size));
  const float step_size = s.lr / sqrtf(m_ms > 1e-16f ? m_ms : 1e-16f);

  const uint32_t key = mix32((uint32_t)seed) ^ mix32((uint32_t)step ^ 0x2545F491u);
  const int64_t flips = phase_settle(&s, grad, coord, moment_int, moment_block, bits, step_size, key);

  free(row_part);
  free(col_part);
  free(rf);
  free(cf);
  return flips;
}
