/*
 * cpu_port.c -- the reference's CPU backend, restated for timing only.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it on the GPU
 * box's host cores.  It is not the checker (qste_oracle.c is) and no product
 * code path calls it.  It restates the algorithm of the reference's native
 * CPU backend, src/qste/kernels/cpu.cpp, with OpenMP in place of ATen's
 * at::parallel_for, including cpu.cpp's own numerics, which differ from the
 * specification backend (fallback.py) in small ways: +1e-12 after the mean,
 * fp32 sums, the gain folded with the clip divisor, one division for the
 * step size, rint(m * (1/S)):
 *
 *   cp_expand             byte -> eight +-1 floats through a table
 *                         (cpu.cpp:59-87), the tile operand of the BLAS
 *                         products the caller runs (cpu.cpp:342-456)
 *   cp_scale_rows         row-scale fold into an expanded tile (cpu.cpp:402)
 *   cp_pack_affine_rows   one-bit affine encoding (cpu.cpp:143-203)
 *   cp_row_inner          sum_c m[r,c] * sign[r,c] (cpu.cpp:460-496)
 *   cp_coordinate_update  the four-pass fused step (cpu.cpp:578-808)
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float g_sign_table[256 * 8];
static int g_table_ready = 0;

static const float* sign_table(void) {
  if (!g_table_ready) {
    for (int byte = 0; byte < 256; ++byte)
      for (int bit = 0; bit < 8; ++bit) g_sign_table[byte * 8 + bit] = ((byte >> bit) & 1) ? 1.0f : -1.0f;
    g_table_ready = 1;
  }
  return g_sign_table;
}

int cp_threads(void) { return omp_get_max_threads(); }
void cp_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

/* out [rows, stride * 8] floats; pad columns decode to -1 and the caller
 * narrows them away, as cpu.cpp does. */
void cp_expand(const uint8_t* packed, int64_t rows, int64_t stride, float* out) {
  const float* lut = sign_table();
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t* src = packed + r * stride;
    float* dst = out + r * stride * 8;
    for (int64_t b = 0; b < stride; ++b) memcpy(dst + b * 8, lut + src[b] * 8, 8 * sizeof(float));
  }
}

/* tile[r, :width] *= scale[r], width = stride * 8 (the tile's row pitch) */
void cp_scale_rows(float* tile, int64_t rows, int64_t width, const float* scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float s = scale[r];
    float* line = tile + r * width;
    for (int64_t c = 0; c < width; ++c) line[c] *= s;
  }
}

void cp_pack_affine_rows(const float* x, int64_t rows, int64_t cols, uint8_t* bits, float* offset,
                         float* scale) {
  const int64_t stride = (cols + 7) / 8, full = cols / 8;
  const float inverse = 1.0f / (float)(cols > 0 ? cols : 1);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + r * cols;
    uint8_t* out = bits + r * stride;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int64_t c = 0;
    for (; c + 4 <= cols; c += 4) {
      s0 += in[c];
      s1 += in[c + 1];
      s2 += in[c + 2];
      s3 += in[c + 3];
    }
    for (; c < cols; ++c) s0 += in[c];
    const float mean = (s0 + s1 + s2 + s3) * inverse;
    float d0 = 0.f, d1 = 0.f;
    for (int64_t b = 0; b < full; ++b) {
      const float* v = in + b * 8;
      uint8_t byte = 0;
      for (int j = 0; j < 8; ++j) {
        const float cen = v[j] - mean;
        if (j < 4) d0 += fabsf(cen);
        else d1 += fabsf(cen);
        byte |= (uint8_t)((cen >= 0.0f) << j);
      }
      out[b] = byte;
    }
    uint8_t tail = 0;
    for (int64_t i = full * 8; i < cols; ++i) {
      const float cen = in[i] - mean;
      d0 += fabsf(cen);
      if (cen >= 0.0f) tail |= (uint8_t)(1u << (i - full * 8));
    }
    if (full < stride) out[full] = tail;
    offset[r] = mean;
    scale[r] = (d0 + d1) * inverse;
  }
}

void cp_row_inner(const float* mat, const uint8_t* packed, int64_t rows, int64_t cols, float* out) {
  const int64_t stride = (cols + 7) / 8;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float acc = 0.f;
    for (int64_t c = 0; c < cols; ++c) {
      const float v = mat[r * cols + c];
      acc += ((packed[r * stride + c / 8] >> (c % 8)) & 1) ? v : -v;
    }
    out[r] = acc;
  }
}

/* ---- half <-> float (round to nearest even) --------------------------- */
static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t u;
  if (exp == 0) {
    const float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) u = sign | 0x7F800000u | (man << 13);
  else u = sign | ((exp + 112u) << 23) | (man << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t float_to_half(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, abs = u & 0x7FFFFFFFu;
  if (abs > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (abs >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  if (abs < 0x38800000u) {
    float a;
    memcpy(&a, &abs, 4);
    return (uint16_t)(sign | (uint32_t)rintf(a * 16777216.0f));
  }
  const uint32_t mant = abs & 0x7FFFFFu, exp = (abs >> 23) - 112u;
  uint32_t half = (exp << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) half += 1u;
  return (uint16_t)(sign | half);
}

static uint32_t scramble(uint32_t v) {
  v = (v ^ 61u) ^ (v >> 16);
  v += v << 3;
  v ^= v >> 4;
  v *= 0x27D4EB2Du;
  v ^= v >> 15;
  return v;
}

/* The four-pass step of cpu.cpp:578-808; `grad` is consumed as scratch. */
int64_t cp_coordinate_update(float* grad, int8_t* coord, uint8_t* bits, int8_t* moment_int,
                             uint16_t* moment_block, uint16_t* row_stat, uint16_t* col_stat, int64_t rows,
                             int64_t columns, double beta1_in, double beta2_in, double clip_in,
                             double lr_in, int64_t block_size, int64_t seed, int64_t step) {
  const int64_t count = rows * columns;
  const int64_t blocks = (count + block_size - 1) / block_size;
  const int64_t stride = (columns + 7) / 8;
  const float beta1 = (float)beta1_in, beta2 = (float)beta2_in;
  const float update_clip = (float)clip_in, coordinate_lr = (float)lr_in;
  const int threads = omp_get_max_threads();
  float* col_part = (float*)calloc((size_t)threads * (size_t)columns, sizeof(float));
  float* row_stats = (float*)malloc(sizeof(float) * (size_t)rows);
  float* col_stats = (float*)malloc(sizeof(float) * (size_t)columns);
  float* row_factor = (float*)malloc(sizeof(float) * (size_t)rows);
  float* col_factor = (float*)malloc(sizeof(float) * (size_t)columns);

  /* pass 1: row and column second moments, per-thread column strips */
#pragma omp parallel
  {
    float* local = col_part + (size_t)omp_get_thread_num() * (size_t)columns;
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const float* line = grad + r * columns;
      float total = 0.f;
      for (int64_t c = 0; c < columns; ++c) {
        const float sq = line[c] * line[c];
        total += sq;
        local[c] += sq;
      }
      const float upd =
          half_to_float(row_stat[r]) * beta2 + (total / (float)columns + 1e-12f) * (1.0f - beta2);
      row_stats[r] = upd;
      row_stat[r] = float_to_half(upd);
    }
  }
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < columns; ++c) {
    float total = 0.f;
    for (int t = 0; t < threads; ++t) total += col_part[(size_t)t * (size_t)columns + c];
    const float upd = half_to_float(col_stat[c]) * beta2 + (total / (float)rows + 1e-12f) * (1.0f - beta2);
    col_stats[c] = upd;
    col_stat[c] = float_to_half(upd);
  }
  double row_acc = 0.0;
  for (int64_t r = 0; r < rows; ++r) row_acc += row_stats[r];
  float row_mean = (float)(row_acc / (double)rows);
  if (row_mean < 1e-10f) row_mean = 1e-10f;
  const float sqrt_row_mean = sqrtf(row_mean);
  for (int64_t r = 0; r < rows; ++r) row_factor[r] = sqrt_row_mean / sqrtf(fmaxf(row_stats[r], 1e-10f));
  for (int64_t c = 0; c < columns; ++c) col_factor[c] = 1.0f / sqrtf(fmaxf(col_stats[c], 1e-10f));

  /* pass 2: normalize in place, global update RMS */
  double square_sum = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : square_sum)
  for (int64_t r = 0; r < rows; ++r) {
    float* line = grad + r * columns;
    const float m = row_factor[r];
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int64_t c = 0;
    for (; c + 4 <= columns; c += 4) {
      const float u0 = line[c] * m * col_factor[c], u1 = line[c + 1] * m * col_factor[c + 1];
      const float u2 = line[c + 2] * m * col_factor[c + 2], u3 = line[c + 3] * m * col_factor[c + 3];
      line[c] = u0;
      line[c + 1] = u1;
      line[c + 2] = u2;
      line[c + 3] = u3;
      a0 += u0 * u0;
      a1 += u1 * u1;
      a2 += u2 * u2;
      a3 += u3 * u3;
    }
    for (; c < columns; ++c) {
      const float u = line[c] * m * col_factor[c];
      line[c] = u;
      a0 += u * u;
    }
    square_sum += (double)(a0 + a1) + (double)(a2 + a3);
  }
  float mean_sq = (float)(square_sum / (double)count);
  const float update_rms = sqrtf(mean_sq > 1e-16f ? mean_sq : 1e-16f);
  const float divisor = fmaxf(1.0f, update_rms / update_clip);
  const float inverse_divisor = 1.0f / divisor;

  /* pass 3: block momentum, new fp16 block scale */
  double moment_sq = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : moment_sq)
  for (int64_t b = 0; b < blocks; ++b) {
    const int64_t start = b * block_size;
    const int64_t stop = start + block_size < count ? start + block_size : count;
    const float decay = half_to_float(moment_block[b]) * beta1;
    const float gain = (1.0f - beta1) * inverse_divisor;
    float maximum = 1e-6f, block_sq = 0.f;
    for (int64_t i = start; i < stop; ++i) {
      const float m = (float)moment_int[i] * decay + grad[i] * gain;
      grad[i] = m;
      block_sq += m * m;
      maximum = fmaxf(maximum, fabsf(m));
    }
    moment_sq += (double)block_sq;
    moment_block[b] = float_to_half(maximum / 127.0f);
  }
  float mmean = (float)(moment_sq / (double)(blocks * block_size));
  const float moment_rms = sqrtf(mmean > 1e-16f ? mmean : 1e-16f);
  const float coordinate_step = coordinate_lr / moment_rms;

  /* pass 4: stochastic rounding, requantization, repack, flips */
  const uint32_t hash_seed = scramble((uint32_t)seed) ^ scramble((uint32_t)step ^ 0x2545F491u);
  int64_t flips = 0;
#pragma omp parallel for schedule(static) reduction(+ : flips)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t base = r * columns;
    int64_t c = 0;
    while (c < columns) {
      const int64_t index = base + c;
      const int64_t block = index / block_size;
      const int64_t span = (block + 1) * block_size - index;
      const int64_t seg = columns < c + span ? columns : c + span;
      const float inv_scale = 1.0f / fmaxf(half_to_float(moment_block[block]), 1e-12f);
      for (int64_t k = c; k < seg; ++k) {
        const int64_t i = base + k;
        const float m = grad[i];
        const float target = (float)coord[i] - m * coordinate_step;
        const float lower = floorf(target);
        const float u = (float)scramble((uint32_t)i ^ hash_seed) * (1.0f / 4294967296.0f);
        const float rounded = lower + (u < (target - lower) ? 1.0f : 0.0f);
        coord[i] = (int8_t)fminf(127.0f, fmaxf(-127.0f, rounded));
        moment_int[i] = (int8_t)fminf(127.0f, fmaxf(-127.0f, rintf(m * inv_scale)));
      }
      c = seg;
    }
    const int8_t* line = coord + base;
    uint8_t* slot = bits + r * stride;
    for (int64_t b = 0; b < stride; ++b) {
      const int64_t c0 = b * 8;
      const int64_t limit = columns - c0 < 8 ? columns - c0 : 8;
      uint8_t next = 0;
      for (int64_t j = 0; j < limit; ++j)
        if (line[c0 + j] >= 0) next |= (uint8_t)(1u << j);
      const uint8_t mask = (uint8_t)(limit >= 8 ? 0xFF : ((1u << limit) - 1u));
      const uint8_t prev = slot[b];
      flips += __builtin_popcount((unsigned)((prev ^ next) & mask));
      slot[b] = (uint8_t)((prev & (uint8_t)~mask) | next);
    }
  }
  free(col_part);
  free(row_stats);
  free(col_stats);
  free(row_factor);
  free(col_factor);
  return flips;
}
