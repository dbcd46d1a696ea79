// Row and column reductions of the backward pass.
//
//   row_inner   gs[r] = sum_c E[r, c] * sign[r, c]   (fallback.py:141-148)
//   colsums     v[r]  = sum_t dy[t, r] * offset[t]   (functional.py:139-144)
//               db[r] = sum_t dy[t, r]               (functional.py:193)
//
// Column sums run in two deterministic stages (chunk partials, then a fixed
// order sum) so results do not depend on scheduling; nothing uses atomics.
#include "common.hpp"

namespace qste {

constexpr int kRowThreads = 256;
constexpr int kColChunk = 256;

__global__ __launch_bounds__(kRowThreads) void row_inner_kernel(const float* __restrict__ mat,
                                                                const uint8_t* __restrict__ packed,
                                                                float* __restrict__ out,
                                                                int64_t cols, int64_t stride) {
  __shared__ float red[kRowThreads / kWave];
  const int64_t r = blockIdx.x;
  const float* row = mat + r * cols;
  const uint8_t* bits = packed + r * stride;
  float acc = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += kRowThreads) acc += row[c] * sign_of(bits, c);
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) out[r] = acc;
}

// Sum of `parts` partial vectors [parts][n] into out[n], in order of p (the
// loads are issued 32 at a time, so a few rounds of memory latency cover
// the usual 16-64 parts; the additions stay sequential).
__global__ void sum_partials_kernel(const float* __restrict__ partial, int64_t parts, int64_t n,
                                    float* __restrict__ out) {
  constexpr int kBatch = 32;
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  float s = 0.0f;
  int64_t p = 0;
  for (; p + kBatch <= parts; p += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) v[u] = partial[(p + u) * n + i];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) s += v[u];
  }
  for (; p + 8 <= parts; p += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = partial[(p + u) * n + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; p < parts; ++p) s += partial[p * n + i];
  out[i] = s;
}

template <int DT>
__global__ void colsum_partial_kernel(const typename Elem<DT>::T* __restrict__ dy,
                                      const float* __restrict__ offset, int64_t samples,
                                      int64_t rows, float* __restrict__ v_part,
                                      float* __restrict__ db_part) {
  const int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (r >= rows) return;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kColChunk;
  const int64_t t1 = t0 + kColChunk < samples ? t0 + kColChunk : samples;
  float v = 0.0f, db = 0.0f;
  for (int64_t t = t0; t < t1; ++t) {
    const float g = Elem<DT>::load(dy, t * rows + r);
    v = fmaf(g, offset[t], v);
    db += g;
  }
  v_part[blockIdx.y * rows + r] = v;
  if (db_part) db_part[blockIdx.y * rows + r] = db;
}

// rows a multiple of the 16-byte vector (8 bf16 / f16 or 4 fp32 columns):
// each lane reduces one vector of adjacent columns (one 16-byte load per
// sample), so a wave covers 512 (or 256) columns.  The chunk's
// kColChunk samples are split over the workgroup's kColWaves waves (a
// contiguous quarter each, UNROLL loads in flight), and the waves' sums are
// added in wave order through LDS: a fixed order, so the result does not
// depend on scheduling.  Four waves per chunk keep ~28 waves resident per CU
// at 16384 x 14336, where one wave per chunk left the loads latency-bound.
constexpr int kColWaves = 4;
constexpr int kColThreads = kColWaves * kWave;

template <int DT>
__global__ __launch_bounds__(kColThreads) void colsum_partial_x8_kernel(
    const typename Elem<DT>::T* __restrict__ dy, const float* __restrict__ offset, int64_t samples, int64_t rows,
    float* __restrict__ v_part, float* __restrict__ db_part) {
  using T = typename Elem<DT>::T;
  constexpr int NV = 16 / sizeof(T);  // columns per lane
  constexpr int UNROLL = 8;
  constexpr int kPad = 2 * NV + 1;  // 2 NV sums per lane, padded against bank conflicts
  __shared__ float red[kColWaves * kWave * kPad];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kWave * NV);
  const int64_t r = base + lane * NV;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kColChunk;
  const int64_t c1 = c0 + kColChunk < samples ? c0 + kColChunk : samples;
  constexpr int kPer = kColChunk / kColWaves;
  const int64_t t0 = c0 + wave * kPer < c1 ? c0 + wave * kPer : c1;
  const int64_t t1 = t0 + kPer < c1 ? t0 + kPer : c1;
  float v[NV], db[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = db[i] = 0.0f;
  if (r < rows) {
    const T* col = dy + r;
    int64_t t = t0;
    for (; t + UNROLL <= t1; t += UNROLL) {
      uint4 q[UNROLL];
      float o[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        q[u] = *reinterpret_cast<const uint4*>(col + (t + u) * rows);
        o[u] = offset[t + u];
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const T* e = reinterpret_cast<const T*>(&q[u]);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const float g = Elem<DT>::load(e, i);
          v[i] = fmaf(g, o[u], v[i]);
          db[i] += g;
        }
      }
    }
    for (; t < t1; ++t) {
      const uint4 q = *reinterpret_cast<const uint4*>(col + t * rows);
      const float o = offset[t];
      const T* e = reinterpret_cast<const T*>(&q);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const float g = Elem<DT>::load(e, i);
        v[i] = fmaf(g, o, v[i]);
        db[i] += g;
      }
    }
  }
  float* mine = red + (wave * kWave + lane) * kPad;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    mine[i] = v[i];
    mine[NV + i] = db[i];
  }
  __syncthreads();
  // 2 * 64 NV results per workgroup (its columns of v, then of db),
  // consecutive threads on consecutive columns; waves summed in order
  // 0..kColWaves-1.
  const int64_t part = static_cast<int64_t>(blockIdx.y) * rows;
#pragma unroll
  for (int j = threadIdx.x; j < 2 * kWave * NV; j += kColThreads) {
    const int which = j / (kWave * NV);
    const int c = j % (kWave * NV);
    const int64_t rc = base + c;
    const int slot = (c / NV) * kPad + which * NV + c % NV;
    float s = red[slot];
#pragma unroll
    for (int w = 1; w < kColWaves; ++w) s += red[w * kWave * kPad + slot];
    if (rc < rows) {
      if (which == 0) v_part[part + rc] = s;
      else if (db_part) db_part[part + rc] = s;
    }
  }
}

int launch_row_inner(const float* mat, const uint8_t* packed, float* out, int64_t rows,
                     int64_t cols, hipStream_t stream) {
  if (rows == 0) return 0;
  row_inner_kernel<<<rows, kRowThreads, 0, stream>>>(mat, packed, out, cols, (cols + 7) / 8);
  return static_cast<int>(hipGetLastError());
}

int launch_sum_partials(const float* partial, int64_t parts, int64_t n, float* out,
                        hipStream_t stream) {
  if (n == 0) return 0;
  // one wave per workgroup: a few thousand outputs still spread over most CUs
  sum_partials_kernel<<<ceil_div(n, kWave), kWave, 0, stream>>>(partial, parts, n, out);
  return static_cast<int>(hipGetLastError());
}

int colsum_chunks(int64_t samples) { return ceil_div(samples, kColChunk); }

// v_part / db_part: [colsum_chunks(samples)][rows] floats each.
int launch_colsums(const void* dy, int dtype, const float* offset, int64_t samples, int64_t rows,
                   float* v_part, float* db_part, float* v_out, float* db_out,
                   hipStream_t stream) {
  if (rows == 0) return 0;
  const int chunks = colsum_chunks(samples);
  const int nv = dtype == QSTE_F32 ? 4 : 8;  // columns per 16-byte vector
  const bool x8 = (dtype == QSTE_BF16 || dtype == QSTE_F16 || dtype == QSTE_F32) && rows % nv == 0 &&
                  (reinterpret_cast<uintptr_t>(dy) & 15) == 0;
  if (chunks > 0 && x8) {
    dim3 grid(ceil_div(rows, kWave * nv), chunks);
    if (dtype == QSTE_BF16)
      colsum_partial_x8_kernel<QSTE_BF16><<<grid, kColThreads, 0, stream>>>(
          static_cast<const uint16_t*>(dy), offset, samples, rows, v_part, db_part);
    else if (dtype == QSTE_F16)
      colsum_partial_x8_kernel<QSTE_F16><<<grid, kColThreads, 0, stream>>>(
          static_cast<const uint16_t*>(dy), offset, samples, rows, v_part, db_part);
    else
      colsum_partial_x8_kernel<QSTE_F32><<<grid, kColThreads, 0, stream>>>(
          static_cast<const float*>(dy), offset, samples, rows, v_part, db_part);
    int rc = static_cast<int>(hipGetLastError());
    if (rc) return rc;
  } else if (chunks > 0) {
    dim3 grid(ceil_div(rows, 256), chunks);
    switch (dtype) {
      case QSTE_F32:
        colsum_partial_kernel<QSTE_F32><<<grid, 256, 0, stream>>>(
            static_cast<const float*>(dy), offset, samples, rows, v_part, db_part);
        break;
      case QSTE_F16:
        colsum_partial_kernel<QSTE_F16><<<grid, 256, 0, stream>>>(
            static_cast<const uint16_t*>(dy), offset, samples, rows, v_part, db_part);
        break;
      case QSTE_BF16:
        colsum_partial_kernel<QSTE_BF16><<<grid, 256, 0, stream>>>(
            static_cast<const uint16_t*>(dy), offset, samples, rows, v_part, db_part);
        break;
      default:
        return QSTE_E_DTYPE;
    }
    int rc = static_cast<int>(hipGetLastError());
    if (rc) return rc;
  }
  int rc = launch_sum_partials(v_part, chunks, rows, v_out, stream);
  if (rc || !db_out) return rc;
  return launch_sum_partials(db_part, chunks, rows, db_out, stream);
}

}  // namespace qste
