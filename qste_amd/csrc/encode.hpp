// The one-bit affine encoding of a bf16 row held in registers
// (src/qste/kernels/fallback.py:77-88, encode_activation of
// src/qste/functional.py:98-115): offset = mean, bit = (x - offset >= 0),
// scale = mean |x - offset|.  Shared by pack_affine_rows and by the fused
// SwiGLU forward, which encodes the rows it produces, so both give the same
// bytes for the same row.
#pragma once

#include "common.hpp"

namespace qste {

// bf16 value i (0..7) of an 8-value chunk
__device__ __forceinline__ float chunk_value(const uint4& c, int i) {
  const uint32_t w = i < 2 ? c.x : i < 4 ? c.y : i < 6 ? c.z : c.w;
  return (i & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
}

// One row of `stride` 8-value chunks, chunk t + k * THREADS of it in v[k] of
// thread t (zero past the row), a workgroup of THREADS per row.  Sums of
// eight values are pairwise in double, then per thread in k order, then
// across the workgroup in a fixed order: sums of bf16 values this long are
// exact in double, and the deviation sum rounds once, so the result does not
// depend on the thread count.
template <int THREADS, int CH>
__device__ __forceinline__ void encode_row_chunks(const uint4 (&v)[CH], uint8_t* __restrict__ dst,
                                                  float* __restrict__ offset, float* __restrict__ scale,
                                                  int64_t cols, int64_t stride, double* red) {
  const int t = threadIdx.x;
  double sum = 0.0;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    double d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = static_cast<double>(chunk_value(v[k], i));
    sum += ((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7]));
  }
  sum = block_sum(sum, red);
  const float n = static_cast<float>(cols);
  const float mean = static_cast<float>(sum) / n;
  double dev = 0.0;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t q = t + static_cast<int64_t>(k) * THREADS;
    uint32_t byte = 0;
    double d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float c = chunk_value(v[k], i) - mean;
      byte |= (c >= 0.0f ? 1u : 0u) << i;
      d[i] = static_cast<double>(fabsf(c));
    }
    if (q < stride) {
      dst[q] = static_cast<uint8_t>(byte);
      dev += ((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7]));
    }
  }
  dev = block_sum(dev, red);
  if (t == 0) {
    *offset = mean;
    *scale = static_cast<float>(dev) / n;
  }
}

}  // namespace qste
