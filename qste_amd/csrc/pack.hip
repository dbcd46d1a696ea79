// Sign packing, expansion and the one-bit affine activation encoding.
//
// pack_coordinate  -- src/qste/kernels/fallback.py:91-92 (bits of coord >= 0)
// unpack_rows      -- fallback.py:27-29
// pack_affine_rows -- fallback.py:77-88, the encoding of functional.py:98-115
//
// All three are HBM-bound byte work: one thread owns one packed output byte,
// so no two threads ever write the same byte and no atomics are needed.
#include "common.hpp"
#include "encode.hpp"

namespace qste {

// Nonnegative-lane byte of eight int8 values held in a 64-bit word: the sign
// bit of each byte is moved to bit 0 of that byte, inverted, then the eight
// bits are gathered into the top byte by a multiply whose partial products
// land on distinct bit positions (so no carries can disturb the result).
__device__ __forceinline__ uint32_t nonneg_bits8(uint64_t w) {
  uint64_t neg = (w >> 7) & 0x0101010101010101ull;
  uint64_t pos = neg ^ 0x0101010101010101ull;
  return static_cast<uint32_t>((pos * 0x0102040810204080ull) >> 56);
}

__global__ void pack_coordinate_kernel(const int8_t* __restrict__ coord,
                                       uint8_t* __restrict__ packed, int64_t rows,
                                       int64_t cols, int64_t stride) {
  const int64_t total = rows * stride;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / stride;
    const int64_t b = idx - r * stride;
    const int64_t c0 = b * 8;
    const int8_t* src = coord + r * cols + c0;
    uint32_t byte;
    if ((cols & 7) == 0) {
      byte = nonneg_bits8(*reinterpret_cast<const uint64_t*>(src));
    } else {
      const int64_t n = cols - c0 < 8 ? cols - c0 : 8;
      byte = 0;
      for (int j = 0; j < n; ++j) byte |= (src[j] >= 0 ? 1u : 0u) << j;
    }
    packed[idx] = static_cast<uint8_t>(byte);
  }
}

template <int DT>
__global__ void unpack_rows_kernel(const uint8_t* __restrict__ packed,
                                   const float* __restrict__ row_scale,
                                   typename Elem<DT>::T* __restrict__ out, int64_t rows,
                                   int64_t cols, int64_t stride) {
  const int64_t total = rows * cols;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cols;
    const int64_t c = idx - r * cols;
    float v = sign_of(packed + r * stride, c);
    if (row_scale) v *= row_scale[r];
    Elem<DT>::store(out, idx, v);
  }
}

// One workgroup per row. Pass 1 sums the row in double (the correctly
// rounded fp32 sum in all but vanishingly rare cases, independent of the
// thread count); offset = fp32(sum) / fp32(cols), as ATen's mean is
// sum-then-divide. Pass 2 writes each byte from eight centered values and
// sums |x - offset| the same way.
template <int DT, int THREADS>
__global__ __launch_bounds__(THREADS) void pack_affine_rows_kernel(
    const typename Elem<DT>::T* __restrict__ x, uint8_t* __restrict__ packed,
    float* __restrict__ offset, float* __restrict__ scale, int64_t cols, int64_t stride) {
  __shared__ double red[THREADS / kWave];
  const int64_t row = blockIdx.x;
  const typename Elem<DT>::T* src = x + row * cols;
  uint8_t* dst = packed + row * stride;

  double sum = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += THREADS) sum += static_cast<double>(Elem<DT>::load(src, c));
  sum = block_sum(sum, red);
  const float n = static_cast<float>(cols);
  const float mean = static_cast<float>(sum) / n;

  double dev = 0.0;
  for (int64_t b = threadIdx.x; b < stride; b += THREADS) {
    const int64_t c0 = b * 8;
    const int64_t cnt = cols - c0 < 8 ? cols - c0 : 8;
    uint32_t byte = 0;
    for (int j = 0; j < cnt; ++j) {
      const float centered = Elem<DT>::load(src, c0 + j) - mean;
      dev += static_cast<double>(fabsf(centered));
      byte |= (centered >= 0.0f ? 1u : 0u) << j;
    }
    dst[b] = static_cast<uint8_t>(byte);
  }
  dev = block_sum(dev, red);
  if (threadIdx.x == 0) {
    offset[row] = mean;
    scale[row] = static_cast<float>(dev) / n;
  }
}

// Vectorized variant for bf16 rows whose width is a multiple of 8: each
// thread reads 16 bytes (8 values) per packed byte it owns.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void pack_affine_rows_bf16x8_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ packed, float* __restrict__ offset,
    float* __restrict__ scale, int64_t cols, int64_t stride) {
  __shared__ double red[THREADS / kWave];
  const int64_t row = blockIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(x + row * cols);
  uint8_t* dst = packed + row * stride;

  double sum = 0.0;
  for (int64_t b = threadIdx.x; b < stride; b += THREADS) {
    const uint4 v = src[b];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sum += static_cast<double>(__uint_as_float(w[i] << 16));
      sum += static_cast<double>(__uint_as_float(w[i] & 0xFFFF0000u));
    }
  }
  sum = block_sum(sum, red);
  const float n = static_cast<float>(cols);
  const float mean = static_cast<float>(sum) / n;

  double dev = 0.0;
  for (int64_t b = threadIdx.x; b < stride; b += THREADS) {
    const uint4 v = src[b];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t byte = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = __uint_as_float(w[i] << 16) - mean;
      const float hi = __uint_as_float(w[i] & 0xFFFF0000u) - mean;
      dev += static_cast<double>(fabsf(lo));
      dev += static_cast<double>(fabsf(hi));
      byte |= (lo >= 0.0f ? 1u : 0u) << (2 * i);
      byte |= (hi >= 0.0f ? 1u : 0u) << (2 * i + 1);
    }
    dst[b] = static_cast<uint8_t>(byte);
  }
  dev = block_sum(dev, red);
  if (threadIdx.x == 0) {
    offset[row] = mean;
    scale[row] = static_cast<float>(dev) / n;
  }
}

// Rows of bf16 whose 8-value chunks number at most CH * THREADS: a
// workgroup per row, each thread's chunks t, t + THREADS, ... held in
// registers from the first pass to the second (encode_row_chunks), so the
// row is read once.
template <int THREADS, int CH>
__global__ __launch_bounds__(THREADS) void pack_affine_rows_bf16_reg_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ packed, float* __restrict__ offset,
    float* __restrict__ scale, int64_t cols, int64_t stride) {
  __shared__ double red[THREADS / kWave];
  const int64_t row = blockIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(x + row * cols);
  const int t = threadIdx.x;
  uint4 v[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t q = t + static_cast<int64_t>(k) * THREADS;
    v[k] = q < stride ? src[q] : make_uint4(0, 0, 0, 0);
  }
  encode_row_chunks<THREADS, CH>(v, packed + row * stride, offset + row, scale + row, cols, stride, red);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static int grid_for(int64_t work, int threads) {
  int64_t blocks = (work + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return static_cast<int>(blocks);
}

// Bit transpose of a packed sign matrix: in [rows][in_pitch] bytes (bit j of
// byte b is column 8b + j) -> out [cols][out_pitch] bytes (bit i of byte b is
// row 8b + i); bits for rows >= rows are zero.  One thread per 8 x 8 block:
// eight row bytes become one 64-bit word (byte = row, bit = column) whose
// transpose (three delta swaps) gives one byte per column.
__device__ __forceinline__ uint64_t transpose_8x8(uint64_t x) {
  uint64_t t;
  t = (x ^ (x >> 7)) & 0x00AA00AA00AA00AAull;
  x = x ^ t ^ (t << 7);
  t = (x ^ (x >> 14)) & 0x0000CCCC0000CCCCull;
  x = x ^ t ^ (t << 14);
  t = (x ^ (x >> 28)) & 0x00000000F0F0F0F0ull;
  x = x ^ t ^ (t << 28);
  return x;
}

// A workgroup transposes 128-row x 512-column tiles through LDS (walking
// row tiles by gridDim.y): the input rows arrive as 16-byte loads, a thread
// transposes the 8 x 8 blocks of one column byte over a 64-row group (eight
// row blocks at a time, so each of its 8 columns gathers 64 rows into one
// 8-byte LDS word), and every output column leaves as 16 contiguous bytes
// (8-byte stores by consecutive lanes).  Tiles of 128 rows give a
// 3072 x 768 sign matrix 48 workgroups (12 with 512-row tiles: 6.0 instead
// of 11.8 us).  out_pitch must be a multiple of 8.
constexpr int kTrRows = 128, kTrColBytes = 64;  // tile: 128 rows x 512 columns
constexpr int kTrGroups = kTrRows / 64;          // 64-row groups per tile
constexpr int kTrPad = 4;                        // bytes of padding per staged input row
__global__ __launch_bounds__(256) void transpose_bits_kernel(const uint8_t* __restrict__ in,
                                                             uint8_t* __restrict__ out, int64_t rows,
                                                             int64_t cols, int64_t in_pitch,
                                                             int64_t out_pitch, int64_t row_tiles) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTrRows][kTrColBytes + kTrPad];
  __shared__ uint64_t otile[8 * kTrColBytes][kTrGroups];  // [column][64-row group]
  const int64_t cb0 = static_cast<int64_t>(blockIdx.x) * kTrColBytes;
  const int tid = threadIdx.x;
  const bool vec = (in_pitch & 15) == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  for (int64_t ty = blockIdx.y; ty < row_tiles; ty += gridDim.y) {
    const int64_t r0 = ty * kTrRows;
    // 128 rows x 64 bytes: load i of thread t is row (t >> 2) + 64 i, bytes
    // 16 (t & 3) .. + 15
#pragma unroll
    for (int i = 0; i < kTrGroups; ++i) {
      const int row = (tid >> 2) + 64 * i, part = tid & 3;
      const int64_t r = r0 + row;
      const int64_t cb = cb0 + 16 * part;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (r < rows) {
        if (vec && cb + 16 <= in_pitch) {
          const uint4 q = *reinterpret_cast<const uint4*>(in + r * in_pitch + cb);
          w[0] = q.x, w[1] = q.y, w[2] = q.z, w[3] = q.w;
        } else {
#pragma unroll
          for (int k = 0; k < 16; ++k)
            if (cb + k < in_pitch) w[k >> 2] |= static_cast<uint32_t>(in[r * in_pitch + cb + k]) << (8 * (k & 3));
        }
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) *reinterpret_cast<uint32_t*>(&tile[row][16 * part + 4 * d]) = w[d];
    }
    __syncthreads();
    if ((tid >> 6) < kTrGroups) {
      // column byte cbl of 64-row group g
      const int cbl = tid & 63, g = tid >> 6;
      uint64_t col[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int rb = 8 * g + b;  // row block: rows 8 rb .. 8 rb + 7
        uint64_t x = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) x |= static_cast<uint64_t>(tile[8 * rb + i][cbl]) << (8 * i);
        x = transpose_8x8(x);  // byte j: column 8 cbl + j over the block's 8 rows
#pragma unroll
        for (int j = 0; j < 8; ++j) col[j] |= ((x >> (8 * j)) & 0xFFull) << (8 * b);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) otile[8 * cbl + j][g] = col[j];
    }
    __syncthreads();
    // 512 columns x 16 bytes: store i of thread t is column t / 2 + 128 i,
    // bytes 8 (t % 2) .. + 7
#pragma unroll
    for (int i = 0; i < 2 * kTrGroups; ++i) {
      const int cl = tid / kTrGroups + (256 / kTrGroups) * i, piece = tid % kTrGroups;
      const int64_t c = 8 * cb0 + cl;
      const int64_t ob = r0 / 8 + 8 * piece;
      if (c < cols && ob < out_pitch) *reinterpret_cast<uint64_t*>(out + c * out_pitch + ob) = otile[cl][piece];
    }
    __syncthreads();  // the next row tile reuses tile and otile
  }
}

template <int DT>
__global__ void f32_to_16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out, int64_t n,
                                 int64_t padded) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < padded) out[i] = i < n ? (DT == QSTE_F16 ? f32_to_f16(in[i]) : f32_to_bf16(in[i])) : 0;
}

int launch_transpose_bits(const uint8_t* in, uint8_t* out, int64_t rows, int64_t cols, int64_t in_pitch,
                          int64_t out_pitch, hipStream_t stream) {
  if (rows == 0 || cols == 0 || out_pitch == 0) return 0;
  if (out_pitch % 8 != 0 || (reinterpret_cast<uintptr_t>(out) & 7)) return QSTE_E_ALIGN;
  // row tiles cover every output byte (out_pitch * 8 rows, the padding
  // included, which reads as zero); beyond the grid's 65535 rows of
  // workgroups each walks several tiles
  const int64_t row_tiles = (out_pitch * 8 + kTrRows - 1) / kTrRows;
  const dim3 grid(ceil_div(in_pitch, kTrColBytes), static_cast<unsigned>(row_tiles < 65535 ? row_tiles : 65535));
  transpose_bits_kernel<<<grid, 256, 0, stream>>>(in, out, rows, cols, in_pitch, out_pitch, row_tiles);
  return static_cast<int>(hipGetLastError());
}

// fp32 -> the 16-bit operand dtype (bf16 or fp16), zero-padded to `padded`
int launch_f32_to_16(const float* in, uint16_t* out, int64_t n, int64_t padded, int dtype, hipStream_t stream) {
  if (padded == 0) return 0;
  if (dtype == QSTE_F16)
    f32_to_16_kernel<QSTE_F16><<<ceil_div(padded, 256), 256, 0, stream>>>(in, out, n, padded);
  else
    f32_to_16_kernel<QSTE_BF16><<<ceil_div(padded, 256), 256, 0, stream>>>(in, out, n, padded);
  return static_cast<int>(hipGetLastError());
}

int launch_pack_coordinate(const int8_t* coord, uint8_t* packed, int64_t rows, int64_t cols,
                           hipStream_t stream) {
  const int64_t stride = (cols + 7) / 8;
  if (rows * stride == 0) return 0;
  pack_coordinate_kernel<<<grid_for(rows * stride, 256), 256, 0, stream>>>(coord, packed, rows,
                                                                            cols, stride);
  return static_cast<int>(hipGetLastError());
}

int launch_unpack_rows(const uint8_t* packed, const float* row_scale, void* out, int dtype,
                       int64_t rows, int64_t cols, hipStream_t stream) {
  const int64_t stride = (cols + 7) / 8;
  if (rows * cols == 0) return 0;
  const int grid = grid_for(rows * cols, 256);
  switch (dtype) {
    case QSTE_F32:
      unpack_rows_kernel<QSTE_F32><<<grid, 256, 0, stream>>>(packed, row_scale,
                                                             static_cast<float*>(out), rows, cols, stride);
      break;
    case QSTE_F16:
      unpack_rows_kernel<QSTE_F16><<<grid, 256, 0, stream>>>(packed, row_scale,
                                                             static_cast<uint16_t*>(out), rows, cols, stride);
      break;
    case QSTE_BF16:
      unpack_rows_kernel<QSTE_BF16><<<grid, 256, 0, stream>>>(packed, row_scale,
                                                              static_cast<uint16_t*>(out), rows, cols, stride);
      break;
    default:
      return QSTE_E_DTYPE;
  }
  return static_cast<int>(hipGetLastError());
}

int launch_pack_affine_rows(const void* x, int dtype, uint8_t* packed, float* offset, float* scale,
                            int64_t rows, int64_t cols, hipStream_t stream) {
  const int64_t stride = (cols + 7) / 8;
  if (rows == 0) return 0;
  constexpr int T = 256;
  const bool aligned16 = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  switch (dtype) {
    case QSTE_F32:
      pack_affine_rows_kernel<QSTE_F32, T><<<rows, T, 0, stream>>>(
          static_cast<const float*>(x), packed, offset, scale, cols, stride);
      break;
    case QSTE_F16:
      pack_affine_rows_kernel<QSTE_F16, T><<<rows, T, 0, stream>>>(
          static_cast<const uint16_t*>(x), packed, offset, scale, cols, stride);
      break;
    case QSTE_BF16:
      if ((cols & 7) == 0 && aligned16 && stride <= 2 * 256) {
        pack_affine_rows_bf16_reg_kernel<256, 2><<<rows, 256, 0, stream>>>(
            static_cast<const uint16_t*>(x), packed, offset, scale, cols, stride);
      } else if ((cols & 7) == 0 && aligned16 && stride <= 8 * 256) {
        pack_affine_rows_bf16_reg_kernel<256, 8><<<rows, 256, 0, stream>>>(
            static_cast<const uint16_t*>(x), packed, offset, scale, cols, stride);
      } else if ((cols & 7) == 0 && aligned16) {
        pack_affine_rows_bf16x8_kernel<T><<<rows, T, 0, stream>>>(
            static_cast<const uint16_t*>(x), packed, offset, scale, cols, stride);
      } else {
        pack_affine_rows_kernel<QSTE_BF16, T><<<rows, T, 0, stream>>>(
            static_cast<const uint16_t*>(x), packed, offset, scale, cols, stride);
      }
      break;
    default:
      return QSTE_E_DTYPE;
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
