// Skinny-M forward (decode): y[m, n] = (sum_k x[m, k] sign[n, k]) * scale[n]
// + bias[n] for M <= 16 bf16 rows (fallback.py:95-108; the small-batch path of
// the reference GPU backend, cuda.py:198-501).
//
// The weight bits are the only large operand (R * C / 8 bytes), read once
// from HBM.  The rows of x (M <= 16) are padded to the 16 rows of
// v_mfma_f32_16x16x32_bf16 and staged through LDS in slices of 2048 columns;
// every x fragment feeds the MFMAs of two 16-row weight blocks, and each
// weight byte is expanded to eight bf16 signs in registers right before use.
//
// MFMA 16x16x32 bf16 layout used here: lane l holds A[l%16][8(l/16) + i] and
// B[8(l/16) + i][l%16]; accumulator register j holds D[4(l/16) + j][l%16].
// Within one MFMA the k-values of lane group q = l/16 are chosen freely (A and
// B agree): at k-step s of a 512-column chunk they are the 8 columns of byte
// 16q + s, so each lane streams 16 contiguous bytes of a weight row.
#include "common.hpp"

namespace qste {
namespace gemv {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int THREADS = 256;     // 4 waves
constexpr int SLICE = 2048;      // x columns per LDS slice
constexpr int CHUNK = 512;       // columns per 16-byte lane load (64 bytes of a weight row)
constexpr int DEPTH = SLICE / CHUNK;  // chunks in flight per row (the whole next slice)
constexpr int XLD = SLICE + 8;   // bf16 per LDS row of x (pad: conflict-free b128 reads)

__device__ __forceinline__ uint32_t pk_shl(uint32_t x, u16x2 sh) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, x) << sh);
}

__device__ __forceinline__ uint32_t bf16_one_pair() {
  uint32_t v;
  asm volatile("v_mov_b32 %0, 0x3F803F80" : "=v"(v));
  return v;
}

// 8 signs along k from one byte; `neg` has bit i set where k-offset i is -1.
__device__ __forceinline__ bf16x8 signs(uint32_t neg, uint32_t one) {
  const uint32_t tt = neg * 0x10001u;
  u32x4 r;
  r.x = (pk_shl(tt, u16x2{15, 14}) & 0x80008000u) | one;
  r.y = (pk_shl(tt, u16x2{13, 12}) & 0x80008000u) | one;
  r.z = (pk_shl(tt, u16x2{11, 10}) & 0x80008000u) | one;
  r.w = (pk_shl(tt, u16x2{9, 8}) & 0x80008000u) | one;
  return __builtin_bit_cast(bf16x8, r);
}

// NBW 16-row weight blocks per wave; a workgroup covers 4 * NBW * 16 rows.
template <int NBW>
__global__ __launch_bounds__(THREADS, 2) void decode_kernel(const uint16_t* __restrict__ x,
                                                            const uint8_t* __restrict__ bits,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ bias,
                                                            uint16_t* __restrict__ y, int M, int64_t N,
                                                            int64_t K) {
  constexpr int ROWS = 4 * NBW * 16;
  __shared__ __attribute__((aligned(16))) uint16_t xs[16 * XLD];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, q = lane >> 4;
  const int64_t pb = K / 8;
  const int64_t n_base = static_cast<int64_t>(blockIdx.x) * ROWS + wave * (NBW * 16);
  const uint32_t one = bf16_one_pair();

  f32x4 acc[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) acc[b] = f32x4{};

  // this lane's rows (clamped to the last row: out-of-range rows are computed
  // on valid memory and never stored)
  const uint8_t* rowp[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) {
    int64_t n = n_base + 16 * b + l16;
    if (n >= N) n = N - 1;
    rowp[b] = bits + n * pb + 16 * q;
  }
  const int64_t chunks = K / CHUNK;
  // ring of DEPTH chunks per row: buf[d] holds chunk (slice * DEPTH + d)
  uint4 buf[DEPTH][NBW];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d)
#pragma unroll
    for (int b = 0; b < NBW; ++b) buf[d][b] = *reinterpret_cast<const uint4*>(rowp[b] + d * 64);

  for (int64_t s0 = 0; s0 < K; s0 += SLICE) {
    // stage the M real rows of x[:, s0 : s0 + SLICE]; rows >= M are zero
    // registers in the loop below, not LDS
    __syncthreads();
    for (int e = tid; e < M * (SLICE / 8); e += THREADS) {
      const int m = e / (SLICE / 8), c8 = e % (SLICE / 8);
      *reinterpret_cast<uint4*>(&xs[m * XLD + 8 * c8]) =
          *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(m) * K + s0 + 8 * c8);
    }
    __syncthreads();
    const int64_t first = s0 / CHUNK;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      uint32_t w[NBW][4];
#pragma unroll
      for (int b = 0; b < NBW; ++b) {
        w[b][0] = ~buf[d][b].x; w[b][1] = ~buf[d][b].y; w[b][2] = ~buf[d][b].z; w[b][3] = ~buf[d][b].w;
      }
      // refill this ring slot with the same slot of the next slice
      if (first + d + DEPTH < chunks) {
#pragma unroll
        for (int b = 0; b < NBW; ++b)
          buf[d][b] = *reinterpret_cast<const uint4*>(rowp[b] + (first + d + DEPTH) * 64);
      }
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        // byte 16q + s of this lane's 64-byte row chunk = columns 8(16q + s) ..
        const int col = d * CHUNK + 8 * (16 * q + s);
        bf16x8 a = bf16x8{};
        if (l16 < M) a = *reinterpret_cast<const bf16x8*>(&xs[l16 * XLD + col]);
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
          const bf16x8 bv = signs((w[b][s >> 2] >> (8 * (s & 3))) & 0xFFu, one);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bv, acc[b], 0, 0, 0);
        }
      }
    }
  }

#pragma unroll
  for (int b = 0; b < NBW; ++b) {
    const int64_t n = n_base + 16 * b + l16;
    if (n >= N) continue;
    const float sc = scale[n];
    const float bi = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = 4 * q + j;
      if (m < M) {
        float v = acc[b][j] * sc;
        v = v + bi;
        y[static_cast<int64_t>(m) * N + n] = f32_to_bf16(v);
      }
    }
  }
}

}  // namespace gemv

// Returns 1 when the call is not for this path.
int gemv_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  if (dtype != QSTE_BF16 || m < 1 || m > 16 || rows < 1 || cols % gemv::SLICE != 0 ||
      (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(packed) & 15))
    return 1;
  // few rows of x: more, smaller workgroups for more weight bytes in flight;
  // up to 16 rows: two weight blocks per wave share each x fragment
  if (m <= 8) {
    const int grid = static_cast<int>((rows + 63) / 64);
    gemv::decode_kernel<1><<<grid, gemv::THREADS, 0, stream>>>(
        static_cast<const uint16_t*>(x), packed, scale, bias, static_cast<uint16_t*>(y), static_cast<int>(m),
        rows, cols);
  } else {
    const int grid = static_cast<int>((rows + 127) / 128);
    gemv::decode_kernel<2><<<grid, gemv::THREADS, 0, stream>>>(
        static_cast<const uint16_t*>(x), packed, scale, bias, static_cast<uint16_t*>(y), static_cast<int>(m),
        rows, cols);
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
