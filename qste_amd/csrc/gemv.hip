// Skinny-M forward (decode): y[m, n] = (sum_k x[m, k] sign[n, k]) * scale[n]
// + bias[n] for M <= 16 bf16 rows (fallback.py:95-108; the small-batch path of
// the reference GPU backend, cuda.py:198-501).
//
// The weight bits (R * C / 8 bytes) are the only large operand and are read
// once from HBM, so the kernel has to stream them at memory speed.  Two costs
// stand in the way on CDNA4, and the design answers both:
//
// * Sign expansion.  Turning bits into +-1 bf16 costs at least two VALU ops per
//   element pair with a shift-and-mask scheme (about 6 us of VALU time at
//   M=1 for the config-5 matrix, more than the 3.7 us of HBM time).  Here a
//   bit becomes a bf16 of value v0 + 0.5 * bit with ONE v_and_or_b32 per
//   element pair: from one of four shifted copies of a weight dword (w << 4,
//   w, w >> 4, w >> 8), bit a in 4..7 of each 16-bit half is OR-ed into the
//   mantissa (a = 4..6) or the exponent LSB (a = 7) of the power-of-two base
//   v0 = 4, 2, 1, 0.5, whose bit a is clear; every set bit therefore adds
//   exactly 0.5.  With v0(k) = 4, 2, 1, 0.5 for k mod 4 = 0..3 the MFMA sums
//       acc[m, n] = sum_k x[m, k] v0(k) + 0.5 * sum_{k: bit} x[m, k]
//   and with C[m] = sum_k x[m, k] v0(k), S[m] = sum_k x[m, k]:
//       sum_k x[m, k] sign[n, k] = 2 * sum_{bit} x - S = 4 * acc - (4 C + S).
//   C and S come from one more MFMA per x fragment against the bases (column
//   0) and ones (column 1).  All values involved are exact in bf16; since
//   v0 <= 8 * 0.5, the cancellation costs about 3 of fp32's 24 bits.
// * Sharing x.  Each wave keeps its x fragments in registers and uses every
//   one for 7-8 weight blocks of 16 rows (not once per block from LDS).
//
// Work split: a workgroup of 8 waves owns 16 * NBW weight rows (NBW chosen so
// the grid is about one workgroup per CU); its waves split K in chunks of 512
// columns (lane group q of a wave reads 16 bytes = 128 columns of each row),
// all weight loads of a wave are issued before its first MFMA, and the 8
// partial accumulators are summed through LDS in a fixed order.  The x rows
// of a chunk reach the wave through its own LDS rows (direct buffer->LDS
// loads of one contiguous kilobyte per row) instead of per-lane 16-byte loads
// that touch 16 rows of x each.
//
// MFMA 16x16x32 bf16 layout: lane l holds A[l%16][8(l/16) + i] and
// B[8(l/16) + i][l%16]; accumulator register j holds D[4(l/16) + j][l%16].
// Which k each of a lane group's 8 slots stands for is free as long as A and
// B agree: for a weight dword w (32 columns from k0), MFMA u (0..3) takes the
// copy w_u = w << 4, w, w >> 4, w >> 8, and its slot pair a' (0..3) holds
// columns k0 + 4u + a' (low half, bit 4 + a' of w_u) and k0 + 16 + 4u + a'
// (high half, bit 20 + a' of w_u).
#include "common.hpp"

namespace qste {
namespace gemv {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVES = 8;
constexpr int THREADS = 64 * WAVES;
constexpr int CHUNK_K = 512;  // columns per wave chunk (4 lane groups x 128)
constexpr int DEPTH = 2;      // weight loads in flight per wave (swept 2-16: fewer requests per wave keep the
                              // CUs' streams interleaved; 2 is fastest at M = 4 and 16)
constexpr uint32_t kRsrcWord3 = 0x00020000u;
constexpr uint32_t kOob = 0x80000000u;  // an offset past every buffer: reads zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes > 0x7FFFFFFFll ? 0x7FFFFFFFu : static_cast<uint32_t>(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(n), kRsrcWord3);
}

__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}

// a literal held in a VGPR (VOP3 instructions take at most one SGPR and no
// literal on gfx9, so the base of each v_and_or_b32 lives in a VGPR)
template <uint32_t V>
__device__ __forceinline__ uint32_t vreg() {
  uint32_t v;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "i"(V));
  return v;
}

// Per activation dtype: the 16-bit pairs of the bases v0 = 4, 2, 1, 0.5,
// the position of slot a' = 0's bit in each half-word (bf16: bits 4..7,
// fp16: bits 7..10 -- the top three mantissa bits and the exponent LSB in
// both, which add exactly 0.5 to bases 4, 2, 1, 0.5, whose bit there is
// clear), the pair of ones, and the MFMA.
template <int DT>
struct Dec;

template <>
struct Dec<QSTE_BF16> {
  static constexpr uint32_t base[4] = {0x40804080u, 0x40004000u, 0x3F803F80u, 0x3F003F00u};
  static constexpr int pos = 4;
  static constexpr uint32_t ones = 0x3F803F80u;
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_bf16(v); }
};

template <>
struct Dec<QSTE_F16> {
  static constexpr uint32_t base[4] = {0x44004400u, 0x40004000u, 0x3C003C00u, 0x38003800u};
  static constexpr int pos = 7;
  static constexpr uint32_t ones = 0x3C003C00u;
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_f16(v); }
};

// Copy u (0..3) of a weight dword: the column 4u + a' (low half) and
// 16 + 4u + a' (high half) bits moved to position pos + a' of each half.
template <int POS>
__device__ __forceinline__ uint32_t weight_copy(uint32_t w, int u) {
  const int shift = POS - 4 * u;  // compile-time after unrolling
  return shift >= 0 ? w << shift : w >> -shift;
}

// Workgroup barrier that waits only for this wave's LDS operations.
// (__syncthreads() also waits for every outstanding global load, which here
// would make the prologue wait for the whole weight stream.)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}


typedef __attribute__((address_space(3))) void lds_t;
constexpr int XP = 1024 + 16;  // LDS bytes per staged x row: conflict-free 16-byte reads across 16 rows

template <int NBW, int MP>
struct Smem {
  static constexpr int x_bytes = WAVES * MP * XP;
  static constexpr int red_bytes = WAVES * (NBW + 1) * 64 * 16;
  static constexpr int bytes = x_bytes > red_bytes ? x_bytes : red_bytes;
};

// NBW weight blocks of 16 rows per workgroup; x rows staged MP (>= M, a
// power of two) at a time.
template <int DT, int NBW, int MP>
__global__ __launch_bounds__(THREADS, 1) void decode_kernel(const uint16_t* __restrict__ x,
                                                            const uint8_t* __restrict__ bits,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ bias,
                                                            uint16_t* __restrict__ y, int M, int64_t N,
                                                            int64_t K) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[Smem<NBW, MP>::bytes];
  __shared__ float dsum[16];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l16 = lane & 15, q = lane >> 4;
  const int64_t pb = K / 8;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * NBW);
  const int nchunks = static_cast<int>((K + CHUNK_K - 1) / CHUNK_K);

  // rows past N and x rows past M read zero through the buffer bounds
  const __amdgpu_buffer_rsrc_t rb = rsrc(bits, N * pb);
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, static_cast<int64_t>(M) * K * 2);
  uint32_t boff[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) boff[b] = static_cast<uint32_t>((n0 + 16 * b + l16) * pb + 16 * q);

  using T = Dec<DT>;
  uint32_t base[4];
  base[0] = vreg<T::base[0]>(); base[1] = vreg<T::base[1]>();
  base[2] = vreg<T::base[2]>(); base[3] = vreg<T::base[3]>();
  // B of the C/S product (the same for every MFMA): column 0 the bases,
  // column 1 ones, the rest zero
  const uint32_t cs_one = l16 == 1 ? T::ones : 0u;
  u32x4 cf;
  cf.x = l16 == 0 ? base[0] : cs_one;
  cf.y = l16 == 0 ? base[1] : cs_one;
  cf.z = l16 == 0 ? base[2] : cs_one;
  cf.w = l16 == 0 ? base[3] : cs_one;

  f32x4 acc[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) acc[b] = f32x4{};
  f32x4 acc_cs = f32x4{};

  // the epilogue's row scale and bias, fetched now so their latency is not
  // paid after the reduction (thread t finishes column n0 + 16 (t / 64) + t % 16)
  const int64_t n_out = n0 + 16 * (tid >> 6) + (tid & 15);
  float out_scale = 0.0f, out_bias = 0.0f;
  if (tid < 64 * NBW && n_out < N) {
    out_scale = scale[n_out];
    out_bias = bias ? bias[n_out] : 0.0f;
  }

  // x rows of a chunk go to this wave's own LDS rows with one direct
  // buffer->LDS load per row (1 KB, lane-contiguous, so every instruction
  // reads one contiguous kilobyte); no other wave touches them, so no
  // workgroup barrier is needed
  uint8_t* xr = smem + wave * MP * XP;
  auto issue_x = [&](int c) {
    // lane l brings columns 512c + 8l .. + 7; columns past K (a last chunk
    // that K ends inside) and rows past M read zero
    const bool live = c < nchunks && CHUNK_K * c + 8 * lane < K;
    const uint32_t off = static_cast<uint32_t>(c) * 1024u + 16u * lane;
#pragma unroll
    for (int m = 0; m < MP; ++m)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_t*)(xr + m * XP), 16,
                                               live ? off + static_cast<uint32_t>(m * K * 2) : kOob, 0, 0, 0);
  };
  // this lane's 128 columns of its x row.  Lanes of rows past MP read row
  // l16 % MP instead: output rows m >= M are never stored, and an MFMA output
  // row depends only on the same row of A, so those rows may hold any finite
  // values (and identical addresses are broadcast by the LDS)
  auto read_x = [&](u32x4 (&Xd)[16]) {
    const uint8_t* src = xr + (l16 & (MP - 1)) * XP + 256 * q;
#pragma unroll
    for (int i = 0; i < 16; ++i) Xd[i] = *reinterpret_cast<const u32x4*>(src + 16 * i);
    // the next chunk's direct loads overwrite these rows: the values must
    // live in registers from here on, not be re-read from LDS later
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(Xd[i]));
  };
  // The 16 x fragments of a chunk (one per 32-column group j and MFMA u;
  // slot pair a' holds columns 4u + a' and 16 + 4u + a' of the group),
  // permuted once and used for every weight block of the chunk.
  auto fragments = [&](const u32x4 (&Xd)[16], u32x4 (&af)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t xg[16];  // columns k0 + 2i, k0 + 2i + 1 of group j
#pragma unroll
      for (int i = 0; i < 16; ++i) xg[i] = Xd[4 * j + i / 4][i % 4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        af[4 * j + u].x = __builtin_amdgcn_perm(xg[8 + 2 * u], xg[2 * u], 0x05040100u);
        af[4 * j + u].y = __builtin_amdgcn_perm(xg[8 + 2 * u], xg[2 * u], 0x07060302u);
        af[4 * j + u].z = __builtin_amdgcn_perm(xg[9 + 2 * u], xg[2 * u + 1], 0x05040100u);
        af[4 * j + u].w = __builtin_amdgcn_perm(xg[9 + 2 * u], xg[2 * u + 1], 0x07060302u);
      }
    }
  };
  auto block = [&](const u32x4 (&af)[16], const u32x4& Bd, int b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = Bd[j];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t wu = weight_copy<T::pos>(w, u);
        constexpr uint32_t m0 = 0x00010001u << T::pos;
        u32x4 bf;
        bf.x = (wu & m0) | base[0];
        bf.y = (wu & (m0 << 1)) | base[1];
        bf.z = (wu & (m0 << 2)) | base[2];
        bf.w = (wu & (m0 << 3)) | base[3];
        acc[b] = T::mma(af[4 * j + u], bf, acc[b]);
      }
    }
  };

  // Chunks wave and wave + 8 (all of K up to 8192; larger K loops), their
  // 2 * NBW weight blocks streamed through a ring of DEPTH loads in flight:
  // the load of block i + DEPTH is issued when block i is consumed.  (All
  // loads at once would make every block complete only at the end of the
  // whole transfer, leaving no compute to overlap with it.)
  constexpr int STEPS = 2 * NBW;
  constexpr int D = DEPTH < STEPS ? DEPTH : STEPS;
  for (int c0 = wave; c0 < nchunks; c0 += 2 * WAVES) {
    const int c1 = c0 + WAVES;
    u32x4 X[16], af[16], Bs[STEPS];
    auto issue_step = [&](int i) {
      const int c = i < NBW ? c0 : c1, b = i < NBW ? i : i - NBW;
      Bs[i] = ld128(rb, c < nchunks ? boff[b] + 64u * static_cast<uint32_t>(c) : kOob);
    };
    issue_x(c0);
#pragma unroll
    for (int i = 0; i < D; ++i) issue_step(i);
    __builtin_amdgcn_sched_barrier(0);
    read_x(X);
    // the x rows are read before the next chunk's rows overwrite them
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    issue_x(c1);
    __builtin_amdgcn_sched_barrier(0);
    fragments(X, af);
#pragma unroll
    for (int i = 0; i < STEPS; ++i) {
      if (i + D < STEPS) issue_step(i + D);
      if (i == NBW) {
        read_x(X);
        fragments(X, af);
      }
      __builtin_amdgcn_sched_barrier(0);
      block(af, Bs[i], i < NBW ? i : i - NBW);
      if (i == NBW - 1 || i == STEPS - 1) {
#pragma unroll
        for (int f = 0; f < 16; ++f) acc_cs = T::mma(af[f], cf, acc_cs);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }

  // partial sums of the 8 waves, added in wave order
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [WAVES][NBW + 1][64]
#pragma unroll
  for (int b = 0; b < NBW; ++b) red[(wave * (NBW + 1) + b) * 64 + lane] = acc[b];
  red[(wave * (NBW + 1) + NBW) * 64 + lane] = acc_cs;
  __syncthreads();
  if (tid < 16) {
    // row m = tid: C at (lane 16(m/4), reg m%4), S at the next lane
    const int src = 16 * (tid >> 2), j = tid & 3;
    float c = 0.0f, s = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      c += red[(w * (NBW + 1) + NBW) * 64 + src][j];
      s += red[(w * (NBW + 1) + NBW) * 64 + src + 1][j];
    }
    dsum[tid] = 4.0f * c + s;
  }
  __syncthreads();
  if (tid < 64 * NBW) {
    const int b = tid >> 6, l = tid & 63;
    f32x4 v = red[b * 64 + l];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[(w * (NBW + 1) + b) * 64 + l];
    const int64_t n = n_out;
    if (n < N) {
      const float sc = out_scale;
      const float bi = out_bias;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = 4 * (l >> 4) + j;
        if (m < M) {
          float r = 4.0f * v[j] - dsum[m];
          r = r * sc;
          r = r + bi;
          y[static_cast<int64_t>(m) * N + n] = T::store(r);
        }
      }
    }
  }
}

template <int DT, int NBW, int MP>
void launch(const void* x, const uint8_t* packed, const float* scale, const float* bias, void* y, int64_t m,
            int64_t rows, int64_t cols, hipStream_t stream) {
  const int grid = static_cast<int>((rows + 16 * NBW - 1) / (16 * NBW));
  decode_kernel<DT, NBW, MP><<<grid, THREADS, 0, stream>>>(static_cast<const uint16_t*>(x), packed, scale, bias,
                                                        static_cast<uint16_t*>(y), static_cast<int>(m), rows,
                                                        cols);
}

template <int DT, int NBW>
void launch_m(const void* x, const uint8_t* packed, const float* scale, const float* bias, void* y, int64_t m,
              int64_t rows, int64_t cols, hipStream_t stream) {
  if (m <= 1) launch<DT, NBW, 1>(x, packed, scale, bias, y, m, rows, cols, stream);
  else if (m <= 2) launch<DT, NBW, 2>(x, packed, scale, bias, y, m, rows, cols, stream);
  else if (m <= 4) launch<DT, NBW, 4>(x, packed, scale, bias, y, m, rows, cols, stream);
  else if (m <= 8) launch<DT, NBW, 8>(x, packed, scale, bias, y, m, rows, cols, stream);
  else launch<DT, NBW, 16>(x, packed, scale, bias, y, m, rows, cols, stream);
}

template <int DT>
void launch_dt(int64_t nbw, const void* x, const uint8_t* packed, const float* scale, const float* bias, void* y,
               int64_t m, int64_t rows, int64_t cols, hipStream_t stream) {
  switch (nbw) {
    case 1: launch_m<DT, 1>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 2: launch_m<DT, 2>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 3: launch_m<DT, 3>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 4: launch_m<DT, 4>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 5: launch_m<DT, 5>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 6: launch_m<DT, 6>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 7: launch_m<DT, 7>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    default: launch_m<DT, 8>(x, packed, scale, bias, y, m, rows, cols, stream); break;
  }
}

}  // namespace gemv

// Returns 1 when the call is not for this path.
int gemv_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  if ((dtype != QSTE_BF16 && dtype != QSTE_F16) || m < 1 || m > 16 || rows < 1 || cols < 128 || cols % 128 != 0 ||
      (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(packed) & 15))
    return 1;
  // 32-bit buffer offsets, with room for the padded last block and the
  // out-of-range marker
  const int64_t pb = cols / 8;
  if ((rows + 128) * pb >= (int64_t{1} << 31) || m * cols * 2 >= (int64_t{1} << 31)) return 1;
  // about one workgroup per CU: 16 * NBW rows each, NBW in 1..8
  int64_t nbw = (rows + 16 * 256 - 1) / (16 * 256);
  if (nbw < 1) nbw = 1;
  if (nbw > 8) nbw = 8;
  if (dtype == QSTE_F16)
    gemv::launch_dt<QSTE_F16>(nbw, x, packed, scale, bias, y, m, rows, cols, stream);
  else
    gemv::launch_dt<QSTE_BF16>(nbw, x, packed, scale, bias, y, m, rows, cols, stream);
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
