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

// bf16 pairs of the bases v0 = 4, 2, 1, 0.5 (bit 4, 5, 6, 7 clear)
constexpr uint32_t kBase[4] = {0x40804080u, 0x40004000u, 0x3F803F80u, 0x3F003F00u};

// Workgroup barrier that waits only for this wave's LDS operations.
// (__syncthreads() also waits for every outstanding global load, which here
// would make the prologue wait for the whole weight stream.)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
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
template <int NBW, int MP>
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

  uint32_t base[4];
  base[0] = vreg<kBase[0]>(); base[1] = vreg<kBase[1]>();
  base[2] = vreg<kBase[2]>(); base[3] = vreg<kBase[3]>();
  // B of the C/S product (the same for every MFMA): column 0 the bases,
  // column 1 ones, the rest zero
  const uint32_t cs_one = l16 == 1 ? 0x3F803F80u : 0u;
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
        const uint32_t wu = u == 0 ? w << 4 : w >> (4 * (u - 1));
        u32x4 bf;
        bf.x = (wu & 0x00100010u) | base[0];
        bf.y = (wu & 0x00200020u) | base[1];
        bf.z = (wu & 0x00400040u) | base[2];
        bf.w = (wu & 0x00800080u) | base[3];
        acc[b] = mma(af[4 * j + u], bf, acc[b]);
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
        for (int f = 0; f < 16; ++f) acc_cs = mma(af[f], cf, acc_cs);
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
          y[static_cast<int64_t>(m) * N + n] = f32_to_bf16(r);
        }
      }
    }
  }
}

template <int NBW, int MP>
void launch(const void* x, const uint8_t* packed, const float* scale, const float* bias, void* y, int64_t m,
            int64_t rows, int64_t cols, hipStream_t stream) {
  const int grid = static_cast<int>((rows + 16 * NBW - 1) / (16 * NBW));
  decode_kernel<NBW, MP><<<grid, THREADS, 0, stream>>>(static_cast<const uint16_t*>(x), packed, scale, bias,
                                                        static_cast<uint16_t*>(y), static_cast<int>(m), rows,
                                                        cols);
}

// ===========================================================================
// M <= 2 (the layout serves M <= 8): fp8 x fp4 MFMA
// (v_mfma_f32_16x16x128_f8f6f4, A fp8 e4m3, B fp4
// e2m1).  The weight bits become the fp4 B operand with four ANDs and one
// shift per 32 weights: e2m1 nibbles 0x1, 0x2, 0x4 are 0.5, 1 and 2, so for a
// weight dword w (32 columns from k0)
//     w & 0x11111111, w & 0x22222222, w & 0x44444444, (w >> 1) & 0x44444444
// are four B dwords whose nibble i of dword d is v_d * bit(4i + d),
// v = (0.5, 1, 2, 2): B slot 8d + i holds column k0 + 4i + d.  x enters as
// two exact fp8 limbs (hi = e4m3(x f), lo = e4m3(x f - hi), f = 2^-s(m) / v_d
// for the slot's class d and a row exponent s(m) that puts the row maximum
// in [64, 128)), hi in A rows 0..7 and lo in A rows 8..15 (rows that M <= 8
// leaves free), so one MFMA gives both halves:
//     sum_{k: bit} x[m, k] = 2^s(m) (D[m, n] + D[8 + m, n]),
//     y[m, n] = (2 sum_{bit} x - S[m]) scale[n] + bias[n],  S[m] = sum_k x[m, k].
// hi + lo holds the bf16 value exactly unless x f falls below e4m3's normal
// range (|x| < 2^-6 of the row maximum), where lo keeps as many bits as the
// e4m3 subnormals allow (absolute error <= 2^-10 / 64 of the row maximum).
// The MFMA itself sums each group of 128 products keeping about 16 bits below
// the group's largest term (measured on the device), which is far below the
// bf16 output's precision but above fp32's: about 0.5% of outputs round to
// the neighbouring bf16 value.
//
// The workgroup converts x once into LDS, already in MFMA fragment order
// (about 4.5 VALU ops per x element, against 5/32 per weight for the
// expansion, which is why this path stops at M = 8), then streams weights as
// the bf16 kernel does.
//
// Operand layouts of the 16x16x128 f8f6f4 MFMA (checked on the device): A
// (fp8) lane group g holds k = 16g + e in bytes e = 0..15 and k = 64 + 16g +
// e - 16 in bytes 16..31; B (fp4) lane group g holds k = 32g + e in nibble e
// (low nibble first); D as for every 16x16 MFMA.
// ===========================================================================
typedef int i32x8 __attribute__((ext_vector_type(8)));
constexpr int FP4_MAX_K = 8192;
constexpr int FRAG_BYTES = 8192;  // LDS bytes of x fragments per 512-column chunk

__device__ __forceinline__ f32x4 mma_f8f4(const i32x8& a, u32x4 b, f32x4 c) {
  const i32x8 bb = {static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w),
                    0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bb, c, 0, 4, 0, 0, 0, 0);
}

// one wave per SIMD: a second wave's first loads on a SIMD return only after
// the first wave's whole weight stream, which would hold x back
constexpr int F4_WAVES = 4;
constexpr int F4_THREADS = 64 * F4_WAVES;
constexpr int F4_CHUNKS = FP4_MAX_K / CHUNK_K / F4_WAVES;  // chunks per wave
constexpr int F4_DEPTH = 8;   // weight loads in flight per wave (swept: 8 beats 4-6 and 12-28)

template <int NBW>
struct SmemF4 {
  static constexpr int x_bytes = (FP4_MAX_K / CHUNK_K) * FRAG_BYTES;
  static constexpr int red_bytes = F4_WAVES * NBW * 64 * 16;
  static constexpr int bytes = x_bytes > red_bytes ? x_bytes : red_bytes;
};

template <int NBW>
__global__ __launch_bounds__(F4_THREADS, 1) void decode_fp4_kernel(const uint16_t* __restrict__ x,
                                                                const uint8_t* __restrict__ bits,
                                                                const float* __restrict__ scale,
                                                                const float* __restrict__ bias,
                                                                uint16_t* __restrict__ y, int M, int64_t N,
                                                                int64_t K) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[SmemF4<NBW>::bytes];
  __shared__ __attribute__((aligned(16))) float wave_max[8][4], wave_sum[8][4];
  __shared__ float row_sum[8], row_unscale[8];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // 4 waves, one per SIMD
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t pb = K / 8;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (16 * NBW);
  const int nchunks = static_cast<int>((K + CHUNK_K - 1) / CHUNK_K);
  const __amdgpu_buffer_rsrc_t rb = rsrc(bits, N * pb);
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, static_cast<int64_t>(M) * K * 2);
  uint32_t boff[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) boff[b] = static_cast<uint32_t>((n0 + 16 * b + l16) * pb + 16 * g);

  // the epilogue's row scale and bias (thread t < 32 NBW finishes column
  // n0 + 16 (t / 32) + t % 16)
  const int64_t n_out = n0 + 16 * (tid >> 5) + (tid & 15);
  float out_scale = 0.0f, out_bias = 0.0f;
  if (tid < 32 * NBW && n_out < N) {
    out_scale = scale[n_out];
    out_bias = bias ? bias[n_out] : 0.0f;
  }

  // ---- x: thread t loads and converts the units t and t + 256 (16 columns
  // each) of every row m < M
  constexpr int XT = F4_THREADS;
  const bool x_thread = true;
  u32x4 xv[8][2][2];  // [row][unit][half]
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (m < M && x_thread) {
#pragma unroll
      for (int uu = 0; uu < 2; ++uu) {
        const int unit = tid + XT * uu;
        const uint32_t off = 16 * unit < K ? static_cast<uint32_t>(m * K * 2 + 32 * unit) : kOob;
        xv[m][uu][0] = ld128(rx, off);
        xv[m][uu][1] = ld128(rx, off + 16);
      }
    }
  }

  // weight ring: this wave's chunks are wave + 4i (i = 0..3, all of K up to
  // 8192), 4 NBW blocks streamed with F4_DEPTH loads in flight
  constexpr int STEPS = F4_CHUNKS * NBW;
  constexpr int D = F4_DEPTH < STEPS ? F4_DEPTH : STEPS;
  u32x4 Bs[STEPS];
  auto issue_step = [&](int i) {
    const int c = wave + F4_WAVES * (i / NBW), b = i % NBW;
    Bs[i] = ld128(rb, c < nchunks ? boff[b] + 64u * static_cast<uint32_t>(c) : kOob);
  };
#pragma unroll
  for (int i = 0; i < D; ++i) issue_step(i);
  __builtin_amdgcn_sched_barrier(0);

  // row maxima (exact in any order) and row sums (fixed order: 16 values,
  // then a butterfly over the wave, then the waves in order)
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (m < M) {
      float mx = 0.0f, sm = 0.0f;
      if (x_thread) {
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t pr = xv[m][uu][h][e];
              const float lo = __uint_as_float(pr << 16), hi = __uint_as_float(pr & 0xFFFF0000u);
              mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
              sm += lo;
              sm += hi;
            }
          }
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, o));
        sm += __shfl_xor(sm, o);
      }
      if (lane == 0 && x_thread) {
        wave_max[m][wave] = mx;
        wave_sum[m][wave] = sm;
      }
    }
  }
  lds_barrier();
  // per row: f = 2^-s with the row maximum times f in [64, 128); thread m < M
  // also finishes the row's sum and 2^s for the epilogue
  float fbase[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (m < M) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&wave_max[m][0]);
      const float mx = fmaxf(fmaxf(a.x, a.y), fmaxf(a.z, a.w));
      const int e = static_cast<int>((__float_as_uint(mx) >> 23) & 0xFF);
      const int fe = e == 0 ? 127 : (260 - e > 254 ? 254 : 260 - e);
      fbase[m] = __uint_as_float(static_cast<uint32_t>(fe) << 23);
      if (tid == m) {
        float smv = wave_sum[m][0];
#pragma unroll
        for (int w = 1; w < 4; ++w) smv += wave_sum[m][w];
        row_sum[m] = smv;
        row_unscale[m] = __uint_as_float(static_cast<uint32_t>(254 - fe) << 23);  // 2^s
      }
    }
  }
  // convert and scatter: unit = (chunk c, q, t, i-half ih); the 4 values of
  // class d (columns d, d + 4, d + 8, d + 12 of the unit) are one dword of
  // fragment (c, t, g = 2(q % 2) + d / 2, h = q / 2), bytes 8(d % 2) + 4ih ..
#pragma unroll
  for (int uu = 0; uu < 2; ++uu) {
    const int unit = tid + XT * uu;
    if (x_thread && 16 * unit < nchunks * CHUNK_K) {
      const int c = unit >> 5, jj = unit & 31;
      const int q = jj >> 3, tw = (jj >> 1) & 3, ih = jj & 1;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        if (m >= M) break;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float f = fbase[m] * (d == 0 ? 2.0f : d == 1 ? 1.0f : 0.5f);
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int col = 4 * r + d;  // bf16 index within the unit's 16
            const uint32_t pr = xv[m][uu][col >> 3][(col >> 1) & 3];
            const float xf = (col & 1) ? __uint_as_float(pr & 0xFFFF0000u) : __uint_as_float(pr << 16);
            v[r] = xf * f;  // columns past K were loaded as zero
          }
          int hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
          hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], hi, true);
          const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
          const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
          int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0] - h01[0], v[1] - h01[1], 0, false);
          lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2] - h23[0], v[3] - h23[1], lo, true);
          const int gg = 2 * (q & 1) + (d >> 1), hh = q >> 1;
          uint8_t* frag = smem + c * FRAG_BYTES + ((tw * 4 + gg) * 2 + hh) * 256 + 8 * (d & 1) + 4 * ih;
          *reinterpret_cast<int*>(frag + 16 * m) = hi;
          *reinterpret_cast<int*>(frag + 16 * (8 + m)) = lo;
        }
      }
    }
  }
  lds_barrier();

  f32x4 acc[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) acc[b] = f32x4{};

  // this lane's A fragments of a chunk: window t, halves h = 0, 1
  i32x8 af[4];
  auto read_frags = [&](int c) {
    const uint8_t* src = smem + (c < nchunks ? c : 0) * FRAG_BYTES + g * 512 + 16 * l16;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 h0 = *reinterpret_cast<const u32x4*>(src + t * 2048);
      const u32x4 h1 = *reinterpret_cast<const u32x4*>(src + t * 2048 + 256);
      af[t] = i32x8{static_cast<int>(h0.x), static_cast<int>(h0.y), static_cast<int>(h0.z), static_cast<int>(h0.w),
                    static_cast<int>(h1.x), static_cast<int>(h1.y), static_cast<int>(h1.z), static_cast<int>(h1.w)};
    }
  };
  // The MFMA adds its C operand with the same reduced precision as its
  // products, so a long chain through C would align late products to an
  // ever larger partial sum: each block's 4 windows start from zero and the
  // block's sum joins the fp32 accumulator through ordinary adds.
  auto block = [&](const u32x4& Bd, int b) {
    f32x4 part = f32x4{};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t w = Bd[t];
      u32x4 bf;
      bf.x = w & 0x11111111u;
      bf.y = w & 0x22222222u;
      bf.z = w & 0x44444444u;
      bf.w = (w >> 1) & 0x44444444u;
      part = mma_f8f4(af[t], bf, part);
    }
    acc[b] += part;
  };

  // weight blocks in load order; a chunk past K reads zero weights and
  // contributes nothing
#pragma unroll
  for (int i = 0; i < STEPS; ++i) {
    if (i + D < STEPS) issue_step(i + D);
    if (i % NBW == 0) read_frags(wave + F4_WAVES * (i / NBW));
    __builtin_amdgcn_sched_barrier(0);
    block(Bs[i], i % NBW);
    __builtin_amdgcn_sched_barrier(0);
  }

  // partial sums of the 4 waves, added in wave order (every wave has read
  // its last fragments before the region is reused)
  lds_barrier();
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [WAVES][NBW][64]
#pragma unroll
  for (int b = 0; b < NBW; ++b) red[(wave * NBW + b) * 64 + lane] = acc[b];
  lds_barrier();
  if (tid < 32 * NBW) {
    // rows m = 4 (l / 16) + j (hi limbs) and 8 + m (lo limbs, 32 lanes on)
    const int b = tid >> 5, l = tid & 31;
    f32x4 part[2 * F4_WAVES];
#pragma unroll
    for (int w = 0; w < F4_WAVES; ++w) {
      part[2 * w] = red[(w * NBW + b) * 64 + l];
      part[2 * w + 1] = red[(w * NBW + b) * 64 + l + 32];
    }
    f32x4 v = part[0] + part[1];
#pragma unroll
    for (int w = 1; w < F4_WAVES; ++w) v += part[2 * w] + part[2 * w + 1];
    const int64_t n = n_out;
    if (n < N) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = 4 * (l >> 4) + j;
        if (m < M) {
          const float pos = v[j] * row_unscale[m];  // sum of x over set bits
          float r = 2.0f * pos - row_sum[m];
          r = r * out_scale;
          r = r + out_bias;
          y[static_cast<int64_t>(m) * N + n] = f32_to_bf16(r);
        }
      }
    }
  }
}

template <int NBW>
void launch_fp4(const void* x, const uint8_t* packed, const float* scale, const float* bias, void* y, int64_t m,
                int64_t rows, int64_t cols, hipStream_t stream) {
  const int grid = static_cast<int>((rows + 16 * NBW - 1) / (16 * NBW));
  decode_fp4_kernel<NBW><<<grid, F4_THREADS, 0, stream>>>(static_cast<const uint16_t*>(x), packed, scale, bias,
                                                       static_cast<uint16_t*>(y), static_cast<int>(m), rows, cols);
}

template <int NBW>
void launch_m(const void* x, const uint8_t* packed, const float* scale, const float* bias, void* y, int64_t m,
              int64_t rows, int64_t cols, hipStream_t stream) {
  if (m <= 1) launch<NBW, 1>(x, packed, scale, bias, y, m, rows, cols, stream);
  else if (m <= 2) launch<NBW, 2>(x, packed, scale, bias, y, m, rows, cols, stream);
  else if (m <= 4) launch<NBW, 4>(x, packed, scale, bias, y, m, rows, cols, stream);
  else if (m <= 8) launch<NBW, 8>(x, packed, scale, bias, y, m, rows, cols, stream);
  else launch<NBW, 16>(x, packed, scale, bias, y, m, rows, cols, stream);
}

}  // namespace gemv

// Returns 1 when the call is not for this path.
int gemv_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  if (dtype != QSTE_BF16 || m < 1 || m > 16 || rows < 1 || cols < 128 || cols % 128 != 0 ||
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
  // the fp8 x fp4 path converts x once per workgroup, a cost that grows with
  // m; it wins only for the smallest batches
  if (m <= 2 && cols <= gemv::FP4_MAX_K) {
    switch (nbw) {
      case 1: gemv::launch_fp4<1>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      case 2: gemv::launch_fp4<2>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      case 3: gemv::launch_fp4<3>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      case 4: gemv::launch_fp4<4>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      case 5: gemv::launch_fp4<5>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      case 6: gemv::launch_fp4<6>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      case 7: gemv::launch_fp4<7>(x, packed, scale, bias, y, m, rows, cols, stream); break;
      default: gemv::launch_fp4<8>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    }
    return static_cast<int>(hipGetLastError());
  }
  switch (nbw) {
    case 1: gemv::launch_m<1>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 2: gemv::launch_m<2>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 3: gemv::launch_m<3>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 4: gemv::launch_m<4>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 5: gemv::launch_m<5>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 6: gemv::launch_m<6>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    case 7: gemv::launch_m<7>(x, packed, scale, bias, y, m, rows, cols, stream); break;
    default: gemv::launch_m<8>(x, packed, scale, bias, y, m, rows, cols, stream); break;
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
