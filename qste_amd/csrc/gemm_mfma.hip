// bf16 MFMA products over packed signs for gfx950 (CDNA4).
//
// All three products of a binary linear layer are GEMMs whose one operand
// is a matrix of +-1 (times a per-k scale in the backward ones) held as
// bits.  The bits are expanded to bf16 in registers right before
// v_mfma_f32_32x32x16_bf16 consumes them, so the expanded operand never
// exists in HBM or LDS; global traffic for it is 1/16 of a bf16 operand.
//
//   forward   y  = x  [M=T, K=C] . sign_w^T          -> * scale[n] + bias[n]
//             bits run along K (row n of W): a lane's 8 k-values are one byte
//   dgrad     dx = dy [M=T, K=R] . (s (*) sign_w)    bits run along N
//   evidence  E  = dy^T [M=R, K=T] . (xs (*) sign_x) bits run along N,
//             dy^T is transposed in registers on its way into LDS; fused
//             epilogue + v[m], row partials of E0 . sign_w, * scale[m]
//
// Tile: 256 x 128 per workgroup of 4 waves (2 x 2), each wave 128 x 64 as
// 4 x 2 blocks of 32 x 32, K step 64 (4 MFMA k-steps of 16).  The dense
// operand (A) goes through double-buffered LDS with one barrier per K step;
// the next step's global loads (buffer loads, whose out-of-range reads
// return zero and so pad ragged edges for free) are issued before the
// current step's MFMAs.  Where bits run along N they are staged through LDS
// as a small transposed byte tile, inverted so a set bit means "negative".
//
// MFMA 32x32x16 bf16 operand layout used here: lane l holds A[l%32][8(l/32)
// + i] and B[8(l/32) + i][l%32], i = 0..7; the accumulator's register r
// holds D[8(r/4) + 4(l/32) + r%4][l%32].
#include "common.hpp"

namespace qste {
namespace mfma {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 128, BK = 64, THREADS = 256;
constexpr int LDA = BK + 8;                 // bf16 per LDS row of A (144 B)
constexpr int LDB = BK + 8;                 // bytes per LDS row of staged bits ([n/8][k])
constexpr int A_TILE = BM * LDA;            // bf16 elements per A buffer
constexpr int B_TILE = (BN / 8) * LDB;      // bytes per staged-bits buffer
constexpr uint32_t kRsrcWord3 = 0x00020000u;

enum { A_ROWS_M = 0, A_ROWS_K = 1 };        // A[m][k] stored with k (or m) contiguous
enum { B_BITS_ALONG_K = 0, B_BITS_ALONG_N = 1 };
enum { EPI_FORWARD = 0, EPI_PLAIN = 1, EPI_EVIDENCE = 2 };

struct Params {
  const uint16_t* a;     // bf16 dense operand (x or dy)
  const uint8_t* bits;   // packed signs of the +-1 operand
  const float* kscale;   // per-k scale folded into the bit operand (dgrad/evidence)
  void* out;
  int64_t M, N, K;
  int64_t lda;           // elements between rows of the dense source
  int64_t pb;            // bytes per packed row
  int64_t a_rows;        // rows of the dense source (bounds of its buffer)
  int64_t bit_rows;      // rows of the packed source
  // epilogue
  const float* n_scale;  // forward
  const float* n_bias;   // forward
  const float* m_add;    // evidence
  const float* m_scale;  // evidence
  const uint8_t* w_bits; // evidence: sign_w for the scale gradient
  float* gs_partial;     // evidence: [2 * tiles_n][M]
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFll ? 0xFFFFFFFFu : static_cast<uint32_t>(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(n), kRsrcWord3);
}

__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}
__device__ __forceinline__ uint64_t ld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0));
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ uint32_t pk_shl(uint32_t x, u16x2 sh) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, x) << sh);
}

// 0x3F803F80 (a pair of bf16 +1.0) held in a VGPR so the sign insertion below
// is one v_and_or_b32 per pair.
__device__ __forceinline__ uint32_t bf16_one_pair() {
  uint32_t v;
  asm volatile("v_mov_b32 %0, 0x3F803F80" : "=v"(v));
  return v;
}

// 8 signs along k from one byte; `neg` has bit i set where k-offset i is -1.
__device__ __forceinline__ bf16x8 signs_along_k(uint32_t neg, uint32_t one) {
  const uint32_t tt = neg * 0x10001u;
  u32x4 r;
  r.x = (pk_shl(tt, u16x2{15, 14}) & 0x80008000u) | one;
  r.y = (pk_shl(tt, u16x2{13, 12}) & 0x80008000u) | one;
  r.z = (pk_shl(tt, u16x2{11, 10}) & 0x80008000u) | one;
  r.w = (pk_shl(tt, u16x2{9, 8}) & 0x80008000u) | one;
  return __builtin_bit_cast(bf16x8, r);
}

// 8 scaled signs across k: byte i of `neg8` is the (inverted) bit row for
// k-offset i; this lane's column is bit `bit` of each byte.  `scale` holds
// the 8 nonnegative bf16 scales as pairs; a set bit sets the sign.
__device__ __forceinline__ bf16x8 signs_across_k(uint64_t neg8, int bit, uint4 scale) {
  const uint64_t x = neg8 >> bit;
  const uint32_t lo = static_cast<uint32_t>(x), hi = static_cast<uint32_t>(x >> 32);
  u32x4 r;
  r.x = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C010C00u), u16x2{15, 15}) | scale.x;
  r.y = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C030C02u), u16x2{15, 15}) | scale.y;
  r.z = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C050C04u), u16x2{15, 15}) | scale.z;
  r.w = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C070C06u), u16x2{15, 15}) | scale.w;
  return __builtin_bit_cast(bf16x8, r);
}

// Workgroup barrier for LDS hand-off only.  __syncthreads() carries a
// workgroup memory fence, which makes the compiler wait for every
// outstanding global load (vmcnt(0)) at each barrier and so cancels the
// prefetch; here only this wave's LDS operations are drained (lgkmcnt(0))
// before the barrier, and in-flight global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt: no wait, expcnt: no wait, lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Workgroup -> output tile.  Consecutive workgroup ids land on different
// XCDs (round-robin), so ids are first regrouped so each XCD gets a
// contiguous range, then walked in column-major groups of 2 M-tiles, so the
// workgroups that run together on one XCD share two dense-operand row blocks
// (the large operand) and many small bit tiles in that XCD's L2.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
  constexpr int G = 2;
  const int per_group = G * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * G;
  const int gm = min(tiles_m - first_m, G);
  const int in_group = pid % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// Index of this 16-byte chunk of a transposed (A_ROWS_K) A row in LDS: XOR
// swizzled by (row / 8) so the transposed stores do not collide on banks.
__device__ __forceinline__ int a_chunk(int akind, int chunk, int row) {
  return akind == A_ROWS_K ? (chunk ^ ((row >> 3) & 7)) : chunk;
}

template <int AKIND, int BKIND, int EPI>
__global__ __launch_bounds__(THREADS, 2) void gemm_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2 * A_TILE];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[BKIND == B_BITS_ALONG_N ? 2 * B_TILE : 16];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[BKIND == B_BITS_ALONG_N ? 2 * BK : 8];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, kg = lane >> 5;
  const int tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  const int tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint32_t one = bf16_one_pair();
  const int nk = static_cast<int>((p.K + BK - 1) / BK);

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  // ---- A source --------------------------------------------------------
  // A_ROWS_M: thread loads rows (arow + 32 i), 16-byte chunk achunk.
  // A_ROWS_K: thread loads an 8 x 8 block: k rows 8kb..8kb+7, m cols 8rb..
  const int arow = tid >> 3, achunk = tid & 7;
  const int rb = tid & 31, kb = tid >> 5;
  __amdgpu_buffer_rsrc_t ra;
  uint32_t aoff;
  if (AKIND == A_ROWS_M) {
    // buffer starts at the tile's first row: rows past M read as zero
    const int64_t rows_left = p.a_rows - m0;
    ra = rsrc(p.a + m0 * p.lda, rows_left * p.lda * 2);
    aoff = static_cast<uint32_t>((arow * p.lda + achunk * 8) * 2);
  } else {
    // buffer starts at column m0: k rows past K read as zero
    ra = rsrc(p.a + m0, (p.a_rows * p.lda - m0) * 2);
    aoff = static_cast<uint32_t>(((8 * kb) * p.lda + 8 * rb) * 2);
  }
  const uint32_t a_step = AKIND == A_ROWS_M ? BK * 2 : static_cast<uint32_t>(BK * p.lda * 2);
  const uint32_t a_stride = AKIND == A_ROWS_M ? static_cast<uint32_t>(32 * p.lda * 2)
                                              : static_cast<uint32_t>(p.lda * 2);
  uint4 areg[8];
  auto load_a = [&](int it) {
    const uint32_t base = aoff + static_cast<uint32_t>(it) * a_step;
#pragma unroll
    for (int i = 0; i < 8; ++i) areg[i] = ld128(ra, base + i * a_stride);
  };
  auto store_a = [&](uint16_t* buf) {
    if (AKIND == A_ROWS_M) {
#pragma unroll
      for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(&buf[(arow + 32 * i) * LDA + achunk * 8]) = areg[i];
    } else {
      const uint32_t* in = reinterpret_cast<const uint32_t*>(areg);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        uint4 o;
        o.x = __builtin_amdgcn_perm(in[4 + (j >> 1)], in[0 + (j >> 1)], sel);
        o.y = __builtin_amdgcn_perm(in[12 + (j >> 1)], in[8 + (j >> 1)], sel);
        o.z = __builtin_amdgcn_perm(in[20 + (j >> 1)], in[16 + (j >> 1)], sel);
        o.w = __builtin_amdgcn_perm(in[28 + (j >> 1)], in[24 + (j >> 1)], sel);
        const int row = 8 * rb + j;
        *reinterpret_cast<uint4*>(&buf[row * LDA + a_chunk(A_ROWS_K, kb, row) * 8]) = o;
      }
    }
  };

  // ---- B source ----------------------------------------------------------
  __amdgpu_buffer_rsrc_t rb_bits = rsrc(p.bits, p.bit_rows * p.pb);
  __amdgpu_buffer_rsrc_t rb_scale = rsrc(p.kscale, p.kscale ? p.K * 4 : 0);
  uint64_t breg[2] = {0, 0};   // B_BITS_ALONG_K: this lane's 64 k-bits of its two columns
  uint32_t bword = 0;          // B_BITS_ALONG_N: one staged dword of bits
  float bscale = 0.0f;
  uint32_t boff[2];
  if (BKIND == B_BITS_ALONG_K) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t n = n0 + 64 * wn + 32 * nb + l32;
      boff[nb] = static_cast<uint32_t>(n * p.pb);  // rows past N read as zero
    }
  } else {
    boff[0] = static_cast<uint32_t>((tid >> 2) * p.pb + n0 / 8 + (tid & 3) * 4);
    boff[1] = 0;
  }
  auto load_b = [&](int it) {
    const int64_t k0 = static_cast<int64_t>(it) * BK;
    if (BKIND == B_BITS_ALONG_K) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) breg[nb] = ld64(rb_bits, boff[nb] + static_cast<uint32_t>(k0 / 8));
    } else {
      bword = ld32(rb_bits, boff[0] + static_cast<uint32_t>(k0 * p.pb));
      if (tid < BK) bscale = p.kscale ? __uint_as_float(ld32(rb_scale, static_cast<uint32_t>((k0 + tid) * 4)))
                                      : (k0 + tid < p.K ? 1.0f : 0.0f);
    }
  };
  auto store_b = [&](int buf) {
    if (BKIND == B_BITS_ALONG_N) {
      uint8_t* bs = Bs + buf * B_TILE;
      const int k = tid >> 2, col = (tid & 3) * 4;
      const uint32_t neg = ~bword;
#pragma unroll
      for (int i = 0; i < 4; ++i) bs[(col + i) * LDB + k] = static_cast<uint8_t>(neg >> (8 * i));
      if (tid < BK) Ss[buf * BK + tid] = f32_to_bf16(bscale);
    }
  };

  // ---- main loop ---------------------------------------------------------
  load_a(0);
  load_b(0);
  store_a(As);
  store_b(0);
  uint64_t bcur[2] = {~breg[0], ~breg[1]};
  lds_barrier();

  for (int it = 0; it < nk; ++it) {
    const int cur = it & 1;
    const bool more = it + 1 < nk;
    if (more) {
      load_a(it + 1);
      load_b(it + 1);
    }
    const uint16_t* a_buf = As + cur * A_TILE;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 b0, b1;
      if (BKIND == B_BITS_ALONG_K) {
        const int sh = 8 * (2 * s + kg);
        b0 = signs_along_k(static_cast<uint32_t>(bcur[0] >> sh) & 0xFFu, one);
        b1 = signs_along_k(static_cast<uint32_t>(bcur[1] >> sh) & 0xFFu, one);
      } else {
        const uint8_t* bs = Bs + cur * B_TILE;
        const int kk = 16 * s + 8 * kg;
        const uint4 sc = *reinterpret_cast<const uint4*>(&Ss[cur * BK + kk]);
        const int c0 = 64 * wn + l32, c1 = c0 + 32;
        b0 = signs_across_k(*reinterpret_cast<const uint64_t*>(&bs[(c0 >> 3) * LDB + kk]), c0 & 7, sc);
        b1 = signs_across_k(*reinterpret_cast<const uint64_t*>(&bs[(c1 >> 3) * LDB + kk]), c1 & 7, sc);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int row = 128 * wm + 32 * mb + l32;
        const bf16x8 a =
            *reinterpret_cast<const bf16x8*>(&a_buf[row * LDA + a_chunk(AKIND, 2 * s + kg, row) * 8]);
        acc[mb][0] = mma(a, b0, acc[mb][0]);
        acc[mb][1] = mma(a, b1, acc[mb][1]);
      }
    }
    if (more) {
      store_a(As + (cur ^ 1) * A_TILE);
      store_b(cur ^ 1);
      if (BKIND == B_BITS_ALONG_K) {
        bcur[0] = ~breg[0];
        bcur[1] = ~breg[1];
      }
    }
    lds_barrier();
  }

  // ---- epilogue ------------------------------------------------------------
  if (EPI == EPI_FORWARD || EPI == EPI_PLAIN) {
    uint16_t* y = static_cast<uint16_t*>(p.out);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t col = n0 + 64 * wn + 32 * nb + l32;
      if (col >= p.N) continue;
      const float sc = (EPI == EPI_FORWARD && p.n_scale) ? p.n_scale[col] : 1.0f;
      const float bi = (EPI == EPI_FORWARD && p.n_bias) ? p.n_bias[col] : 0.0f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + 128 * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
          if (row < p.M) {
            float v = acc[mb][nb][r];
            if (EPI == EPI_FORWARD) {
              v = v * sc;
              v = v + bi;
            }
            y[row * p.N + col] = f32_to_bf16(v);
          }
        }
      }
    }
  } else {
    // E0 = acc + v[m]; row partials of E0 * sign_w; E = E0 * s[m]
    float* ev = static_cast<float*>(p.out);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      float part[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        part[r] = 0.0f;
        const int64_t row = m0 + 128 * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
        if (row >= p.M) continue;
        const float add = p.m_add ? p.m_add[row] : 0.0f;
        const float mul = p.m_scale ? p.m_scale[row] : 1.0f;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int64_t col = n0 + 64 * wn + 32 * nb + l32;
          if (col >= p.N) continue;
          const float e0 = acc[mb][nb][r] + add;
          if (p.w_bits) {
            const uint32_t byte = p.w_bits[row * p.pb + (col >> 3)];
            part[r] += ((byte >> (col & 7)) & 1u) ? e0 : -e0;
          }
          ev[row * p.N + col] = e0 * mul;
        }
      }
      if (p.gs_partial) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = part[r];
#pragma unroll
          for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
          part[r] = v;
        }
        if (l32 == 0) {
          const int64_t slot = 2 * static_cast<int64_t>(tn) + wn;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + 128 * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
            if (row < p.M) p.gs_partial[slot * p.M + row] = part[r];
          }
        }
      }
    }
  }
}


// ===========================================================================
// Wide tiles for the forward product: 256 x 256 outputs per workgroup of 4
// waves (2 x 2, each 128 x 128 = 4 x 4 blocks of 32 x 32 held in AGPRs), one
// workgroup per CU.  Operands reach LDS by direct buffer->LDS loads (no
// register staging) into four stages, issued three K steps ahead; the
// workgroup synchronises once per K step, three quarters into it, after
// which the next stage's first fragments are read while the step's last
// MFMAs run.  Output rows leave through LDS as 16-byte stores.
// ===========================================================================
namespace wide {
constexpr int BM = 256, BN = 256, BK = 64, THREADS = 256;
constexpr int A_STAGE = BM * BK * 2;  // bytes: 256 rows x 128 B, 16-byte chunks XOR-swizzled
constexpr int B_STAGE = BN * BK / 8;  // bytes: 256 rows x 8 B of sign bits
constexpr int EPL = 272;              // bytes per staged output row (256 + pad)
constexpr int LOADS_PER_STEP = 10;    // buffer->LDS loads per wave per K step
typedef __attribute__((address_space(3))) void lds_t;

// Chunk c of A row r is stored at chunk c ^ swz(r): the 16 rows that one
// ds_read_b128 quarter-wave touches then cover all 64 banks once.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Wait until at most N vector-memory operations of this wave are in flight
// (the buffer->LDS loads retire in order), then barrier the workgroup.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  compiler_fence();
  // s_waitcnt fields: vmcnt [3:0] and [15:14], expcnt [6:4] (7: none), lgkmcnt [11:8] (0)
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | 0x70);
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}

__global__ __launch_bounds__(THREADS, 1) void forward_kernel(Params p) {
  // one array per stage: the compiler then tracks each stage's direct loads
  // separately and waits only where this code says
  __shared__ __attribute__((aligned(16))) uint8_t A0[A_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t A1[A_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t A2[A_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t A3[A_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t B0[B_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t B1[B_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t B2[B_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t B3[B_STAGE];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, kg = lane >> 5;
  const int tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  const int tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint32_t one = bf16_one_pair();
  const int nk = static_cast<int>(p.K / BK);

  // A (x rows, K contiguous): the buffer starts at row m0, so rows past M
  // read zero.  Wave w fills rows 64w .. 64w+63 with 8 loads of 8 rows;
  // lane -> row 8j + lane/8 and LDS chunk lane%8, which holds global chunk
  // (lane%8) ^ swz(row); swz depends on j only through its parity.
  const __amdgpu_buffer_rsrc_t ra = rsrc(p.a + m0 * p.lda, (p.a_rows - m0) * p.lda * 2);
  const int q8 = lane >> 3, pos = lane & 7;
  uint32_t a_voff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    a_voff[par] = static_cast<uint32_t>((64 * wave + q8) * p.lda * 2 + 16 * (pos ^ (4 * par + (q8 >> 1))));
  const uint32_t a_row8 = static_cast<uint32_t>(8 * p.lda * 2);
  // B (sign bits along K): 256 rows x 8 bytes per stage; wave w fills rows
  // 64w .. 64w+63 with 2 loads of 4 bytes per lane.
  const __amdgpu_buffer_rsrc_t rb = rsrc(p.bits + n0 * p.pb, (p.bit_rows - n0) * p.pb);
  const uint32_t b_voff = static_cast<uint32_t>((64 * wave + (lane >> 1)) * p.pb + 4 * (lane & 1));
  const uint32_t b_row32 = static_cast<uint32_t>(32 * p.pb);

  // Steps past the end are issued too, at an offset past every buffer's
  // end: they read zero without touching memory and keep the number of
  // loads in flight the same on every step.
  auto issue = [&](int it, uint8_t* As, uint8_t* Bs) {
    const bool live = it < nk;
    const uint32_t k_off = live ? static_cast<uint32_t>(it) * (BK * 2) : 0x80000000u;
    const uint32_t kb = live ? static_cast<uint32_t>(it) * (BK / 8) : 0x80000000u;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_t*)(As + (64 * wave + 8 * j) * 128), 16, a_voff[j & 1],
                                               static_cast<int>(j * a_row8 + k_off), 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_t*)(Bs + (64 * wave + 32 * j) * 8), 4, b_voff,
                                               static_cast<int>(j * b_row32 + kb), 0, 0);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // fragments: a[buf][mb] rows of x, b[buf][nb] expanded signs; substep s
  // (k = 16s .. 16s+15 of the step) uses buffer s & 1
  bf16x8 a[2][4], b[2][4];
  uint64_t bits[4];
  auto load_a = [&](const uint8_t* As, int s, bf16x8* dst) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int row = 128 * wm + 32 * mb + l32;
      dst[mb] = *reinterpret_cast<const bf16x8*>(As + row * 128 + 16 * ((2 * s + kg) ^ swz(row)));
    }
  };
  auto load_bits = [&](const uint8_t* Bs) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      bits[nb] = ~*reinterpret_cast<const uint64_t*>(Bs + 8 * (128 * wn + 32 * nb + l32));
  };
  auto expand_b = [&](int s, bf16x8* dst) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      dst[nb] = signs_along_k(static_cast<uint32_t>(bits[nb] >> (8 * (2 * s + kg))) & 0xFFu, one);
  };
  auto mfmas = [&](int s) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mma(a[s & 1][mb], b[s & 1][nb], acc[mb][nb]);
  };

  // K step `it` on stage As (its bits already in `bits`, substep 0's
  // fragments in buffer 0).  After substep 2 every wave has finished step
  // it-1, so step it+3 may overwrite that step's stage (N3a, N3b); waiting
  // for all but the newest step's loads makes step it+1's stage (N1a, N1b)
  // complete, and its first fragments are read during substep 3.
  auto step = [&](int it, const uint8_t* As, const uint8_t* N1a, const uint8_t* N1b, uint8_t* N3a,
                  uint8_t* N3b) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      load_a(As, s + 1, a[(s + 1) & 1]);
      mfmas(s);
      expand_b(s + 1, b[(s + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    stage_barrier<LOADS_PER_STEP>();
    issue(it + 3, N3a, N3b);
    load_a(N1a, 0, a[0]);
    load_bits(N1b);
    mfmas(3);
    expand_b(0, b[0]);
    __builtin_amdgcn_sched_barrier(0);
  };

  issue(0, A0, B0);
  issue(1, A1, B1);
  issue(2, A2, B2);
  stage_barrier<2 * LOADS_PER_STEP>();
  load_a(A0, 0, a[0]);
  load_bits(B0);
  expand_b(0, b[0]);
  int it = 0;
  for (; it + 4 <= nk; it += 4) {
    step(it, A0, A1, B1, A3, B3);
    step(it + 1, A1, A2, B2, A0, B0);
    step(it + 2, A2, A3, B3, A1, B1);
    step(it + 3, A3, A0, B0, A2, B2);
  }
  if (it < nk) step(it, A0, A1, B1, A3, B3);
  if (it + 1 < nk) step(it + 1, A1, A2, B2, A0, B0);
  if (it + 2 < nk) step(it + 2, A2, A3, B3, A1, B1);

  // Epilogue: scale and bias, round to bf16, stage through LDS one quarter
  // (32 of the wave's 128 rows) at a time so each row segment of 128
  // outputs leaves as 16 lanes x 16 contiguous bytes.  Waves 0, 1 stage in
  // A0 and waves 2, 3 in A1, after every in-flight load has landed.
  stage_barrier<0>();
  uint16_t* y = static_cast<uint16_t*>(p.out);
  uint8_t* stg = (wave < 2 ? A0 : A1) + (wave & 1) * (32 * EPL);
  float sc[4], bi[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int64_t col = n0 + 128 * wn + 32 * nb + l32;
    sc[nb] = (col < p.N && p.n_scale) ? p.n_scale[col] : 1.0f;
    bi[nb] = (col < p.N && p.n_bias) ? p.n_bias[col] : 0.0f;
  }
  // Lanes l, l^1 trade one value per row pair so each holds two adjacent
  // columns of one row: even lanes row r, odd lanes row r+1.
  const bool odd = l32 & 1;
  const bool vec_ok = (p.N & 7) == 0;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float v0 = acc[mb][nb][r] * sc[nb];
        v0 = v0 + bi[nb];
        float v1 = acc[mb][nb][r + 1] * sc[nb];
        v1 = v1 + bi[nb];
        const float send = odd ? v0 : v1;
        const float recv = __int_as_float(
            __builtin_amdgcn_update_dpp(0, __float_as_int(send), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
        const float lo = odd ? recv : v0;
        const float hi = odd ? v1 : recv;
        const uint32_t word =
            static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
        const int row = 8 * (r >> 2) + 4 * kg + (r & 3) + (odd ? 1 : 0);
        *reinterpret_cast<uint32_t*>(stg + row * EPL + 2 * (32 * nb + (l32 & ~1))) = word;
      }
    }
    // 32 rows x 256 bytes: lane -> row 4i + lane/16, 16-byte chunk lane%16
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 4 * i + (lane >> 4), chunk = lane & 15;
      const uint4 v = *reinterpret_cast<const uint4*>(stg + row * EPL + 16 * chunk);
      const int64_t grow = m0 + 128 * wm + 32 * mb + row;
      const int64_t gcol = n0 + 128 * wn + 8 * chunk;
      if (grow < p.M) {
        if (vec_ok && gcol + 8 <= p.N) {
          *reinterpret_cast<uint4*>(y + grow * p.N + gcol) = v;
        } else {
          const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
          for (int t = 0; t < 8; ++t)
            if (gcol + t < p.N) y[grow * p.N + gcol + t] = e[t];
        }
      }
    }
  }
}
}  // namespace wide
}  // namespace mfma

// ---------------------------------------------------------------------------
// dispatch: returns 1 when the call is not for this path
// ---------------------------------------------------------------------------

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int grid_tiles(int64_t M, int64_t N) {
  return static_cast<int>(((M + mfma::BM - 1) / mfma::BM) * ((N + mfma::BN - 1) / mfma::BN));
}

// Buffer offsets are 32-bit: every operand must stay under 4 GiB.
static bool fits32(int64_t bytes) { return bytes < (int64_t{1} << 32); }

int mfma_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  if (dtype != QSTE_BF16 || cols % 64 != 0 || cols == 0 || m == 0 || !aligned16(x) || !aligned16(packed) ||
      !fits32(m * cols * 2) || !fits32(rows * cols / 8))
    return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(x);
  p.bits = packed;
  p.out = y;
  p.M = m; p.N = rows; p.K = cols;
  p.lda = cols; p.pb = cols / 8;
  p.a_rows = m; p.bit_rows = rows;
  p.n_scale = scale; p.n_bias = bias;
  const int grid = static_cast<int>(((m + mfma::wide::BM - 1) / mfma::wide::BM) *
                                    ((rows + mfma::wide::BN - 1) / mfma::wide::BN));
  mfma::wide::forward_kernel<<<grid, mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

int mfma_linear_dgrad(const void* dy, int dtype, const uint8_t* packed, const float* row_scale, void* dx,
                      int64_t m, int64_t rows, int64_t cols, hipStream_t stream) {
  if (dtype != QSTE_BF16 || cols % 64 != 0 || rows % 64 != 0 || rows == 0 || cols == 0 || m == 0 ||
      !aligned16(dy) || !aligned16(packed) || !fits32(m * rows * 2) || !fits32(rows * cols / 8))
    return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = packed;
  p.kscale = row_scale;
  p.out = dx;
  p.M = m; p.N = cols; p.K = rows;
  p.lda = rows; p.pb = cols / 8;
  p.a_rows = m; p.bit_rows = rows;
  mfma::gemm_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_N, mfma::EPI_PLAIN>
      <<<grid_tiles(m, cols), mfma::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

int64_t mfma_evidence_tiles(int64_t cols) { return 2 * ((cols + mfma::BN - 1) / mfma::BN); }

int mfma_evidence(const void* dy, int dtype, const uint8_t* packed_x, const float* x_scale, float* ev,
                  int64_t samples, int64_t rows, int64_t cols, const float* m_add, const float* m_scale,
                  const uint8_t* w_bits, float* gs_partial, hipStream_t stream) {
  if (dtype != QSTE_BF16 || cols % 64 != 0 || rows % 64 != 0 || rows == 0 || cols == 0 || samples == 0 ||
      !aligned16(dy) || !aligned16(packed_x) || !fits32(samples * rows * 2) || !fits32(samples * cols / 8))
    return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = packed_x;
  p.kscale = x_scale;
  p.out = ev;
  p.M = rows; p.N = cols; p.K = samples;
  p.lda = rows; p.pb = cols / 8;
  p.a_rows = samples; p.bit_rows = samples;
  p.m_add = m_add; p.m_scale = m_scale; p.w_bits = w_bits; p.gs_partial = gs_partial;
  mfma::gemm_kernel<mfma::A_ROWS_K, mfma::B_BITS_ALONG_N, mfma::EPI_EVIDENCE>
      <<<grid_tiles(rows, cols), mfma::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
