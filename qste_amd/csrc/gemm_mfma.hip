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
// operand (A) goes through LDS; the next K step's global loads are issued
// before the current step's MFMAs so their latency hides under compute.
// Where bits run along N they are staged through LDS as a small transposed
// byte tile (already inverted, so a set bit means "negative").
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

constexpr int BM = 256, BN = 128, BK = 64, THREADS = 256;
constexpr int LDA = BK + 8;        // bf16 per LDS row of A (144 B: conflict-free b128 reads)
constexpr int LDB = BK + 8;        // bytes per LDS row of staged bits ([n/8][k])

union Frag {
  bf16x8 v;
  uint32_t d[4];
  uint4 q;
};

__device__ __forceinline__ uint32_t pk_shl(uint32_t x, u16x2 sh) {
  u16x2 v = __builtin_bit_cast(u16x2, x);
  v = v << sh;
  return __builtin_bit_cast(uint32_t, v);
}

// 8 signs along k from one byte; `neg` has bit i set where k-offset i is -1.
__device__ __forceinline__ bf16x8 signs_along_k(uint32_t neg) {
  const uint32_t tt = neg | (neg << 16);
  Frag f;
  f.d[0] = (pk_shl(tt, u16x2{15, 14}) & 0x80008000u) | 0x3F803F80u;
  f.d[1] = (pk_shl(tt, u16x2{13, 12}) & 0x80008000u) | 0x3F803F80u;
  f.d[2] = (pk_shl(tt, u16x2{11, 10}) & 0x80008000u) | 0x3F803F80u;
  f.d[3] = (pk_shl(tt, u16x2{9, 8}) & 0x80008000u) | 0x3F803F80u;
  return f.v;
}

// 8 scaled signs across k: byte i of `neg8` is the (inverted) bit row for
// k-offset i; this lane's column is bit `bit` of each byte.  `scale` holds
// the 8 nonnegative bf16 scales as pairs; a set bit sets the sign.
__device__ __forceinline__ bf16x8 signs_across_k(uint64_t neg8, int bit, uint4 scale) {
  const uint64_t x = neg8 >> bit;
  const uint32_t lo = static_cast<uint32_t>(x), hi = static_cast<uint32_t>(x >> 32);
  Frag f;
  f.d[0] = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C010C00u), u16x2{15, 15}) | scale.x;
  f.d[1] = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C030C02u), u16x2{15, 15}) | scale.y;
  f.d[2] = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C050C04u), u16x2{15, 15}) | scale.z;
  f.d[3] = pk_shl(__builtin_amdgcn_perm(hi, lo, 0x0C070C06u), u16x2{15, 15}) | scale.w;
  return f.v;
}

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint16_t bf16_rne(float f) { return f32_to_bf16(f); }

// Workgroup -> output tile.  Consecutive workgroup ids land on different
// XCDs (round-robin), so ids are first regrouped so each XCD gets a
// contiguous range, then walked in column-major groups of 8 M-tiles so
// workgroups that run together share operand tiles in their XCD's L2.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
  constexpr int G = 8;
  const int per_group = G * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * G;
  const int gm = min(tiles_m - first_m, G);
  const int in_group = pid % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

struct Params {
  const uint16_t* a;     // bf16 dense operand (x or dy)
  const uint8_t* bits;   // packed signs of the +-1 operand
  const float* kscale;   // per-k scale folded into the bit operand (dgrad/evidence)
  void* out;
  int64_t M, N, K;
  int64_t lda;           // elements between rows of the dense source
  int64_t pb;            // bytes per packed row
  // epilogue
  const float* n_scale;  // forward
  const float* n_bias;   // forward
  const float* m_add;    // evidence
  const float* m_scale;  // evidence
  const uint8_t* w_bits; // evidence: sign_w for the scale gradient
  float* gs_partial;     // evidence: [2 * tiles_n][M]
};

// ---------------------------------------------------------------------------
// forward: y[m, n] = sum_k x[m, k] sign_w[n, k]; bits of row n run along k
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(THREADS, 2) void forward_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, kg = lane >> 5;
  const int tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  const int tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  uint4 areg[8];
  const int arow = tid >> 3, achunk = tid & 7;
  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = m0 + arow + 32 * i;
      areg[i] = r < p.M ? *reinterpret_cast<const uint4*>(p.a + r * p.lda + k0 + achunk * 8)
                        : make_uint4(0, 0, 0, 0);
    }
  };
  uint64_t breg[2];
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t n = n0 + 64 * wn + 32 * nb + l32;
      breg[nb] = n < p.N ? *reinterpret_cast<const uint64_t*>(p.bits + n * p.pb + k0 / 8) : 0ull;
    }
  };

  load_a(0);
  load_b(0);
  for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<uint4*>(&As[(arow + 32 * i) * LDA + achunk * 8]) = areg[i];
    __syncthreads();
    const uint64_t neg0 = ~breg[0], neg1 = ~breg[1];
    if (k0 + BK < p.K) {
      load_a(k0 + BK);
      load_b(k0 + BK);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int sh = 8 * (2 * s + kg);
      bf16x8 b0 = signs_along_k(static_cast<uint32_t>(neg0 >> sh) & 0xFFu);
      bf16x8 b1 = signs_along_k(static_cast<uint32_t>(neg1 >> sh) & 0xFFu);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int row = 128 * wm + 32 * mb + l32;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&As[row * LDA + 16 * s + 8 * kg]);
        acc[mb][0] = mma(a, b0, acc[mb][0]);
        acc[mb][1] = mma(a, b1, acc[mb][1]);
      }
    }
  }

  uint16_t* y = static_cast<uint16_t*>(p.out);
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = n0 + 64 * wn + 32 * nb + l32;
    if (col >= p.N) continue;
    const float sc = p.n_scale ? p.n_scale[col] : 1.0f;
    const float bi = p.n_bias ? p.n_bias[col] : 0.0f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + 128 * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
        if (row < p.M) {
          float v = acc[mb][nb][r] * sc;
          v = v + bi;
          y[row * p.N + col] = bf16_rne(v);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Bits along N, staged per K step into LDS as [n/8][k] inverted bytes, and
// the per-k scale as bf16.  Thread t stages one dword (32 columns) of row
// k = t / 4 of the tile.
// ---------------------------------------------------------------------------
struct BitStage {
  uint32_t word;
  float scale;
};

__device__ __forceinline__ BitStage load_bits_kn(const Params& p, int64_t k0, int64_t n0, int tid) {
  BitStage s;
  const int64_t k = k0 + (tid >> 2);
  const int64_t byte = n0 / 8 + (tid & 3) * 4;
  s.word = (k < p.K && byte < p.pb) ? *reinterpret_cast<const uint32_t*>(p.bits + k * p.pb + byte) : 0u;
  s.scale = 0.0f;
  if (tid < BK) {
    const int64_t kk = k0 + tid;
    s.scale = kk < p.K ? (p.kscale ? p.kscale[kk] : 1.0f) : 0.0f;
  }
  return s;
}

__device__ __forceinline__ void store_bits_kn(uint8_t* Bs, uint16_t* Ss, const BitStage& s, int tid) {
  const int k = tid >> 2;
  const int col = (tid & 3) * 4;
  const uint32_t neg = ~s.word;
#pragma unroll
  for (int i = 0; i < 4; ++i) Bs[(col + i) * LDB + k] = static_cast<uint8_t>(neg >> (8 * i));
  if (tid < BK) Ss[tid] = bf16_rne(s.scale);
}

__device__ __forceinline__ bf16x8 b_frag_kn(const uint8_t* Bs, const uint16_t* Ss, int ncol, int s,
                                            int kg) {
  const int kk = 16 * s + 8 * kg;
  const uint64_t neg8 = *reinterpret_cast<const uint64_t*>(&Bs[(ncol >> 3) * LDB + kk]);
  const uint4 sc = *reinterpret_cast<const uint4*>(&Ss[kk]);
  return signs_across_k(neg8, ncol & 7, sc);
}

// ---------------------------------------------------------------------------
// dgrad: dx[m, n] = sum_k dy[m, k] bf16(s[k]) sign_w[k, n]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(THREADS, 2) void dgrad_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[(BN / 8) * LDB];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[BK];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, kg = lane >> 5;
  const int tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  const int tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  uint4 areg[8];
  const int arow = tid >> 3, achunk = tid & 7;
  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = m0 + arow + 32 * i;
      areg[i] = r < p.M ? *reinterpret_cast<const uint4*>(p.a + r * p.lda + k0 + achunk * 8)
                        : make_uint4(0, 0, 0, 0);
    }
  };
  BitStage bst = load_bits_kn(p, 0, n0, tid);
  load_a(0);
  for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<uint4*>(&As[(arow + 32 * i) * LDA + achunk * 8]) = areg[i];
    store_bits_kn(Bs, Ss, bst, tid);
    __syncthreads();
    if (k0 + BK < p.K) {
      load_a(k0 + BK);
      bst = load_bits_kn(p, k0 + BK, n0, tid);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 b0 = b_frag_kn(Bs, Ss, 64 * wn + l32, s, kg);
      const bf16x8 b1 = b_frag_kn(Bs, Ss, 64 * wn + 32 + l32, s, kg);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int row = 128 * wm + 32 * mb + l32;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&As[row * LDA + 16 * s + 8 * kg]);
        acc[mb][0] = mma(a, b0, acc[mb][0]);
        acc[mb][1] = mma(a, b1, acc[mb][1]);
      }
    }
  }

  uint16_t* dx = static_cast<uint16_t*>(p.out);
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = n0 + 64 * wn + 32 * nb + l32;
    if (col >= p.N) continue;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + 128 * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
        if (row < p.M) dx[row * p.N + col] = bf16_rne(acc[mb][nb][r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// evidence: E[m, n] = sum_k dy[k, m] bf16(xs[k]) sign_x[k, n]  (m = output row
// r of the layer, k = sample t).  dy is read as [k][m] rows, an 8 x 8 block
// per thread, transposed in registers with v_perm and written to LDS as
// [m][k] with the 16-byte chunk index XOR-swizzled by (m / 8) so the
// transposed stores do not collide on LDS banks.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz(int chunk, int row) { return chunk ^ ((row >> 3) & 7); }

__global__ __launch_bounds__(THREADS, 2) void evidence_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[(BN / 8) * LDB];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[BK];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, kg = lane >> 5;
  const int tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  const int tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  // this thread's 8 x 8 block: m in [m0 + 8*rb, +8), k in [k0 + 8*kb, +8)
  const int rb = tid & 31, kb = tid >> 5;
  uint4 areg[8];
  auto load_a = [&](int64_t k0) {
    const int64_t m = m0 + 8 * rb;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = k0 + 8 * kb + i;
      areg[i] = (k < p.K && m < p.M) ? *reinterpret_cast<const uint4*>(p.a + k * p.lda + m)
                                     : make_uint4(0, 0, 0, 0);
    }
  };
  BitStage bst = load_bits_kn(p, 0, n0, tid);
  load_a(0);
  for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
    __syncthreads();
    {
      // transpose: out[j] holds k = 8kb..8kb+7 for m = 8rb + j
      const uint32_t* in = reinterpret_cast<const uint32_t*>(areg);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        uint4 o;
        o.x = __builtin_amdgcn_perm(in[1 * 4 + (j >> 1)], in[0 * 4 + (j >> 1)], sel);
        o.y = __builtin_amdgcn_perm(in[3 * 4 + (j >> 1)], in[2 * 4 + (j >> 1)], sel);
        o.z = __builtin_amdgcn_perm(in[5 * 4 + (j >> 1)], in[4 * 4 + (j >> 1)], sel);
        o.w = __builtin_amdgcn_perm(in[7 * 4 + (j >> 1)], in[6 * 4 + (j >> 1)], sel);
        const int row = 8 * rb + j;
        *reinterpret_cast<uint4*>(&As[row * LDA + swz(kb, row) * 8]) = o;
      }
    }
    store_bits_kn(Bs, Ss, bst, tid);
    __syncthreads();
    if (k0 + BK < p.K) {
      load_a(k0 + BK);
      bst = load_bits_kn(p, k0 + BK, n0, tid);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 b0 = b_frag_kn(Bs, Ss, 64 * wn + l32, s, kg);
      const bf16x8 b1 = b_frag_kn(Bs, Ss, 64 * wn + 32 + l32, s, kg);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int row = 128 * wm + 32 * mb + l32;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&As[row * LDA + swz(2 * s + kg, row) * 8]);
        acc[mb][0] = mma(a, b0, acc[mb][0]);
        acc[mb][1] = mma(a, b1, acc[mb][1]);
      }
    }
  }

  // epilogue: E0 = acc + v[m]; row partials of E0 * sign_w; E = E0 * s[m]
  float* ev = static_cast<float*>(p.out);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    float part[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
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

}  // namespace mfma

// ---------------------------------------------------------------------------
// dispatch: returns 1 when the call is not for this path
// ---------------------------------------------------------------------------

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int grid_tiles(int64_t M, int64_t N) {
  return static_cast<int>(((M + mfma::BM - 1) / mfma::BM) * ((N + mfma::BN - 1) / mfma::BN));
}

int mfma_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  if (dtype != QSTE_BF16 || cols % 64 != 0 || cols == 0 || !aligned16(x) || !aligned16(packed)) return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(x);
  p.bits = packed;
  p.out = y;
  p.M = m; p.N = rows; p.K = cols;
  p.lda = cols; p.pb = cols / 8;
  p.n_scale = scale; p.n_bias = bias;
  mfma::forward_kernel<<<grid_tiles(m, rows), mfma::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

int mfma_linear_dgrad(const void* dy, int dtype, const uint8_t* packed, const float* row_scale, void* dx,
                      int64_t m, int64_t rows, int64_t cols, hipStream_t stream) {
  if (dtype != QSTE_BF16 || cols % 64 != 0 || rows % 64 != 0 || rows == 0 || cols == 0 || !aligned16(dy) ||
      !aligned16(packed))
    return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = packed;
  p.kscale = row_scale;
  p.out = dx;
  p.M = m; p.N = cols; p.K = rows;
  p.lda = rows; p.pb = cols / 8;
  mfma::dgrad_kernel<<<grid_tiles(m, cols), mfma::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

int64_t mfma_evidence_tiles(int64_t cols) { return 2 * ((cols + mfma::BN - 1) / mfma::BN); }

int mfma_evidence(const void* dy, int dtype, const uint8_t* packed_x, const float* x_scale, float* ev,
                  int64_t samples, int64_t rows, int64_t cols, const float* m_add, const float* m_scale,
                  const uint8_t* w_bits, float* gs_partial, hipStream_t stream) {
  if (dtype != QSTE_BF16 || cols % 64 != 0 || rows % 64 != 0 || rows == 0 || cols == 0 || samples == 0 ||
      !aligned16(dy) || !aligned16(packed_x))
    return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = packed_x;
  p.kscale = x_scale;
  p.out = ev;
  p.M = rows; p.N = cols; p.K = samples;
  p.lda = rows; p.pb = cols / 8;
  p.m_add = m_add; p.m_scale = m_scale; p.w_bits = w_bits; p.gs_partial = gs_partial;
  mfma::evidence_kernel<<<grid_tiles(rows, cols), mfma::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

int gemv_linear_forward(const void*, int, const uint8_t*, const float*, const float*, void*, int64_t,
                        int64_t, int64_t, hipStream_t) {
  return 1;
}

}  // namespace qste
