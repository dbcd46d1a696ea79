// bf16 / fp16 MFMA products over packed signs for gfx950 (CDNA4).
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
//   evidence  E  = dy^T [M=R, K=T] . (xs (*) sign_x) bits run along N, dy
//             is read as stored ([K][M]) and transposed by the LDS read;
//             fused epilogue + v[m], row partials of E0 . sign_w, * scale[m]
//
// One kernel template serves all three (wide_kernel below): 256 x 256
// outputs per workgroup of 4 waves, one workgroup per CU, the dense operand
// brought into LDS by direct buffer->LDS loads over four stages, and buffer
// loads' zero fill for every ragged edge.
//
// MFMA 32x32x16 bf16 operand layout used here: lane l holds A[l%32][8(l/32)
// + i] and B[8(l/32) + i][l%32], i = 0..7; the accumulator's register r
// holds D[8(r/4) + 4(l/32) + r%4][l%32].
#include <map>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace qste {
namespace mfma {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kRsrcWord3 = 0x00020000u;

enum { A_ROWS_M = 0, A_ROWS_K = 1 };        // A[m][k] stored with k (or m) contiguous
// B_BITS_ALONG_K_SCALED: bits along K (a transposed copy of the signs) and
// a per-k bf16 scale, both brought in by direct loads.
enum { B_BITS_ALONG_K = 0, B_BITS_ALONG_N = 1, B_BITS_ALONG_K_SCALED = 2 };
// EPI_PARTIAL: the bare fp32 accumulators of one K range of a split-K
// evidence, finished by evidence_combine_kernel.  EPI_FORWARD_F32: the
// forward's scale and bias, stored as fp32 (the fp32 products, whose dense
// operand arrives as three bf16 limbs along K).
enum { EPI_FORWARD = 0, EPI_PLAIN = 1, EPI_EVIDENCE = 2, EPI_PARTIAL = 3, EPI_FORWARD_F32 = 4 };

struct Params {
  const uint16_t* a;     // bf16 dense operand (x or dy)
  const uint8_t* bits;   // packed signs of the +-1 operand
  const float* kscale;   // per-k scale folded into the bit operand (dgrad/evidence)
  const uint16_t* kscale16;  // the same as bf16 (bits along K with a scale)
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
  int64_t w_pb;          // evidence: bytes per row of w_bits
  float* gs_partial;     // evidence: [WAVES_N * tiles_n][M]
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFll ? 0xFFFFFFFFu : static_cast<uint32_t>(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(n), kRsrcWord3);
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

// 8 scaled signs along k: as signs_along_k, with the 8 nonnegative bf16
// scales (as pairs) in place of +1.
__device__ __forceinline__ bf16x8 scaled_signs_along_k(uint32_t neg, uint4 scale) {
  const uint32_t tt = neg * 0x10001u;
  u32x4 r;
  r.x = (pk_shl(tt, u16x2{15, 14}) & 0x80008000u) | scale.x;
  r.y = (pk_shl(tt, u16x2{13, 12}) & 0x80008000u) | scale.y;
  r.z = (pk_shl(tt, u16x2{11, 10}) & 0x80008000u) | scale.z;
  r.w = (pk_shl(tt, u16x2{9, 8}) & 0x80008000u) | scale.w;
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

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The same products on fp16 operands: the 16-bit fragments are only
// reinterpreted (a sign insertion into a nonnegative 16-bit value is the same
// bit operation in both formats); only the +1 pattern, the MFMA and the
// rounding of scales and outputs depend on DT.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ f32x16 mma_dt(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (DT == QSTE_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  } else {
    return mma(a, b, c);
  }
}

// a pair of +1.0 in DT (bf16 0x3F80, fp16 0x3C00), held in a VGPR
template <int DT>
__device__ __forceinline__ uint32_t one_pair() {
  if constexpr (DT == QSTE_F16) {
    uint32_t v;
    asm volatile("v_mov_b32 %0, 0x3C003C00" : "=v"(v));
    return v;
  } else {
    return bf16_one_pair();
  }
}

template <int DT>
__device__ __forceinline__ uint16_t round16(float f) {
  if constexpr (DT == QSTE_F16) return f32_to_f16(f);
  else return f32_to_bf16(f);
}

// two outputs to a 16-bit pair (lo in bits 0..15)
template <int DT>
__device__ __forceinline__ uint32_t round16x2(float lo, float hi) {
  if constexpr (DT == QSTE_F16)
    return static_cast<uint32_t>(f32_to_f16(lo)) | (static_cast<uint32_t>(f32_to_f16(hi)) << 16);
  else return f32x2_to_bf16x2(lo, hi);
}

// Workgroup -> output tile.  Consecutive workgroup ids land on different
// XCDs (round-robin), so ids are first regrouped so each XCD gets a
// contiguous range, then walked in column-major groups of G M-tiles, so the
// workgroups that run together on one XCD share G dense-operand row blocks
// (the large operand) and many small bit tiles in that XCD's L2.  G = 2 for
// the forward and dX, 1 for the evidence (dense operand as rows of K), as
// measured fastest for each.
template <int G>
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
  const int per_group = G * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * G;
  const int gm = min(tiles_m - first_m, G);
  const int in_group = pid % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// ===========================================================================
// 256 x 256 outputs per workgroup of 4 waves (each all 256 rows and 64
// columns = 8 x 2 blocks of 32 x 32 held in AGPRs), one workgroup per CU.  The dense operand
// reaches LDS by direct buffer->LDS loads (no register staging) into four
// stages, issued three K steps ahead; the workgroup synchronises once per K
// step, three quarters into it, after which the next stage's first
// fragments are read while the step's last MFMAs run.  bf16 outputs leave
// through LDS as 16-byte row segments.
// ===========================================================================
namespace wide {
constexpr int BM = 256, BN = 256, BK = 64, THREADS = 256;
constexpr int A_STAGE = BM * BK * 2;  // bytes: 256 rows x 128 B, 16-byte chunks XOR-swizzled
constexpr int B_STAGE = BN * BK / 8;  // bytes: 256 rows x 8 B of sign bits
// Each wave covers all 256 rows and a quarter of the columns: every sign
// fragment it expands feeds 8 MFMAs (the expansion VALU work, not the LDS
// reads of the dense operand, is what limits a wave).
constexpr int WAVES_N = 4;            // waves across N, the rest across M
constexpr int WAVES_M = 4 / WAVES_N;
constexpr int WMR = BM / WAVES_M;     // rows per wave
constexpr int WNC = BN / WAVES_N;     // columns per wave
constexpr int MBN = WMR / 32, NBN = WNC / 32;  // 32 x 32 blocks per wave
constexpr int EPL = 2 * WNC + 16;     // bytes per staged output row (+ pad)
constexpr int EPR = WNC == 128 ? 32 : 16;  // staged output rows per piece
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

// Bits along N (dgrad, evidence) are staged transposed, [n/8][k] with a
// pitch of LDB_N bytes, inverted so a set bit means "negative", and the per-k
// scale as bf16 beside them: the transposition needs registers, so those
// loads go through VGPRs one step before their stage is written.
constexpr int LDB_N = BK + 8;
constexpr int BN_STAGE = (BN / 8) * LDB_N;  // bytes
template <int BKIND>
struct Loads {
  // buffer loads per wave per K step: 8 A loads, plus 2 direct bit loads
  // (and 1 scale load), or 3 register loads of bits along N
  static constexpr int value = BKIND == B_BITS_ALONG_K ? 10 : 11;
};

// A given as rows of K (evidence: A = dy^T, dy stored [K][M]) is staged
// [k][m] with two k-rows interleaved per 16-byte chunk (one direct load
// covers a row pair) and row pairs APK bytes apart; fragments are read with
// ds_read_b64_tr_b16, which hands lane 4a+b of each 16-lane group element b
// of the 8-byte reads of lanes a, a+4, a+8, a+12.
constexpr int APK = 1152;                    // bytes per staged k-row pair (1024 + pad)
constexpr int A_STAGE_K = (BK / 2) * APK;    // bytes
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// One output tile; the LDS stages are the caller's (one __shared__ array per
// stage, so that the compiler tracks each stage's direct loads separately
// and waits only where this code says).
template <int AKIND, int BKIND, int EPI, int DT>
__device__ __forceinline__ void wide_tile(const Params& p, int pid, uint8_t* A0, uint8_t* A1, uint8_t* A2,
                                          uint8_t* A3, uint8_t* B0, uint8_t* B1, uint8_t* B2, uint8_t* B3,
                                          uint16_t* Sc) {
  constexpr int NL = Loads<BKIND>::value;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int l32 = lane & 31, kg = lane >> 5;
  const int tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  const int tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of<AKIND == A_ROWS_K ? 1 : 2>(pid, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint32_t one = one_pair<DT>();
  const int nk = static_cast<int>((p.K + BK - 1) / BK);  // K % BK != 0 only for A as rows of K

  // A (rows of M, K contiguous): the buffer starts at row m0, so rows past
  // M read zero.  Wave w fills rows 64w .. 64w+63 with 8 loads of 8 rows;
  // lane -> row 8j + lane/8 and LDS chunk lane%8, which holds global chunk
  // (lane%8) ^ swz(row); swz depends on j only through its parity.
  // A as rows of K: the buffer starts at column m0, so k-rows past K read
  // zero.  Wave w fills row pairs 8w .. 8w+7, one direct load each; lane i
  // loads chunk i/2 of k-row 2P + i%2.
  __amdgpu_buffer_rsrc_t ra;
  uint32_t a_voff[2], a_row8;
  if (AKIND == A_ROWS_M) {
    ra = rsrc(p.a + m0 * p.lda, (p.a_rows - m0) * p.lda * 2);
    const int q8 = lane >> 3, pos = lane & 7;
#pragma unroll
    for (int par = 0; par < 2; ++par)
      a_voff[par] = static_cast<uint32_t>((64 * wave + q8) * p.lda * 2 + 16 * (pos ^ (4 * par + (q8 >> 1))));
    a_row8 = static_cast<uint32_t>(8 * p.lda * 2);
  } else {
    ra = rsrc(p.a + m0, (p.a_rows * p.lda - m0) * 2);
    a_voff[0] = a_voff[1] = static_cast<uint32_t>(((16 * wave + (lane & 1)) * p.lda + 8 * (lane >> 1)) * 2);
    a_row8 = static_cast<uint32_t>(2 * p.lda * 2);  // one row pair
  }
  const uint32_t a_kstep = AKIND == A_ROWS_M ? BK * 2 : static_cast<uint32_t>(BK * p.lda * 2);

  // B along K: 256 rows x 8 bytes per stage, wave w fills rows 64w ..
  // 64w+63 with 2 direct loads of 4 bytes per lane.
  // B along N: 64 k-rows x 32 bytes per stage; thread t loads the dwords
  // t and t + 256 (k-row d/8, bytes 4(d%8) ..) and one scale, k = t % 64.
  __amdgpu_buffer_rsrc_t rb;
  uint32_t b_voff, b_step;
  __amdgpu_buffer_rsrc_t rs = rsrc(p.kscale, p.kscale ? p.K * 4 : 0);
  // bf16 scales are padded with zeros to a whole number of K steps
  const __amdgpu_buffer_rsrc_t rs16 = rsrc(p.kscale16, BKIND == B_BITS_ALONG_K_SCALED ? int64_t{nk} * BK * 2 : 0);
  if (BKIND != B_BITS_ALONG_N) {
    rb = rsrc(p.bits + n0 * p.pb, (p.bit_rows - n0) * p.pb);
    b_voff = static_cast<uint32_t>((64 * wave + (lane >> 1)) * p.pb + 4 * (lane & 1));
    b_step = static_cast<uint32_t>(32 * p.pb);
  } else {
    rb = rsrc(p.bits + n0 / 8, p.bit_rows * p.pb - n0 / 8);
    b_voff = static_cast<uint32_t>((tid >> 3) * p.pb + 4 * (tid & 7));
    b_step = static_cast<uint32_t>(32 * p.pb);  // dword t + 256 is 32 k-rows further
  }
  uint32_t bw[2] = {0u, 0u};
  uint32_t bsv = 0u;   // loaded scale bits (with a per-k scale)
  float balt = 0.0f;   // 1 or 0 (without one: k < K)

  // Steps past the end are issued too, at an offset past every buffer's
  // end: they read zero without touching memory and keep the number of
  // loads in flight the same on every step.
  // part < 0: the whole step; part 0..3: a quarter of it (the register
  // loads of bits along N first, the direct bit loads of bits along K last)
  auto issue = [&](int it, uint8_t* As, uint8_t* Bs, uint16_t* Ss, int part = -1) {
    const bool live = it < nk;
    if (BKIND == B_BITS_ALONG_N && part <= 0) {
      const uint32_t koff = live ? static_cast<uint32_t>(it) * BK * static_cast<uint32_t>(p.pb) : 0x80000000u;
      bw[0] = ld32(rb, b_voff + koff);
      bw[1] = ld32(rb, b_voff + b_step + koff);
      const uint32_t soff = live ? static_cast<uint32_t>((it * BK + (tid & 63)) * 4) : 0x80000000u;
      bsv = ld32(rs, soff);
      balt = static_cast<float>(static_cast<int>(live) & static_cast<int>(it * BK + (tid & 63) < p.K));
    }
    const uint32_t k_off = live ? static_cast<uint32_t>(it) * a_kstep : 0x80000000u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (part >= 0 && (j >> 1) != part) continue;
      uint8_t* dst = AKIND == A_ROWS_M ? As + (64 * wave + 8 * j) * 128 : As + (8 * wave + j) * APK;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_t*)dst, 16, a_voff[j & 1],
                                               static_cast<int>(j * a_row8 + k_off), 0, 0);
    }
    if (BKIND != B_BITS_ALONG_N && (part < 0 || part == 3)) {
      const uint32_t kb = live ? static_cast<uint32_t>(it) * (BK / 8) : 0x80000000u;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_t*)(Bs + (64 * wave + 32 * j) * 8), 4, b_voff,
                                                 static_cast<int>(j * b_step + kb), 0, 0);
      if (BKIND == B_BITS_ALONG_K_SCALED) {
        // wave w brings the bf16 scales of k = 16w .. 16w+15, a pair per
        // lane (lanes 0..7: direct loads narrower than a dword still take a
        // dword slot per lane)
        const uint32_t ks = live ? static_cast<uint32_t>(it * BK + 16 * wave) * 2 : 0x80000000u;
        if (lane < 8)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs16, (lds_t*)(Ss + 16 * wave), 4,
                                                   static_cast<uint32_t>(4 * lane), static_cast<int>(ks), 0, 0);
      }
    }
  };
  // bits along N: write the staged registers of a step into its stage
  auto store_b = [&](uint8_t* Bs, uint16_t* Ss) {
    if (BKIND == B_BITS_ALONG_N) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int d = tid + 256 * h;
        const int k = d >> 3, g = d & 7;
        const uint32_t neg = ~bw[h];
#pragma unroll
        for (int i = 0; i < 4; ++i) Bs[(4 * g + i) * LDB_N + k] = static_cast<uint8_t>(neg >> (8 * i));
      }
      if (tid < BK) Ss[tid] = round16<DT>(p.kscale ? __uint_as_float(bsv) : balt);
    }
  };

  f32x16 acc[MBN][NBN];
#pragma unroll
  for (int i = 0; i < MBN; ++i)
#pragma unroll
    for (int j = 0; j < NBN; ++j) acc[i][j] = f32x16{};

  // fragments: a[buf][mb] dense rows, b[buf][nb] expanded signs; substep s
  // (k = 16s .. 16s+15 of the step) uses buffer s & 1
  bf16x8 a[2][MBN], b[2][NBN];
  uint64_t bits[NBN];
  uint4 kscl[4];  // bits along K with a scale: the step's bf16 scales of this lane's k, per substep
  // A as rows of K: this lane, as a source of the transposed read, names
  // k-row 16s + 8kg + 4h + t and m = 128wm + 32mb + 16(g%2) + 4a .. +3
  // (lane = 16g + 4a... with t = (lane%16)/4, a = lane%4, g = lane/16);
  // as a destination it receives A[m = l32][k = 16s + 8kg + 4h + 0..3].
  const int tr_t = (lane & 15) >> 2, tr_a = lane & 3, tr_g = lane >> 4;
  const int tr_base = APK * (4 * (tr_g >> 1) + (tr_t >> 1)) + 32 * (WMR / 8 * wm + 2 * (tr_g & 1) + (tr_a >> 1)) +
                      16 * (tr_t & 1) + 8 * (tr_a & 1);
  auto load_a = [&](const uint8_t* As, int s, bf16x8* dst) {
#pragma unroll
    for (int mb = 0; mb < MBN; ++mb) {
      if (AKIND == A_ROWS_M) {
        const int row = WMR * wm + 32 * mb + l32;
        dst[mb] = *reinterpret_cast<const bf16x8*>(As + row * 128 + 16 * ((2 * s + kg) ^ swz(row)));
      } else {
        const uint8_t* src = As + tr_base + APK * 8 * s + 128 * mb;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(src));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(src + 2 * APK));
        dst[mb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };
  // bits along K: this lane's 64 k-bits of each of its columns, as stored
  // (a set bit is +1); the expansions invert them, so no arithmetic waits on
  // these reads (LDS reads complete in order: a use right after this read
  // would also wait for every dense-fragment read issued before it)
  // (and, with a per-k scale, the step's scales for this lane's k: read
  // here, once per step, rather than beside each expansion, where a use
  // would wait for every dense-fragment read issued before it)
  auto load_bits = [&](const uint8_t* Bs, const uint16_t* Ss) {
    if (BKIND != B_BITS_ALONG_N) {
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) bits[nb] = *reinterpret_cast<const uint64_t*>(Bs + 8 * (WNC * wn + 32 * nb + l32));
    }
    if (BKIND == B_BITS_ALONG_K_SCALED) {
#pragma unroll
      for (int q = 0; q < 4; ++q) kscl[q] = *reinterpret_cast<const uint4*>(Ss + 16 * q + 8 * kg);
    }
  };
  // the inverted byte of k-bits of substep s (a set bit is -1)
  auto neg_byte = [&](int nb, int s) { return ~static_cast<uint32_t>(bits[nb] >> (8 * (2 * s + kg))) & 0xFFu; };
  auto expand_b = [&](const uint8_t* Bs, const uint16_t* Ss, int s, bf16x8* dst) {
    if (BKIND == B_BITS_ALONG_K) {
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) dst[nb] = signs_along_k(neg_byte(nb, s), one);
    } else if (BKIND == B_BITS_ALONG_K_SCALED) {
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) dst[nb] = scaled_signs_along_k(neg_byte(nb, s), kscl[s]);
    } else {
      const int kk = 16 * s + 8 * kg;
      const uint4 sc = *reinterpret_cast<const uint4*>(Ss + kk);
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        const int c = WNC * wn + 32 * nb + l32;
        dst[nb] = signs_across_k(*reinterpret_cast<const uint64_t*>(Bs + (c >> 3) * LDB_N + kk), c & 7, sc);
      }
    }
  };
  auto load_a1 = [&](const uint8_t* As, int s, int mb, bf16x8* dst) {
    if (AKIND == A_ROWS_M) {
      const int row = WMR * wm + 32 * mb + l32;
      dst[mb] = *reinterpret_cast<const bf16x8*>(As + row * 128 + 16 * ((2 * s + kg) ^ swz(row)));
    } else {
      const uint8_t* src = As + tr_base + APK * 8 * s + 128 * mb;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(src));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(src + 2 * APK));
      dst[mb] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  auto expand_b1 = [&](const uint8_t* Bs, const uint16_t* Ss, int s, int nb, bf16x8* dst) {
    if (BKIND == B_BITS_ALONG_K) {
      dst[nb] = signs_along_k(neg_byte(nb, s), one);
    } else if (BKIND == B_BITS_ALONG_K_SCALED) {
      dst[nb] = scaled_signs_along_k(neg_byte(nb, s), kscl[s]);
    } else {
      const int kk = 16 * s + 8 * kg;
      const uint4 sc = *reinterpret_cast<const uint4*>(Ss + kk);
      const int c = WNC * wn + 32 * nb + l32;
      dst[nb] = signs_across_k(*reinterpret_cast<const uint64_t*>(Bs + (c >> 3) * LDB_N + kk), c & 7, sc);
    }
  };
  // MFMA chunk q (0..3) of a substep: blocks 4q .. 4q+3 in (mb, nb) order
  auto mfma_row = [&](int s, int q) {
#pragma unroll
    for (int i = 4 * q; i < 4 * q + 4; ++i)
      acc[i / NBN][i % NBN] = mma_dt<DT>(a[s & 1][i / NBN], b[s & 1][i % NBN], acc[i / NBN][i % NBN]);
  };

  // K step `it` on stage (As, Bs, Ss); substep 0's fragments are in buffer 0.
  // After substep 2 every wave has finished step it-1, so step it+3 may
  // overwrite that step's stage (N3*).  Waiting for all but the newest
  // step's direct loads (its 8 A loads when bits run along N, whose 3
  // register loads are issued first) completes step it+1's stage (N1*) and,
  // for bits along N, the registers of step it+2, which are then written to
  // its stage (N2*).
  // Step it+1's first fragments are read while substep 3 runs.
  auto step = [&](int it, const uint8_t* As, const uint8_t* Bs, const uint16_t* Ss, const uint8_t* N1a,
                  const uint8_t* N1b, const uint16_t* N1s, uint8_t* N2b, uint16_t* N2s, uint8_t* N3a,
                  uint8_t* N3b, uint16_t* N3s) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      // one block row of MFMAs at a time, each beside one fragment read and
      // one sign expansion for the next substep
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (MBN >= 4) {
#pragma unroll
          for (int mb = q * MBN / 4; mb < (q + 1) * MBN / 4; ++mb) load_a1(As, s + 1, mb, a[(s + 1) & 1]);
        } else if (q < MBN) {
          load_a1(As, s + 1, q, a[(s + 1) & 1]);
        }
        mfma_row(s, q);
#pragma unroll
        for (int nb = q * NBN / 4; nb < (q + 1) * NBN / 4; ++nb) expand_b1(Bs, Ss, s + 1, nb, b[(s + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    stage_barrier<BKIND != B_BITS_ALONG_N ? NL : 8>();
    store_b(N2b, N2s);
    // substep 3, one block row at a time, with a quarter of step it+3's
    // loads issued beside each, then step it+1's first fragments
    issue(it + 3, N3a, N3b, N3s, 0);
    mfma_row(3, 0);
    __builtin_amdgcn_sched_barrier(0);
    issue(it + 3, N3a, N3b, N3s, 1);
    load_bits(N1b, N1s);
    load_a(N1a, 0, a[0]);
    mfma_row(3, 1);
    __builtin_amdgcn_sched_barrier(0);
    issue(it + 3, N3a, N3b, N3s, 2);
    mfma_row(3, 2);
    __builtin_amdgcn_sched_barrier(0);
    issue(it + 3, N3a, N3b, N3s, 3);
    mfma_row(3, 3);
    expand_b(N1b, N1s, 0, b[0]);
    __builtin_amdgcn_sched_barrier(0);
  };

  uint16_t* S0 = Sc;
  uint16_t* S1 = Sc + (BKIND != B_BITS_ALONG_K ? BK : 0);
  uint16_t* S2 = Sc + (BKIND != B_BITS_ALONG_K ? 2 * BK : 0);
  uint16_t* S3 = Sc + (BKIND != B_BITS_ALONG_K ? 3 * BK : 0);
  // prologue: stages 0 and 1 complete (bits along N written from registers),
  // step 2 issued
  issue(0, A0, B0, S0);
  if (BKIND == B_BITS_ALONG_N) {
    stage_barrier<8>();  // registers of step 0 (the 8 A loads may stay in flight)
    store_b(B0, S0);
  }
  issue(1, A1, B1, S1);
  if (BKIND == B_BITS_ALONG_N) {
    stage_barrier<8>();
    store_b(B1, S1);
  }
  issue(2, A2, B2, S2);
  stage_barrier<BKIND != B_BITS_ALONG_N ? 2 * NL : NL>();  // along K: steps 0, 1 complete; along N: step 0, 1
  load_bits(B0, S0);
  load_a(A0, 0, a[0]);
  expand_b(B0, S0, 0, b[0]);
  int it = 0;
  for (; it + 4 <= nk; it += 4) {
    step(it, A0, B0, S0, A1, B1, S1, B2, S2, A3, B3, S3);
    step(it + 1, A1, B1, S1, A2, B2, S2, B3, S3, A0, B0, S0);
    step(it + 2, A2, B2, S2, A3, B3, S3, B0, S0, A1, B1, S1);
    step(it + 3, A3, B3, S3, A0, B0, S0, B1, S1, A2, B2, S2);
  }
  if (it < nk) step(it, A0, B0, S0, A1, B1, S1, B2, S2, A3, B3, S3);
  if (it + 1 < nk) step(it + 1, A1, B1, S1, A2, B2, S2, B3, S3, A0, B0, S0);
  if (it + 2 < nk) step(it + 2, A2, B2, S2, A3, B3, S3, B0, S0, A1, B1, S1);

  // every in-flight load has landed (the stages are free for the epilogue)
  stage_barrier<0>();

  if (EPI == EPI_PARTIAL) {
    // the tile's BM x BN accumulators, row-major at p.out (32 lanes x 4
    // bytes per row per store, as the evidence epilogue)
    float* part = static_cast<float*>(p.out);
#pragma unroll
    for (int mb = 0; mb < MBN; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = WMR * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) part[lrow * BN + WNC * wn + 32 * nb + l32] = acc[mb][nb][r];
      }
    return;
  }

  if (EPI == EPI_FORWARD_F32) {
    // y = acc * scale[n] + bias[n] in fp32, stored as computed (32 lanes x 4
    // bytes per row per store)
    float* y = static_cast<float*>(p.out);
    float sc[NBN], bi[NBN];
#pragma unroll
    for (int nb = 0; nb < NBN; ++nb) {
      const int64_t col = n0 + WNC * wn + 32 * nb + l32;
      sc[nb] = (col < p.N && p.n_scale) ? p.n_scale[col] : 1.0f;
      bi[nb] = (col < p.N && p.n_bias) ? p.n_bias[col] : 0.0f;
    }
#pragma unroll
    for (int mb = 0; mb < MBN; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + WMR * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          const int64_t col = n0 + WNC * wn + 32 * nb + l32;
          float v = acc[mb][nb][r] * sc[nb];
          v = v + bi[nb];
          if (row < p.M && col < p.N) y[row * p.N + col] = v;
        }
      }
    return;
  }

  if (EPI == EPI_EVIDENCE) {
    // E0 = acc + v[m]; E = E0 * s[m] (fp32, 32 lanes x 4 bytes per row per
    // store); row partials of E0 * sign_w over this wave's columns.
    // The tile's sign_w bits (256 rows x 32 bytes), v and s go to LDS first.
    uint8_t* wst = A0;                                  // [256][32] bytes
    float* vst = reinterpret_cast<float*>(A0 + 8192);   // [256]
    float* sst = vst + BM;                              // [256]
    {
      const int64_t row = m0 + tid;
      const __amdgpu_buffer_rsrc_t rw = rsrc(p.w_bits, p.w_bits ? p.M * p.w_pb : 0);
      const uint32_t off = static_cast<uint32_t>(row * p.w_pb + n0 / 8);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint32_t w = (p.w_bits && row < p.M) ? ld32(rw, off + 4 * d) : 0u;
        *reinterpret_cast<uint32_t*>(wst + tid * 32 + 4 * d) = w;
      }
      vst[tid] = (p.m_add && row < p.M) ? p.m_add[row] : 0.0f;
      sst[tid] = (p.m_scale && row < p.M) ? p.m_scale[row] : 1.0f;
    }
    stage_barrier<0>();
    float* ev = static_cast<float*>(p.out);
#pragma unroll
    for (int mb = 0; mb < MBN; ++mb) {
      float part[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = WMR * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
        const int64_t row = m0 + lrow;
        const float add = vst[lrow], mul = sst[lrow];
        uint32_t wd[NBN];
#pragma unroll
        for (int h = 0; h < NBN; ++h) wd[h] = *reinterpret_cast<const uint32_t*>(wst + lrow * 32 + (WNC / 8) * wn + 4 * h);
        float acc_part = 0.0f;
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          const int64_t col = n0 + WNC * wn + 32 * nb + l32;
          const float e0 = acc[mb][nb][r] + add;
          // columns past N hold zero bits and contribute -e0: skip them
          if (col < p.N) acc_part += ((wd[nb] >> l32) & 1u) ? e0 : -e0;
          if (row < p.M && col < p.N) ev[row * p.N + col] = e0 * mul;
        }
        part[r] = acc_part;
      }
      if (p.gs_partial) {
        // sum part[r] over the 32 lanes of each half-wave: four halving
        // steps leave lane l one row's partial over 16 lanes, the last step
        // adds lane l ^ 1; row index bits come from lane bits 4, 3, 2, 1
#pragma unroll
        for (int o = 16, c = 16; o >= 2; o >>= 1, c >>= 1) {
          const bool hi = (l32 & o) != 0;
#pragma unroll
          for (int i = 0; i < c / 2; ++i) {
            const float keep = hi ? part[i + c / 2] : part[i];
            const float send = hi ? part[i] : part[i + c / 2];
            part[i] = keep + __shfl_xor(send, o, 64);
          }
        }
        const float tot = part[0] + __shfl_xor(part[0], 1, 64);
        const int r = 8 * ((l32 >> 4) & 1) + 4 * ((l32 >> 3) & 1) + 2 * ((l32 >> 2) & 1) + ((l32 >> 1) & 1);
        const int64_t row = m0 + WMR * wm + 32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3);
        if ((l32 & 1) == 0 && row < p.M) {
          const int64_t slot = WAVES_N * static_cast<int64_t>(tn) + wn;
          p.gs_partial[slot * p.M + row] = tot;
        }
      }
    }
    return;
  }

  // Epilogue: (scale and bias,) round to bf16 and stage through LDS EPR rows
  // at a time so each row segment of the wave's WNC outputs leaves as
  // 16-byte stores of consecutive lanes.  Waves 0, 1 stage in A0 and waves
  // 2, 3 in A1.
  uint16_t* y = static_cast<uint16_t*>(p.out);
  uint8_t* stg = (wave < 2 ? A0 : A1) + (wave & 1) * (EPR * EPL);
  float sc[NBN], bi[NBN];
#pragma unroll
  for (int nb = 0; nb < NBN; ++nb) {
    const int64_t col = n0 + WNC * wn + 32 * nb + l32;
    sc[nb] = (EPI == EPI_FORWARD && col < p.N && p.n_scale) ? p.n_scale[col] : 1.0f;
    bi[nb] = (EPI == EPI_FORWARD && col < p.N && p.n_bias) ? p.n_bias[col] : 0.0f;
  }
  // Lanes l, l^1 trade one value per row pair so each holds two adjacent
  // columns of one row: even lanes row r, odd lanes row r+1.
  const bool odd = l32 & 1;
  const bool vec_ok = (p.N & 7) == 0;
  constexpr int CPR = 2 * WNC / 16;  // 16-byte chunks per staged row
#pragma unroll
  for (int mb = 0; mb < MBN; ++mb) {
#pragma unroll
    for (int h = 0; h < 32 / EPR; ++h) {
      // rows EPR*h .. of the block row: accumulator registers (EPR/2)*h ..
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
#pragma unroll
        for (int r = (EPR / 2) * h; r < (EPR / 2) * (h + 1); r += 2) {
          float v0 = acc[mb][nb][r], v1 = acc[mb][nb][r + 1];
          if (EPI == EPI_FORWARD) {
            v0 = v0 * sc[nb];
            v0 = v0 + bi[nb];
            v1 = v1 * sc[nb];
            v1 = v1 + bi[nb];
          }
          const float send = odd ? v0 : v1;
          const float recv = __int_as_float(
              __builtin_amdgcn_update_dpp(0, __float_as_int(send), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
          const float lo = odd ? recv : v0;
          const float hi = odd ? v1 : recv;
          const uint32_t word = round16x2<DT>(lo, hi);
          const int row = 8 * (r >> 2) + 4 * kg + (r & 3) + (odd ? 1 : 0) - EPR * h;
          *reinterpret_cast<uint32_t*>(stg + row * EPL + 2 * (32 * nb + (l32 & ~1))) = word;
        }
      }
      // EPR rows x 2*WNC bytes: lane -> row (64 / CPR) i + lane / CPR, chunk lane % CPR
#pragma unroll
      for (int i = 0; i < EPR * CPR / 64; ++i) {
        const int row = (64 / CPR) * i + lane / CPR, chunk = lane % CPR;
        const uint4 v = *reinterpret_cast<const uint4*>(stg + row * EPL + 16 * chunk);
        const int64_t grow = m0 + WMR * wm + 32 * mb + EPR * h + row;
        const int64_t gcol = n0 + WNC * wn + 8 * chunk;
        if (grow < p.M) {
          if (vec_ok && gcol + 8 <= p.N) {
            // streaming (nontemporal) stores: nothing in this launch reads
            // the outputs again (0.3-3% faster per launch than plain stores)
            const u32x4 w = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(y + grow * p.N + gcol));
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
}

// sizes of the per-stage arrays for a kernel instance
template <int AKIND, int BKIND>
struct StageSizes {
  static constexpr int a = AKIND == A_ROWS_M ? A_STAGE : A_STAGE_K;
  static constexpr int b = BKIND == B_BITS_ALONG_N ? BN_STAGE : B_STAGE;
  static constexpr int s = BKIND == B_BITS_ALONG_K ? 8 : 4 * BK;
};

#define QSTE_WIDE_STAGES(ASZ, BSZ, SSZ)                           \
  __shared__ __attribute__((aligned(16))) uint8_t A0[ASZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t A1[ASZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t A2[ASZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t A3[ASZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t B0[BSZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t B1[BSZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t B2[BSZ];       \
  __shared__ __attribute__((aligned(16))) uint8_t B3[BSZ];       \
  __shared__ __attribute__((aligned(16))) uint16_t Sc[SSZ];

template <int AKIND, int BKIND, int EPI, int DT>
__global__ __launch_bounds__(THREADS, 1) void wide_kernel(Params p) {
  using SZ = StageSizes<AKIND, BKIND>;
  QSTE_WIDE_STAGES(SZ::a, SZ::b, SZ::s)
  wide_tile<AKIND, BKIND, EPI, DT>(p, blockIdx.x, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
}

// Split-K evidence, for tiles whose K chain is long against the launch:
// workgroups [0, tiles_full) compute tiles 0 .. tiles_full-1 whole; the
// remaining ns = tiles_e - tiles_full tiles are cut into `splits` K ranges
// of ks_steps K steps, workgroup tiles_full + j * ns + i covering tile
// tiles_full + i over range j and storing its bare accumulators in slab
// j * ns + i of `partial` (BM x BN fp32 each) for evidence_combine_kernel.
struct Split {
  int tiles_full, tiles_e, splits, ks_steps;
  float* partial;
};

// The evidence Params of K range j (rows of dy and of the K-indexed
// operands from k0 = j * ks_steps * BK on); bits along N are rows of K,
// bits along K (scaled) a transposed copy whose bit k0 starts byte k0 / 8.
template <int BKIND>
__device__ __forceinline__ Params range_params(const Params& p, int j, int ks_steps) {
  const int64_t k0 = static_cast<int64_t>(j) * ks_steps * BK;
  Params q = p;
  q.a = p.a + k0 * p.lda;  // A as rows of K
  q.a_rows = p.a_rows - k0;
  if (BKIND == B_BITS_ALONG_N) {
    q.bits = p.bits + k0 * p.pb;
    q.bit_rows = p.bit_rows - k0;
    q.kscale = p.kscale ? p.kscale + k0 : nullptr;
  } else {
    q.bits = p.bits + k0 / 8;  // k0 % 64 == 0
    q.kscale16 = p.kscale16 + k0;
  }
  const int64_t left = p.K - k0, span = static_cast<int64_t>(ks_steps) * BK;
  q.K = left < span ? left : span;  // the host makes every range nonempty
  return q;
}

// Workgroup e >= tiles_full of a split evidence grid: one K range of one tile.
template <int BKIND, int DT>
__device__ __forceinline__ void evidence_range(const Params& p, const Split& sp, int e, uint8_t* A0, uint8_t* A1,
                                               uint8_t* A2, uint8_t* A3, uint8_t* B0, uint8_t* B1, uint8_t* B2,
                                               uint8_t* B3, uint16_t* Sc) {
  const int ns = sp.tiles_e - sp.tiles_full, r = e - sp.tiles_full;
  const int j = r / ns, i = r - j * ns;
  Params q = range_params<BKIND>(p, j, sp.ks_steps);
  q.out = sp.partial + (static_cast<int64_t>(j) * ns + i) * (BM * BN);
  wide_tile<A_ROWS_K, BKIND, EPI_PARTIAL, DT>(q, sp.tiles_full + i, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
}

// The evidence alone (A = dy^T as stored; the signs of x as stored, bits
// along N with the fp32 per-k scale, or a transposed copy, bits along K with
// bf16 per-k scales), some tiles split over K.
template <int BKIND, int DT>
__global__ __launch_bounds__(THREADS, 1) void evidence_split_kernel(Params p, Split sp) {
  using SZ = StageSizes<A_ROWS_K, BKIND>;
  QSTE_WIDE_STAGES(SZ::a, SZ::b, SZ::s)
  const int e = static_cast<int>(blockIdx.x);
  if (e < sp.tiles_full)
    wide_tile<A_ROWS_K, BKIND, EPI_EVIDENCE, DT>(p, e, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
  else
    evidence_range<BKIND, DT>(p, sp, e, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
}

// The two large products of a layer's backward in one launch: evidence
// tiles first (the longer ones), then dgrad tiles, so the grid's last wave
// of one product is filled by the other instead of leaving CUs idle.  Both
// take their signs as transposed copies (bits along K) with bf16 per-k
// scales, prepared by the caller.  SPLIT: every evidence tile is split
// (tiles_full == 0): tiles_e * splits range workgroups, then dgrad.
template <int DT, bool SPLIT>
__global__ __launch_bounds__(THREADS, 1) void backward_pair_kernel(Params pe, Params pd, Split sp) {
  QSTE_WIDE_STAGES(A_STAGE_K, B_STAGE, 4 * BK)
  const int e = static_cast<int>(blockIdx.x);
  if (!SPLIT) {
    if (e < sp.tiles_e)
      wide_tile<A_ROWS_K, B_BITS_ALONG_K_SCALED, EPI_EVIDENCE, DT>(pe, e, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
    else
      wide_tile<A_ROWS_M, B_BITS_ALONG_K_SCALED, EPI_PLAIN, DT>(pd, e - sp.tiles_e, A0, A1, A2, A3, B0, B1, B2, B3,
                                                                Sc);
  } else {
    const int ge = sp.tiles_e * sp.splits;
    if (e < ge)
      evidence_range<B_BITS_ALONG_K_SCALED, DT>(pe, sp, e, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
    else
      wide_tile<A_ROWS_M, B_BITS_ALONG_K_SCALED, EPI_PLAIN, DT>(pd, e - ge, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
  }
}

// The evidence epilogue of the split tiles: E0 = the tile's range partials
// summed in range order + m_add[m]; E = E0 * m_scale[m]; and the
// scale-gradient partials sum_c E0 * sign_w over each 64-column slot, in
// the slots the fused epilogue writes ([WAVES_N * tiles_n][M]).  One wave
// per tile row (4 columns per lane, 16-byte accesses; N % 64 == 0 on this
// path), a 16-lane group per slot; workgroups of 4 rows x split tiles.
__global__ __launch_bounds__(THREADS) void evidence_combine_kernel(Split sp, const float* __restrict__ m_add,
                                                                   const float* __restrict__ m_scale,
                                                                   const uint8_t* __restrict__ w_bits, int64_t w_pb,
                                                                   float* __restrict__ ev,
                                                                   float* __restrict__ gs_partial, int64_t M,
                                                                   int64_t N) {
  constexpr int ROWS = THREADS / kWave;
  const int tiles_m = static_cast<int>((M + BM - 1) / BM), tiles_n = static_cast<int>((N + BN - 1) / BN);
  const int ns = sp.tiles_e - sp.tiles_full, i = static_cast<int>(blockIdx.y);
  int tm, tn;
  tile_of<1>(sp.tiles_full + i, tiles_m, tiles_n, tm, tn);  // the evidence's mapping
  const int lane = threadIdx.x % kWave;
  const int lrow = static_cast<int>(blockIdx.x) * ROWS + static_cast<int>(threadIdx.x) / kWave;
  const int64_t row = static_cast<int64_t>(tm) * BM + lrow;
  if (row >= M) return;  // the whole wave
  const int64_t col = static_cast<int64_t>(tn) * BN + 4 * lane;
  float signed_e0 = 0.0f;
  if (col < N) {
    const int64_t at = static_cast<int64_t>(i) * (BM * BN) + static_cast<int64_t>(lrow) * BN + 4 * lane;
    float4 acc = *reinterpret_cast<const float4*>(sp.partial + at);
    for (int j = 1; j < sp.splits; ++j) {
      const float4 v = *reinterpret_cast<const float4*>(sp.partial + static_cast<int64_t>(j) * ns * (BM * BN) + at);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    const float add = m_add ? m_add[row] : 0.0f, mul = m_scale ? m_scale[row] : 1.0f;
    const float e0[4] = {acc.x + add, acc.y + add, acc.z + add, acc.w + add};
    *reinterpret_cast<float4*>(ev + row * N + col) = make_float4(e0[0] * mul, e0[1] * mul, e0[2] * mul, e0[3] * mul);
    if (w_bits) {
      const uint32_t nib = (w_bits[row * w_pb + (col >> 3)] >> (col & 7)) & 0xFu;
#pragma unroll
      for (int q = 0; q < 4; ++q) signed_e0 += ((nib >> q) & 1u) ? e0[q] : -e0[q];
    }
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) signed_e0 += __shfl_xor(signed_e0, o, kWave);
  if (gs_partial && lane % 16 == 0) gs_partial[(static_cast<int64_t>(tn) * WAVES_N + lane / 16) * M + row] = signed_e0;
}
// Split-K forward for products with few output tiles and a long K chain
// (fp32 limbs at small M): workgroup w covers tile w % tiles over K range
// w / tiles (ks_steps K steps) and stores its bare accumulators in slab w of
// `partial` (BM x BN fp32 each) for forward_combine_kernel.
template <int DT>
__global__ __launch_bounds__(THREADS, 1) void forward_split_kernel(Params p, int tiles, int ks_steps,
                                                                   float* partial) {
  using SZ = StageSizes<A_ROWS_M, B_BITS_ALONG_K>;
  QSTE_WIDE_STAGES(SZ::a, SZ::b, SZ::s)
  const int w = static_cast<int>(blockIdx.x), i = w % tiles, j = w / tiles;
  const int64_t k0 = static_cast<int64_t>(j) * ks_steps * BK;
  Params q = p;
  q.a = p.a + k0;          // columns k0 .. of every dense row (lda unchanged)
  q.bits = p.bits + k0 / 8;  // bits k0 .. of every packed row (pb unchanged)
  q.K = p.K - k0 < static_cast<int64_t>(ks_steps) * BK ? p.K - k0 : static_cast<int64_t>(ks_steps) * BK;
  q.out = partial + static_cast<int64_t>(w) * (BM * BN);
  wide_tile<A_ROWS_M, B_BITS_ALONG_K, EPI_PARTIAL, DT>(q, i, A0, A1, A2, A3, B0, B1, B2, B3, Sc);
}

// y = (the K ranges' accumulators summed in range order) * scale[n] +
// bias[n], as the forward epilogues finish an unsplit tile: stored as fp32
// (OUT = QSTE_F32) or rounded once to bf16 / fp16.  Workgroup (x, i): rows
// 4x .. 4x + 3 of tile i, a wave per row, 4 columns per lane.
template <int OUT>
__global__ __launch_bounds__(THREADS) void forward_combine_kernel(const float* __restrict__ partial, int tiles,
                                                                  int splits, const float* __restrict__ n_scale,
                                                                  const float* __restrict__ n_bias,
                                                                  void* __restrict__ out, int64_t M, int64_t N) {
  const int tiles_m = static_cast<int>((M + BM - 1) / BM), tiles_n = static_cast<int>((N + BN - 1) / BN);
  const int i = static_cast<int>(blockIdx.y);
  int tm, tn;
  tile_of<2>(i, tiles_m, tiles_n, tm, tn);  // the forward's mapping
  const int lrow = static_cast<int>(blockIdx.x) * (THREADS / kWave) + static_cast<int>(threadIdx.x) / kWave;
  const int lcol = 4 * (static_cast<int>(threadIdx.x) % kWave);
  const int64_t row = static_cast<int64_t>(tm) * BM + lrow;
  if (row >= M) return;  // the whole wave
  const float* src = partial + static_cast<int64_t>(i) * (BM * BN) + lrow * BN + lcol;
  float4 acc = *reinterpret_cast<const float4*>(src);
  for (int j = 1; j < splits; ++j) {
    const float4 v = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(j) * tiles * (BM * BN));
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const float a[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t col = static_cast<int64_t>(tn) * BN + lcol + q;
    if (col < N) {
      float v = a[q] * (n_scale ? n_scale[col] : 1.0f);
      v = v + (n_bias ? n_bias[col] : 0.0f);
      if constexpr (OUT == QSTE_F32)
        static_cast<float*>(out)[row * N + col] = v;
      else
        static_cast<uint16_t*>(out)[row * N + col] = round16<OUT>(v);
    }
  }
}
#undef QSTE_WIDE_STAGES
}  // namespace wide
}  // namespace mfma

// ---------------------------------------------------------------------------
// dispatch: returns 1 when the call is not for this path
// ---------------------------------------------------------------------------

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// bf16 and fp16 take the MFMA path (fp32 stays on the fp32 SIMT kernel)
static bool mfma_dtype(int dtype) { return dtype == QSTE_BF16 || dtype == QSTE_F16; }

// Buffer offsets are 32-bit: every operand must stay under 4 GiB.
static bool fits32(int64_t bytes) { return bytes < (int64_t{1} << 32); }

static int wide_grid(int64_t M, int64_t N) {
  return static_cast<int>(((M + mfma::wide::BM - 1) / mfma::wide::BM) * ((N + mfma::wide::BN - 1) / mfma::wide::BN));
}

static bool forward_ok(const void* x, int dtype, const uint8_t* packed, int64_t m, int64_t rows, int64_t cols) {
  return mfma_dtype(dtype) && cols % 64 == 0 && cols > 0 && m > 0 && rows > 0 && aligned16(x) &&
         aligned16(packed) && fits32(m * cols * 2) && fits32(rows * cols / 8);
}
static bool dgrad_ok(const void* dy, int dtype, const uint8_t* packed, int64_t m, int64_t rows, int64_t cols) {
  return mfma_dtype(dtype) && cols % 64 == 0 && rows % 64 == 0 && rows > 0 && cols > 0 && m > 0 &&
         aligned16(dy) && aligned16(packed) && fits32(m * rows * 2) && fits32(rows * cols / 8);
}
static bool evidence_ok(const void* dy, int dtype, const uint8_t* packed_x, int64_t samples, int64_t rows,
                        int64_t cols) {
  return mfma_dtype(dtype) && cols % 64 == 0 && rows % 64 == 0 && rows > 0 && cols > 0 && samples > 0 &&
         aligned16(dy) && aligned16(packed_x) && fits32(samples * rows * 2) && fits32(samples * cols / 8);
}

static mfma::Params dgrad_params(const void* dy, const uint8_t* packed, const float* row_scale, void* dx,
                                 int64_t m, int64_t rows, int64_t cols) {
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = packed;
  p.kscale = row_scale;
  p.out = dx;
  p.M = m; p.N = cols; p.K = rows;
  p.lda = rows; p.pb = cols / 8;
  p.a_rows = m; p.bit_rows = rows;
  return p;
}

static mfma::Params evidence_params(const void* dy, const uint8_t* packed_x, const float* x_scale, float* ev,
                                    int64_t samples, int64_t rows, int64_t cols, const float* m_add,
                                    const float* m_scale, const uint8_t* w_bits, float* gs_partial) {
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = packed_x;
  p.kscale = x_scale;
  p.out = ev;
  p.M = rows; p.N = cols; p.K = samples;
  p.lda = rows; p.pb = cols / 8;
  p.a_rows = samples; p.bit_rows = samples;
  p.m_add = m_add; p.m_scale = m_scale; p.w_bits = w_bits; p.w_pb = cols / 8; p.gs_partial = gs_partial;
  return p;
}

// The combine pass of a split evidence: workgroups of 4 tile rows x split tiles.
static int launch_combine(const mfma::wide::Split& sp, const float* m_add, const float* m_scale,
                          const uint8_t* w_bits, float* ev, float* gs_partial, int64_t rows, int64_t cols,
                          hipStream_t stream) {
  const dim3 grid(mfma::wide::BM / (mfma::wide::THREADS / kWave), static_cast<unsigned>(sp.tiles_e - sp.tiles_full));
  mfma::wide::evidence_combine_kernel<<<grid, mfma::wide::THREADS, 0, stream>>>(sp, m_add, m_scale, w_bits, cols / 8,
                                                                               ev, gs_partial, rows, cols);
  return static_cast<int>(hipGetLastError());
}

int mfma_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  if (!forward_ok(x, dtype, packed, m, rows, cols)) return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(x);
  p.bits = packed;
  p.out = y;
  p.M = m; p.N = rows; p.K = cols;
  p.lda = cols; p.pb = cols / 8;
  p.a_rows = m; p.bit_rows = rows;
  p.n_scale = scale; p.n_bias = bias;
  if (dtype == QSTE_F16)
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_K, mfma::EPI_FORWARD, QSTE_F16>
        <<<wide_grid(m, rows), mfma::wide::THREADS, 0, stream>>>(p);
  else
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_K, mfma::EPI_FORWARD, QSTE_BF16>
        <<<wide_grid(m, rows), mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

// K ranges of a forward with `tiles` output tiles and nk K steps: a product
// with fewer tiles than half the device's 256 CUs and a long K chain is cut
// into up to 16 ranges of at least 4 K steps (one round of workgroups),
// else 1.
struct SplitK {
  int splits, ks_steps;
};
static SplitK forward_split_plan(int tiles, int nk) {
  int s = 1;
  if (tiles > 0 && 2 * tiles <= 256 && nk >= 16) {
    s = 16;
    if (s > 256 / tiles) s = 256 / tiles;
    if (s > nk / 4) s = nk / 4;
  }
  if (s < 2) return {1, nk};
  const int ks = (nk + s - 1) / s;
  return {(nk + ks - 1) / ks, ks};
}
// The 16-bit forward with few output tiles (M past the decode GEMV's 16, a
// round of 256-row tiles or less) over a long K: K ranges as for the fp32
// limbs, their accumulators in a caller workspace, then scale, bias and one
// rounding.  Workspace bytes, 0 where no split pays.
size_t mfma_forward_split_workspace(int64_t m, int64_t rows, int64_t cols, int dtype) {
  if (!mfma_dtype(dtype) || m <= 16 || rows <= 0 || cols <= 0 || cols % 64 != 0) return 0;
  const int tiles = wide_grid(m, rows);
  const SplitK sp = forward_split_plan(tiles, static_cast<int>(cols / mfma::wide::BK));
  return sp.splits > 1 ? static_cast<size_t>(sp.splits) * tiles * mfma::wide::BM * mfma::wide::BN * sizeof(float)
                       : 0;
}

// Returns 1 when the call is not for this path (shape, or too little workspace).
int mfma_linear_forward_split(const void* x, int dtype, const uint8_t* packed, const float* scale,
                              const float* bias, void* y, int64_t m, int64_t rows, int64_t cols, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  const size_t need = mfma_forward_split_workspace(m, rows, cols, dtype);
  if (need == 0 || !workspace || workspace_bytes < need || !forward_ok(x, dtype, packed, m, rows, cols) ||
      !aligned16(workspace))
    return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(x);
  p.bits = packed;
  p.M = m; p.N = rows; p.K = cols;
  p.lda = cols; p.pb = cols / 8;
  p.a_rows = m; p.bit_rows = rows;
  const int tiles = wide_grid(m, rows);
  const SplitK sp = forward_split_plan(tiles, static_cast<int>(cols / mfma::wide::BK));
  float* partial = static_cast<float*>(workspace);
  if (dtype == QSTE_F16)
    mfma::wide::forward_split_kernel<QSTE_F16>
        <<<tiles * sp.splits, mfma::wide::THREADS, 0, stream>>>(p, tiles, sp.ks_steps, partial);
  else
    mfma::wide::forward_split_kernel<QSTE_BF16>
        <<<tiles * sp.splits, mfma::wide::THREADS, 0, stream>>>(p, tiles, sp.ks_steps, partial);
  int rc = static_cast<int>(hipGetLastError());
  if (rc) return rc;
  const dim3 grid(mfma::wide::BM / (mfma::wide::THREADS / kWave), static_cast<unsigned>(tiles));
  if (dtype == QSTE_F16)
    mfma::wide::forward_combine_kernel<QSTE_F16>
        <<<grid, mfma::wide::THREADS, 0, stream>>>(partial, tiles, sp.splits, scale, bias, y, m, rows);
  else
    mfma::wide::forward_combine_kernel<QSTE_BF16>
        <<<grid, mfma::wide::THREADS, 0, stream>>>(partial, tiles, sp.splits, scale, bias, y, m, rows);
  return static_cast<int>(hipGetLastError());
}

int mfma_linear_dgrad(const void* dy, int dtype, const uint8_t* packed, const float* row_scale, void* dx,
                      int64_t m, int64_t rows, int64_t cols, hipStream_t stream) {
  if (!dgrad_ok(dy, dtype, packed, m, rows, cols)) return 1;
  const mfma::Params p = dgrad_params(dy, packed, row_scale, dx, m, rows, cols);
  if (dtype == QSTE_F16)
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_N, mfma::EPI_PLAIN, QSTE_F16>
        <<<wide_grid(m, cols), mfma::wide::THREADS, 0, stream>>>(p);
  else
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_N, mfma::EPI_PLAIN, QSTE_BF16>
        <<<wide_grid(m, cols), mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

// dgrad from a transposed copy of the signs (w_t [cols][w_t_pitch], bit r of
// row c = sign of W[r][c], zero past rows) and the bf16 row scales (zero
// padded to a multiple of 64): the bits run along K, so a lane's 8 k-values
// are one byte and each expansion is one shift-and-OR per pair, as in the
// forward.  Measured 6-10% faster than bits along N at config 4's shapes;
// the results are identical (the same bf16 operand values, the same
// accumulation order).
int mfma_linear_dgrad_t(const void* dy, int dtype, const uint8_t* w_t, int64_t w_t_pitch, const uint16_t* scale16,
                        void* dx, int64_t m, int64_t rows, int64_t cols, hipStream_t stream) {
  if (!dgrad_ok(dy, dtype, w_t, m, rows, cols) || !fits32(cols * w_t_pitch) || !aligned16(w_t)) return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = w_t;
  p.kscale16 = scale16;
  p.out = dx;
  p.M = m; p.N = cols; p.K = rows;
  p.lda = rows; p.pb = w_t_pitch;
  p.a_rows = m; p.bit_rows = cols;
  if (dtype == QSTE_F16)
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_K_SCALED, mfma::EPI_PLAIN, QSTE_F16>
        <<<wide_grid(m, cols), mfma::wide::THREADS, 0, stream>>>(p);
  else
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_K_SCALED, mfma::EPI_PLAIN, QSTE_BF16>
        <<<wide_grid(m, cols), mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

int64_t mfma_evidence_tiles(int64_t cols) { return mfma::wide::WAVES_N * ((cols + mfma::wide::BN - 1) / mfma::wide::BN); }

int mfma_evidence(const void* dy, int dtype, const uint8_t* packed_x, const float* x_scale, float* ev,
                  int64_t samples, int64_t rows, int64_t cols, const float* m_add, const float* m_scale,
                  const uint8_t* w_bits, float* gs_partial, const EvidencePlan* plan, float* partial,
                  hipStream_t stream) {
  if (!evidence_ok(dy, dtype, packed_x, samples, rows, cols)) return 1;
  const mfma::Params p =
      evidence_params(dy, packed_x, x_scale, ev, samples, rows, cols, m_add, m_scale, w_bits, gs_partial);
  const int te = wide_grid(rows, cols);
  if (plan && plan->splits > 1 && aligned16(ev)) {  // the combine pass stores 16 bytes at a time
    if (!partial) return QSTE_E_WORKSPACE;
    const mfma::wide::Split sp{plan->tiles_full, te, plan->splits, plan->ks_steps, partial};
    const int grid = sp.tiles_full + (te - sp.tiles_full) * sp.splits;
    if (dtype == QSTE_F16)
      mfma::wide::evidence_split_kernel<mfma::B_BITS_ALONG_N, QSTE_F16><<<grid, mfma::wide::THREADS, 0, stream>>>(p, sp);
    else
      mfma::wide::evidence_split_kernel<mfma::B_BITS_ALONG_N, QSTE_BF16><<<grid, mfma::wide::THREADS, 0, stream>>>(p, sp);
    int rc = static_cast<int>(hipGetLastError());
    if (rc) return rc;
    return launch_combine(sp, m_add, m_scale, w_bits, ev, gs_partial, rows, cols, stream);
  }
  if (dtype == QSTE_F16)
    mfma::wide::wide_kernel<mfma::A_ROWS_K, mfma::B_BITS_ALONG_N, mfma::EPI_EVIDENCE, QSTE_F16>
        <<<te, mfma::wide::THREADS, 0, stream>>>(p);
  else
    mfma::wide::wide_kernel<mfma::A_ROWS_K, mfma::B_BITS_ALONG_N, mfma::EPI_EVIDENCE, QSTE_BF16>
        <<<te, mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

// The evidence alone from a transposed copy of x's signs (x_t [cols]
// [x_t_pitch], bit k of row c = sign of x[k][c], zero past samples) and its
// scale as bf16 (zero padded to a multiple of 64): bits along K, so a lane's
// 8 k-values are one byte, direct loads bring them, and no wave stages them
// through registers, as the backward pair reads them.  The same operand
// values and K order as mfma_evidence: the results are identical.  Measured
// ~2% faster than bits along N at config 4's gate and up evidence, the
// transposes included.
int mfma_evidence_t(const void* dy, int dtype, const uint8_t* x_t, int64_t x_t_pitch, const uint16_t* x_scale16,
                    float* ev, int64_t samples, int64_t rows, int64_t cols, const float* m_add, const float* m_scale,
                    const uint8_t* w_bits, float* gs_partial, const EvidencePlan* plan, float* partial,
                    hipStream_t stream) {
  if (!evidence_ok(dy, dtype, x_t, samples, rows, cols) || !fits32(cols * x_t_pitch) || !aligned16(x_t)) return 1;
  mfma::Params p{};
  p.a = static_cast<const uint16_t*>(dy);
  p.bits = x_t;
  p.kscale16 = x_scale16;
  p.out = ev;
  p.M = rows; p.N = cols; p.K = samples;
  p.lda = rows; p.pb = x_t_pitch;
  p.a_rows = samples; p.bit_rows = cols;
  p.m_add = m_add; p.m_scale = m_scale; p.w_bits = w_bits; p.w_pb = cols / 8; p.gs_partial = gs_partial;
  const int te = wide_grid(rows, cols);
  if (plan && plan->splits > 1 && aligned16(ev)) {  // the combine pass stores 16 bytes at a time
    if (!partial) return QSTE_E_WORKSPACE;
    const mfma::wide::Split sp{plan->tiles_full, te, plan->splits, plan->ks_steps, partial};
    const int grid = sp.tiles_full + (te - sp.tiles_full) * sp.splits;
    if (dtype == QSTE_F16)
      mfma::wide::evidence_split_kernel<mfma::B_BITS_ALONG_K_SCALED, QSTE_F16>
          <<<grid, mfma::wide::THREADS, 0, stream>>>(p, sp);
    else
      mfma::wide::evidence_split_kernel<mfma::B_BITS_ALONG_K_SCALED, QSTE_BF16>
          <<<grid, mfma::wide::THREADS, 0, stream>>>(p, sp);
    int rc = static_cast<int>(hipGetLastError());
    if (rc) return rc;
    return launch_combine(sp, m_add, m_scale, w_bits, ev, gs_partial, rows, cols, stream);
  }
  if (dtype == QSTE_F16)
    mfma::wide::wide_kernel<mfma::A_ROWS_K, mfma::B_BITS_ALONG_K_SCALED, mfma::EPI_EVIDENCE, QSTE_F16>
        <<<te, mfma::wide::THREADS, 0, stream>>>(p);
  else
    mfma::wide::wide_kernel<mfma::A_ROWS_K, mfma::B_BITS_ALONG_K_SCALED, mfma::EPI_EVIDENCE, QSTE_BF16>
        <<<te, mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

// Whether mfma_backward_pair takes a call (workspace copies are 256-byte
// aligned, so only the caller's operands are checked here).
bool mfma_pair_ok(const void* dy, int dtype, int64_t samples, int64_t rows, int64_t cols) {
  return mfma_dtype(dtype) && cols % 64 == 0 && rows % 64 == 0 && rows > 0 && cols > 0 && samples > 0 &&
         aligned16(dy) && fits32(samples * rows * 2) && fits32(samples * cols / 8) && fits32(rows * cols / 8);
}

// ---------------------------------------------------------------------------
// evidence plan: one launch or two, and which tiles split over K
// ---------------------------------------------------------------------------
// The evidence's K is the token count, usually its longest dimension, and
// its tile count rows/256 x cols/256 can be small against the CU count (64
// tiles at 4096 x 1024) or leave a partial last round (896 = 3.5 x 256 at
// config 4): then long serial tile chains set the launch's length while
// CUs idle.  The plan cuts the last tiles (or all of them) into S = 2, 4 or
// 8 K ranges when that shortens the work, and runs dgrad either in the same
// launch (the backward pair, which fills the evidence's idle CUs) or as a
// second launch (its per-step speed is ~8% higher: measured at config 4's
// shapes).  The choice minimises an estimate: list
// scheduling of the tiles on kCUs CUs, in K steps, each tile costing
// kTileOverhead steps more for its prologue and epilogue, plus the combine
// pass's HBM traffic in step units.  It depends only on the shape, so the
// workspace query and the call agree.
namespace {
constexpr int64_t kCUs = 256;              // MI350X / MI355X
constexpr int64_t kTileOverhead = 14;      // K steps a tile's prologue + epilogue cost
constexpr double kBytesPerStep = 7.5e6;    // combine traffic per K-step time (~5 TB/s x 1.5 us)
constexpr double kPairFactor = 1.08;       // the pair's K steps are this much slower
constexpr int64_t kMaxPartialBytes = int64_t{1} << 30;
constexpr int64_t kTileBytes = int64_t{mfma::wide::BM} * mfma::wide::BN * 4;

// Greedy in-order assignment of `n` groups of (count, length) items onto
// kCUs CUs that start idle; returns the finish time of the last CU.
int64_t list_schedule(const int64_t (*groups)[2], int n) {
  std::map<int64_t, int64_t> free_at{{0, kCUs}};  // time -> CUs idle from then
  for (int g = 0; g < n; ++g) {
    int64_t left = groups[g][0];
    const int64_t len = groups[g][1];
    while (left > 0) {
      auto it = free_at.begin();
      const int64_t t = it->first, c = it->second;
      const int64_t take = left < c ? left : c;
      if (take == c) free_at.erase(it);
      else it->second = c - take;
      free_at[t + len] += take;
      left -= take;
    }
  }
  return free_at.rbegin()->first;
}
}  // namespace

static EvidencePlan compute_plan(int64_t samples, int64_t rows, int64_t cols, bool with_dgrad) {
  const int64_t nk = (samples + mfma::wide::BK - 1) / mfma::wide::BK;
  const int64_t te = wide_grid(rows, cols), td = with_dgrad ? wide_grid(samples, cols) : 0;
  const int64_t nkd = (rows + mfma::wide::BK - 1) / mfma::wide::BK;
  EvidencePlan best{0, static_cast<int>(te), 1, static_cast<int>(nk), 0};
  if (samples <= 0 || rows <= 0 || cols <= 0) return best;
  const int64_t dgrad[1][2] = {{td, nkd + kTileOverhead}};
  const double dgrad_alone = td ? static_cast<double>(list_schedule(dgrad, 1)) : 0.0;
  double best_cost = -1.0;
  for (int S = 1; S <= 8; S *= 2) {
    const int64_t ks = (nk + S - 1) / S;
    if (S > 1 && ks < 16) break;  // ranges shorter than 16 K steps are mostly overhead
    const int64_t splits = (nk + ks - 1) / ks;  // every range nonempty
    // whole tiles: all (no split), or all of the full rounds, or one round fewer, or none
    int64_t fulls[3] = {te, -1, -1};
    if (S > 1) {
      const int64_t rounds = te / kCUs * kCUs;
      fulls[0] = 0;
      fulls[1] = rounds < te && rounds > 0 ? rounds : -1;
      fulls[2] = rounds - kCUs > 0 && rounds < te ? rounds - kCUs : -1;
    }
    for (int64_t F : fulls) {
      if (F < 0) continue;
      const int64_t ns = te - F;
      const int64_t partial = S > 1 ? splits * ns * kTileBytes : 0;
      if (partial > kMaxPartialBytes) continue;
      const double combine = S > 1 ? static_cast<double>((splits + 1) * ns * kTileBytes) / kBytesPerStep + 2.0 : 0.0;
      const int64_t groups[3][2] = {{S > 1 ? F : te, nk + kTileOverhead},
                                    {S > 1 ? ns * splits : 0, ks + kTileOverhead},
                                    {td, nkd + kTileOverhead}};
      // the pair launch splits all of its evidence tiles or none
      for (int pair = 0; pair <= (td > 0 && (S == 1 || F == 0) ? 1 : 0); ++pair) {
        const double cost = pair ? static_cast<double>(list_schedule(groups, 3)) * kPairFactor + combine
                                 : static_cast<double>(list_schedule(groups, 2)) + combine + dgrad_alone;
        if (best_cost < 0.0 || cost < best_cost) {
          best_cost = cost;
          best = EvidencePlan{pair, static_cast<int>(S > 1 ? F : te), static_cast<int>(splits),
                              static_cast<int>(ks), partial};
        }
      }
    }
  }
  return best;
}

// Plans are looked up per shape (every training step asks for the same few
// shapes, each several times per layer).
EvidencePlan mfma_evidence_plan(int64_t samples, int64_t rows, int64_t cols, bool with_dgrad) {
  struct Entry {
    int64_t samples, rows, cols;
    bool with_dgrad;
    EvidencePlan plan;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry& e : cache)
    if (e.samples == samples && e.rows == rows && e.cols == cols && e.with_dgrad == with_dgrad) return e.plan;
  const EvidencePlan plan = compute_plan(samples, rows, cols, with_dgrad);
  if (cache.size() >= 256) cache.erase(cache.begin());
  cache.push_back(Entry{samples, rows, cols, with_dgrad, plan});
  return plan;
}

// Evidence (with its fused epilogue) and dgrad of one layer in one launch,
// from transposed sign copies: x_t [cols][x_t_pitch] (bit k of row c = sign
// of x[k][c]) and w_t [cols][w_t_pitch] (bit r of row c = sign of W[r][c]),
// both zero past their K, and bf16 copies of x_scale and scale, zero-padded
// to a multiple of 64 entries.  `plan` is mfma_evidence_plan's for the
// shape (with pair set); its split tiles need plan.partial_bytes at
// `partial`.  Returns 1 when either product is not for this path.
int mfma_backward_pair(const void* dy, int dtype, const uint8_t* x_t, int64_t x_t_pitch, const uint16_t* x_scale16,
                       float* ev, const uint8_t* w_t, int64_t w_t_pitch, const uint16_t* scale16,
                       const uint8_t* packed_w, void* dx, int64_t samples, int64_t rows, int64_t cols,
                       const float* m_add, const float* scale, float* gs_partial, const EvidencePlan& plan,
                       float* partial, hipStream_t stream) {
  if (!evidence_ok(dy, dtype, x_t, samples, rows, cols) || !fits32(cols * x_t_pitch) || !dx ||
      !dgrad_ok(dy, dtype, w_t, samples, rows, cols) || !fits32(cols * w_t_pitch))
    return 1;
  if (plan.splits > 1 && !partial) return QSTE_E_WORKSPACE;
  mfma::Params pe{};
  pe.a = static_cast<const uint16_t*>(dy);
  pe.bits = x_t;
  pe.kscale16 = x_scale16;
  pe.out = ev;
  pe.M = rows; pe.N = cols; pe.K = samples;
  pe.lda = rows; pe.pb = x_t_pitch;
  pe.a_rows = samples; pe.bit_rows = cols;
  pe.m_add = m_add; pe.m_scale = scale; pe.w_bits = packed_w; pe.w_pb = cols / 8; pe.gs_partial = gs_partial;
  mfma::Params pd{};
  pd.a = static_cast<const uint16_t*>(dy);
  pd.bits = w_t;
  pd.kscale16 = scale16;
  pd.out = dx;
  pd.M = samples; pd.N = cols; pd.K = rows;
  pd.lda = rows; pd.pb = w_t_pitch;
  pd.a_rows = samples; pd.bit_rows = cols;
  const int te = wide_grid(rows, cols), td = wide_grid(samples, cols);
  const bool split = plan.splits > 1 && aligned16(ev);  // the combine pass stores 16 bytes at a time
  const mfma::wide::Split sp{split ? plan.tiles_full : te, te, split ? plan.splits : 1, plan.ks_steps,
                             split ? partial : nullptr};
  const dim3 g(sp.tiles_full + (te - sp.tiles_full) * sp.splits + td), b(mfma::wide::THREADS);
  if (dtype == QSTE_F16) {
    if (split) mfma::wide::backward_pair_kernel<QSTE_F16, true><<<g, b, 0, stream>>>(pe, pd, sp);
    else mfma::wide::backward_pair_kernel<QSTE_F16, false><<<g, b, 0, stream>>>(pe, pd, sp);
  } else {
    if (split) mfma::wide::backward_pair_kernel<QSTE_BF16, true><<<g, b, 0, stream>>>(pe, pd, sp);
    else mfma::wide::backward_pair_kernel<QSTE_BF16, false><<<g, b, 0, stream>>>(pe, pd, sp);
  }
  int rc = static_cast<int>(hipGetLastError());
  if (rc || !split) return rc;
  return launch_combine(sp, m_add, scale, packed_w, ev, gs_partial, rows, cols, stream);
}

// ---------------------------------------------------------------------------
// fp32 products on the bf16 MFMA path.  An fp32 value v splits exactly into
// three bf16 limbs: hi = bf16(v), mid = bf16(v - hi), lo = bf16(v - hi - mid)
// (each difference is exact in fp32; v - hi has at most 16 significant
// bits and v - hi - mid at most 8, so lo holds it exactly; only values whose
// last limb falls below bf16's subnormals lose it).  A limb times +-1 is
// exact, so a product over K becomes the same bf16 MFMA product over 3K --
// the dense operand's three limbs along K against the signs repeated three
// times -- with every product exact and the sums in the MFMA's fp32
// accumulators.  Per-k scales (the row scale of dX, the sample scale of
// the evidence) are multiplied into the fp32 operand first, one fp32
// rounding each, where the reference's fp32 GEMM rounds the product inside
// its fused multiply-add.
// ---------------------------------------------------------------------------

namespace limbs {

// out[plane * p + r * ld + c] for the three limbs p of x[r, c] (times
// row_mul[r] or col_mul[c] when given)
__global__ __launch_bounds__(256) void split_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                    const float* __restrict__ row_mul,
                                                    const float* __restrict__ col_mul, uint16_t* __restrict__ out,
                                                    int64_t ld, int64_t plane) {
  const int64_t n = rows * cols;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / cols, c = i - r * cols;
    float v = x[i];
    if (row_mul) v = v * row_mul[r];
    if (col_mul) v = v * col_mul[c];
    uint16_t hi = f32_to_bf16(v);
    const bool finite = __builtin_isfinite(v);
    // a finite value that rounds past bf16's largest finite one keeps its
    // top 16 bits instead (truncation: the residual is exact as well); an
    // infinite or NaN value is carried by hi alone, its other limbs zero,
    // so the products see the same inf or NaN the fp32 operand holds
    if (finite && (hi & 0x7F80u) == 0x7F80u) hi = static_cast<uint16_t>(__float_as_uint(v) >> 16);
    const float r1 = finite ? v - bf16_to_f32(hi) : 0.0f;
    const uint16_t mid = f32_to_bf16(r1);
    const float r2 = r1 - bf16_to_f32(mid);
    const uint16_t lo = f32_to_bf16(r2);
    uint16_t* o = out + r * ld + c;
    o[0] = hi;
    o[plane] = mid;
    o[2 * plane] = lo;
  }
}

// out[plane * p + r * out_ld + j] = in[r * in_ld + j] for p = 0, 1, 2 and
// j < bytes (the packed signs repeated for each limb); in may be plane 0 of
// out itself, which is then left as it is
__global__ __launch_bounds__(256) void repeat_kernel(const uint8_t* in, int64_t rows, int64_t bytes, int64_t in_ld,
                                                     uint8_t* out, int64_t out_ld, int64_t plane) {
  const int64_t n = rows * bytes;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / bytes, j = i - r * bytes;
    const uint8_t v = in[r * in_ld + j];
    uint8_t* o = out + r * out_ld + j;
    if (o != in + r * in_ld + j) o[0] = v;
    o[plane] = v;
    o[2 * plane] = v;
  }
}

inline int grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return static_cast<int>(b > 16384 ? 16384 : (b < 1 ? 1 : b));
}

inline size_t up256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

}  // namespace limbs

int launch_transpose_bits(const uint8_t*, uint8_t*, int64_t, int64_t, int64_t, int64_t, hipStream_t);

// Whether a product of these sizes takes the limbs (enough rows of output to
// fill 256-row tiles; below that the fp32 SIMT kernels are as fast)
static bool f32_limbs_worth(int64_t m) { return m >= 128; }

// The limbs of the dense operand (6 bytes per fp32 value) are held to this
// many bytes of workspace: the forward and dX products run over chunks of
// output rows whose limbs fit it, and an evidence product whose limbs do not
// fit takes the fp32 SIMT kernels.
constexpr size_t kLimbBudget = static_cast<size_t>(512) << 20;

// Output rows per chunk of a product over k: all m when they fit the budget,
// else a multiple of the 256-row tile (0 when not even one tile fits).
static int64_t f32_chunk_rows(int64_t m, int64_t k) {
  const int64_t fit = static_cast<int64_t>(kLimbBudget / (static_cast<size_t>(k) * 3 * 2));
  return fit >= m ? m : fit / mfma::wide::BM * mfma::wide::BM;
}

static SplitK f32_forward_split(int64_t m, int64_t rows, int64_t cols) {
  return forward_split_plan(wide_grid(m, rows), static_cast<int>(3 * cols / mfma::wide::BK));
}

static size_t f32_forward_partial(int64_t m, int64_t rows, int64_t cols) {
  const SplitK sp = f32_forward_split(m, rows, cols);
  return sp.splits > 1 ? static_cast<size_t>(sp.splits) * wide_grid(m, rows) * mfma::wide::BM * mfma::wide::BN *
                             sizeof(float)
                       : 0;
}

size_t f32_forward_workspace(int64_t m, int64_t rows, int64_t cols) {
  if (m <= 0 || rows <= 0 || cols <= 0 || cols % 64 != 0 || !f32_limbs_worth(m)) return 0;
  const int64_t mc = f32_chunk_rows(m, cols);
  if (mc == 0) return 0;
  // the split-K partials of a full chunk or of the last, shorter one
  size_t partial = f32_forward_partial(mc, rows, cols);
  if (m % mc) {
    const size_t tail = f32_forward_partial(m % mc, rows, cols);
    if (tail > partial) partial = tail;
  }
  return limbs::up256(static_cast<size_t>(mc) * 3 * cols * 2) +
         limbs::up256(static_cast<size_t>(rows) * 3 * cols / 8) + partial;
}

// y [m, rows] fp32 = (x @ sign^T) * scale + bias through the limbs, over
// chunks of f32_chunk_rows rows of x.  Returns 1 when the call is not for
// this path (shape, or too little workspace).
int mfma_f32_forward(const float* x, const uint8_t* packed, const float* scale, const float* bias, float* y,
                     int64_t m, int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  const size_t need = f32_forward_workspace(m, rows, cols);
  if (need == 0 || !workspace || workspace_bytes < need) return 1;
  const int64_t k3 = 3 * cols, kb = cols / 8, mc = f32_chunk_rows(m, cols);
  if (!fits32(mc * k3 * 2) || !fits32(rows * k3 / 8)) return 1;
  uint16_t* a = static_cast<uint16_t*>(workspace);
  uint8_t* b = static_cast<uint8_t*>(workspace) + limbs::up256(static_cast<size_t>(mc) * k3 * 2);
  float* partial = reinterpret_cast<float*>(b + limbs::up256(static_cast<size_t>(rows) * k3 / 8));
  limbs::repeat_kernel<<<limbs::grid_for(rows * kb), 256, 0, stream>>>(packed, rows, kb, kb, b, 3 * kb, kb);
  for (int64_t i0 = 0; i0 < m; i0 += mc) {
    const int64_t mi = m - i0 < mc ? m - i0 : mc;
    float* yi = y + i0 * rows;
    limbs::split_kernel<<<limbs::grid_for(mi * cols), 256, 0, stream>>>(x + i0 * cols, mi, cols, nullptr, nullptr, a,
                                                                        k3, cols);
    mfma::Params p{};
    p.a = a;
    p.bits = b;
    p.out = yi;
    p.M = mi; p.N = rows; p.K = k3;
    p.lda = k3; p.pb = 3 * kb;
    p.a_rows = mi; p.bit_rows = rows;
    p.n_scale = scale; p.n_bias = bias;
    const SplitK sp = f32_forward_split(mi, rows, cols);
    const int tiles = wide_grid(mi, rows);
    if (sp.splits > 1) {
      mfma::wide::forward_split_kernel<QSTE_BF16>
          <<<tiles * sp.splits, mfma::wide::THREADS, 0, stream>>>(p, tiles, sp.ks_steps, partial);
      int rc = static_cast<int>(hipGetLastError());
      if (rc) return rc;
      const dim3 grid(mfma::wide::BM / (mfma::wide::THREADS / kWave), static_cast<unsigned>(tiles));
      mfma::wide::forward_combine_kernel<QSTE_F32>
          <<<grid, mfma::wide::THREADS, 0, stream>>>(partial, tiles, sp.splits, scale, bias, yi, mi, rows);
    } else {
      mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_K, mfma::EPI_FORWARD_F32, QSTE_BF16>
          <<<tiles, mfma::wide::THREADS, 0, stream>>>(p);
    }
    const int rc = static_cast<int>(hipGetLastError());
    if (rc) return rc;
  }
  return 0;
}

size_t f32_dgrad_workspace(int64_t m, int64_t rows, int64_t cols) {
  if (m <= 0 || rows <= 0 || cols <= 0 || rows % 64 != 0 || !f32_limbs_worth(m)) return 0;
  const int64_t mc = f32_chunk_rows(m, rows);
  if (mc == 0) return 0;
  return limbs::up256(static_cast<size_t>(mc) * 3 * rows * 2) +
         limbs::up256(static_cast<size_t>(cols) * 3 * rows / 8);
}

// dx [m, cols] fp32 = dy @ (row_scale * sign) through the limbs: dy scaled
// by the row scale along K, the signs transposed (bits along K); over chunks
// of f32_chunk_rows rows of dy.
int mfma_f32_dgrad(const float* dy, const uint8_t* packed, const float* row_scale, float* dx, int64_t m,
                   int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const size_t need = f32_dgrad_workspace(m, rows, cols);
  if (need == 0 || !workspace || workspace_bytes < need) return 1;
  const int64_t k3 = 3 * rows, kb = rows / 8, mc = f32_chunk_rows(m, rows);
  if (!fits32(mc * k3 * 2) || !fits32(cols * k3 / 8)) return 1;
  uint16_t* a = static_cast<uint16_t*>(workspace);
  uint8_t* b = static_cast<uint8_t*>(workspace) + limbs::up256(static_cast<size_t>(mc) * k3 * 2);
  // the transposed signs into plane 0 of each row of b (its pitch 3 * kb is
  // a multiple of 8 as rows % 64 == 0), then repeated into planes 1 and 2
  int rc = launch_transpose_bits(packed, b, rows, cols, (cols + 7) / 8, 3 * kb, stream);
  if (rc) return rc;
  limbs::repeat_kernel<<<limbs::grid_for(cols * kb), 256, 0, stream>>>(b, cols, kb, 3 * kb, b, 3 * kb, kb);
  for (int64_t i0 = 0; i0 < m; i0 += mc) {
    const int64_t mi = m - i0 < mc ? m - i0 : mc;
    limbs::split_kernel<<<limbs::grid_for(mi * rows), 256, 0, stream>>>(dy + i0 * rows, mi, rows, nullptr, row_scale,
                                                                        a, k3, rows);
    mfma::Params p{};
    p.a = a;
    p.bits = b;
    p.out = dx + i0 * cols;
    p.M = mi; p.N = cols; p.K = k3;
    p.lda = k3; p.pb = 3 * kb;
    p.a_rows = mi; p.bit_rows = cols;
    mfma::wide::wide_kernel<mfma::A_ROWS_M, mfma::B_BITS_ALONG_K, mfma::EPI_FORWARD_F32, QSTE_BF16>
        <<<wide_grid(mi, cols), mfma::wide::THREADS, 0, stream>>>(p);
    if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  }
  return 0;
}

size_t f32_evidence_workspace(int64_t samples, int64_t rows, int64_t cols) {
  if (samples <= 0 || rows <= 0 || cols <= 0 || rows % 64 != 0 || cols % 64 != 0 || !f32_limbs_worth(rows))
    return 0;
  // K is the samples here: the fused epilogue needs the whole sum in one
  // pass, so a product whose limbs exceed the budget is not split up
  const size_t a = static_cast<size_t>(3 * samples) * rows * 2;
  if (a > kLimbBudget) return 0;
  return limbs::up256(a) + limbs::up256(static_cast<size_t>(3 * samples) * (cols / 8));
}

// The evidence of fp32 dy through the limbs: dy scaled by the sample scale,
// its limbs stacked along the samples (rows of K), the sample signs repeated
// the same way, and the fused evidence epilogue (offset correction, row
// scale, scale-gradient partials in mfma_evidence_tiles(cols) slots).
int mfma_f32_evidence(const float* dy, const uint8_t* packed_x, const float* x_scale, float* ev, int64_t samples,
                      int64_t rows, int64_t cols, const float* m_add, const float* m_scale, const uint8_t* w_bits,
                      float* gs_partial, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const size_t need = f32_evidence_workspace(samples, rows, cols);
  if (need == 0 || !workspace || workspace_bytes < need) return 1;
  const int64_t k3 = 3 * samples, cb = cols / 8;
  if (!fits32(k3 * rows * 2) || !fits32(k3 * cb)) return 1;
  uint16_t* a = static_cast<uint16_t*>(workspace);
  uint8_t* b = static_cast<uint8_t*>(workspace) + limbs::up256(static_cast<size_t>(k3) * rows * 2);
  limbs::split_kernel<<<limbs::grid_for(samples * rows), 256, 0, stream>>>(dy, samples, rows, x_scale, nullptr, a,
                                                                          rows, samples * rows);
  limbs::repeat_kernel<<<limbs::grid_for(samples * cb), 256, 0, stream>>>(packed_x, samples, cb, cb, b, cb,
                                                                         samples * cb);
  mfma::Params p = evidence_params(a, b, nullptr, ev, k3, rows, cols, m_add, m_scale, w_bits, gs_partial);
  mfma::wide::wide_kernel<mfma::A_ROWS_K, mfma::B_BITS_ALONG_N, mfma::EPI_EVIDENCE, QSTE_BF16>
      <<<wide_grid(rows, cols), mfma::wide::THREADS, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
