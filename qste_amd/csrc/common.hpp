// Shared device helpers for the gfx950 binary-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qste_hip.h"

namespace qste {

// How the MFMA path runs a layer's evidence (and dgrad) -- gemm_mfma.hip's
// mfma_evidence_plan: `pair` runs both products in one launch from
// transposed sign copies, else they run as two launches; evidence tiles
// [0, tiles_full) are computed whole and the rest over `splits` K ranges
// of ks_steps 64-sample steps (the last range may be shorter), finished by
// a combine pass that needs partial_bytes of workspace.
struct EvidencePlan {
  int pair;
  int tiles_full;
  int splits;
  int ks_steps;
  int64_t partial_bytes;
};

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Element conversions. bf16 / fp16 values widen to fp32 exactly; narrowing
// rounds to nearest even.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// gfx950 converts in hardware (v_cvt_pk_bf16_f32, round to nearest even;
// a NaN stays a quiet NaN)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// two values to a bf16 pair (lo in bits 0..15), one instruction
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  bf16x2_t v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// The empty asm keeps the backend from folding a preceding fp32 multiply or
// add into a mixed-precision instruction that rounds once, straight to fp16:
// the value is rounded to fp32 first, then to fp16, as a tensor expression
// evaluated in fp32 and stored as fp16 is.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT>
struct Elem;

template <>
struct Elem<QSTE_F32> {
  using T = float;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return p[i]; }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = v; }
  // rounding of a folded scale into the operand dtype (identity for fp32)
  __device__ __forceinline__ static float round(float v) { return v; }
};

template <>
struct Elem<QSTE_F16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return f16_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = f32_to_f16(v); }
  __device__ __forceinline__ static float round(float v) { return f16_to_f32(f32_to_f16(v)); }
};

template <>
struct Elem<QSTE_BF16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
  __device__ __forceinline__ static float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};

// ---------------------------------------------------------------------------
// Lookup tables over bf16 inputs.  A function of one bf16 value can be
// tabulated: entry j (0 .. kTab16Entries - 1) holds it for the bf16 value
// with bits tab16_bits(j), the values whose magnitude lies in [2^-12, 2^4)
// (both signs; nearly every activation or gate a layer produces).  A
// workgroup fills its table with the same code it would run per element,
// so a looked-up result is the same bits as the computed one.
// ---------------------------------------------------------------------------

constexpr uint32_t kTab16ExpLo = 127 - 12;        // biased exponent of 2^-12
constexpr uint32_t kTab16Half = 16 * 128;         // 16 exponents x 7 mantissa bits, per sign
constexpr int kTab16Entries = 2 * kTab16Half;
static_assert(kTab16Half == 1u << 11, "sign bit -> table half");

__device__ __forceinline__ uint32_t tab16_bits(uint32_t j) {
  return ((j & kTab16Half) << 4) | ((kTab16ExpLo << 7) + (j & (kTab16Half - 1)));
}

// The entry of bf16 bits `bits`, or false outside the tabulated range
// (zeros, subnormals, tiny or huge magnitudes, infinities, NaN).
__device__ __forceinline__ bool tab16_index(uint32_t bits, uint32_t& idx) {
  const uint32_t off = (bits & 0x7FFFu) - (kTab16ExpLo << 7);  // wraps above the range when below it
  idx = off | ((bits >> 15) << 11);
  return off < kTab16Half;
}

// ---------------------------------------------------------------------------
// Packed signs: bit j of byte b is column 8b + j; set means +1.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float sign_of(const uint8_t* row, int64_t col) {
  return ((row[col >> 3] >> (col & 7)) & 1) ? 1.0f : -1.0f;
}

// ---------------------------------------------------------------------------
// The rounding stream (src/qste/kernels/stream.py:41-66): Thomas Wang's
// 32-bit avalanche with the reference's constants, in uint32 so every shift
// is logical and every product wraps.
// ---------------------------------------------------------------------------

constexpr uint32_t kSalt = 0x2545F491u;
constexpr uint32_t kMultiplier = 0x27D4EB2Du;

__host__ __device__ __forceinline__ uint32_t scramble(uint32_t v) {
  v = (v ^ 61u) ^ (v >> 16);
  v = v + (v << 3);
  v = v ^ (v >> 4);
  v = v * kMultiplier;
  v = v ^ (v >> 15);
  return v;
}

// scramble split after its first step: for j < 2^16, scramble(x ^ j) ==
// scramble_tail(scramble_head(x) ^ j), since j never reaches x >> 16.  The
// eight elements of one packed byte (flat indices i0 + j, i0 % 8 == 0) share
// one head.
__host__ __device__ __forceinline__ uint32_t scramble_head(uint32_t x) { return (x ^ 61u) ^ (x >> 16); }
__host__ __device__ __forceinline__ uint32_t scramble_tail(uint32_t v) {
  v = v + (v << 3);
  v = v ^ (v >> 4);
  v = v * kMultiplier;
  v = v ^ (v >> 15);
  return v;
}

__host__ __device__ __forceinline__ uint32_t seed_hash(int64_t seed) {
  return scramble(static_cast<uint32_t>(static_cast<uint64_t>(seed)));
}

__host__ __device__ __forceinline__ uint32_t step_hash(int64_t step) {
  return scramble(static_cast<uint32_t>(static_cast<uint64_t>(step)) ^ kSalt);
}

// ---------------------------------------------------------------------------
// Reductions across one wavefront (64 lanes) and one workgroup.
// ---------------------------------------------------------------------------

template <class T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
  return v;
}

// Sum over the workgroup; every thread gets the total. `scratch` holds one
// T per wave. blockDim.x must be a multiple of 64.
template <class T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  T total = 0;
  for (int w = 0; w < waves; ++w) total += scratch[w];
  return total;
}

// x / d, correctly rounded, for a divisor shared by many quotients: with
// r = RN(1/d) and q0 = RN(x r) within one ulp of x/d, the residual
// x - q0 d is exact under FMA and RN(q0 + r (x - q0 d)) is the correctly
// rounded quotient (Markstein's correction step).  Three operations instead
// of a full IEEE division per element.  Valid while no step overflows or
// underflows (callers keep d and x in the normal range).  An infinite x or
// d, or a zero d, makes the residual NaN (inf - inf, 0 * inf) while q0 is
// already the IEEE quotient (+-inf, +-0, or NaN for inf / inf and 0 / 0), so
// q0 is returned then.
__device__ __forceinline__ float div_by(float x, float d, float r) {
  const float q0 = x * r;
  const float e = fmaf(-q0, d, x);
  return e == e ? fmaf(e, r, q0) : q0;
}

inline int ceil_div(int64_t a, int64_t b) { return static_cast<int>((a + b - 1) / b); }

// Wave priority `x mod 4` (s_setprio takes an immediate).  The hardware
// breaks ties between waves of equal priority by age, so in a kernel whose
// workgroups each own a fixed share of a stream, the waves a SIMD received
// first finish first and the pass ends on a tail of the youngest.  Rotating
// each wave's priority as it moves through its share, offset by its rank
// among the SIMD's waves, gives waves at the same point distinct
// priorities, each leading in turn.
__device__ __forceinline__ void rotate_priority(int x) {
  switch (x & 3) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
  }
}

}  // namespace qste
