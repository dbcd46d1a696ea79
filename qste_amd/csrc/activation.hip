// Packed activations: what backward keeps of an activation, in bits or bytes.
//
// Reference behaviour (BleedingXiko/QSTE):
//   pack_bits / unpack_bits / apply_bits -- src/qste/kernels/fallback.py:32-70,
//       GPU select semantics of cuda.py:158-195 (a cleared bit gives +0)
//   masked activations (ReLU, ReLU6, Hardtanh, LeakyReLU, Hardsigmoid,
//       Dropout)                                      -- src/qste/nn.py:116-186, 267-282, 352-368
//   smooth activations, int8 derivative per row       -- src/qste/nn.py:392-507
//   relu(x)^2 with an unsigned byte per element       -- src/qste/nn.py:292-330
//   any elementwise function (derivative handed in)   -- src/qste/nn.py:510-555
//
// All of it is HBM-bound element work.  The bit kernels give one thread one
// packed byte (eight elements), so no two threads write the same byte.  The
// smooth forward gives each row to one wave or one workgroup: the row's
// derivative is computed once, held in registers while the row maximum is
// reduced, then quantized, so the input is read from HBM once.
//
// Arithmetic follows the reference's tensor expressions operation by
// operation in fp32 (the library is built without FMA contraction), with a
// rounding to the tensor dtype wherever the reference's expression produces a
// tensor of that dtype.
#include <math.h>

#include "common.hpp"

namespace qste {
namespace act {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// 8-element chunks: element c of a row lives in chunk c / 8.  A chunk is read
// with one vector load when the row is a whole number of chunks.
// ---------------------------------------------------------------------------

template <int DT>
struct Chunk;

// fetch / unpack split a whole chunk's load from its conversion, so a
// caller can issue several loads before the first conversion waits on one.
template <>
struct Chunk<QSTE_F32> {
  struct Raw {
    float4 a, b;
  };
  __device__ __forceinline__ static Raw fetch(const float* p) {
    return {reinterpret_cast<const float4*>(p)[0], reinterpret_cast<const float4*>(p)[1]};
  }
  __device__ __forceinline__ static void unpack(const Raw& r, float v[8]) {
    v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w;
    v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
  }
  __device__ __forceinline__ static void load(const float* p, int n, bool vec, float v[8]) {
    if (vec && n == 8) {
      const float4 a = reinterpret_cast<const float4*>(p)[0];
      const float4 b = reinterpret_cast<const float4*>(p)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = j < n ? p[j] : 0.0f;
    }
  }
  __device__ __forceinline__ static void store(float* p, int n, bool vec, const float v[8]) {
    if (vec && n == 8) {
      reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < n) p[j] = v[j];
    }
  }
};

template <int DT>
struct Chunk16 {
  using E = Elem<DT>;
  using Raw = uint4;
  __device__ __forceinline__ static Raw fetch(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ static void unpack(const Raw& q, float v[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t lo = static_cast<uint16_t>(w[j] & 0xFFFFu);
      const uint16_t hi = static_cast<uint16_t>(w[j] >> 16);
      v[2 * j] = E::load(&lo, 0);
      v[2 * j + 1] = E::load(&hi, 0);
    }
  }
  __device__ __forceinline__ static void load(const uint16_t* p, int n, bool vec, float v[8]) {
    if (vec && n == 8) {
      const uint4 q = *reinterpret_cast<const uint4*>(p);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = static_cast<uint16_t>(w[j] & 0xFFFFu);
        const uint16_t hi = static_cast<uint16_t>(w[j] >> 16);
        v[2 * j] = E::load(&lo, 0);
        v[2 * j + 1] = E::load(&hi, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = j < n ? E::load(p, j) : 0.0f;
    }
  }
  __device__ __forceinline__ static void store(uint16_t* p, int n, bool vec, const float v[8]) {
    if (vec && n == 8) {
      uint16_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) E::store(h, j, v[j]);
      uint4 q;
      q.x = h[0] | (static_cast<uint32_t>(h[1]) << 16);
      q.y = h[2] | (static_cast<uint32_t>(h[3]) << 16);
      q.z = h[4] | (static_cast<uint32_t>(h[5]) << 16);
      q.w = h[6] | (static_cast<uint32_t>(h[7]) << 16);
      *reinterpret_cast<uint4*>(p) = q;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < n) E::store(p, j, v[j]);
    }
  }
};

template <>
struct Chunk<QSTE_F16> : Chunk16<QSTE_F16> {};
template <>
struct Chunk<QSTE_BF16> : Chunk16<QSTE_BF16> {};

// ---------------------------------------------------------------------------
// pack_bits / unpack_bits
// ---------------------------------------------------------------------------

__global__ void pack_bits_kernel(const uint8_t* __restrict__ mask, uint8_t* __restrict__ packed,
                                 int64_t rows, int64_t cols, int64_t pb) {
  const int64_t total = rows * pb;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / pb;
    const int64_t b = idx - r * pb;
    const uint8_t* src = mask + r * cols + b * 8;
    const int64_t n = cols - b * 8 < 8 ? cols - b * 8 : 8;
    uint32_t byte = 0;
    if (n == 8 && (cols & 7) == 0) {
      const uint64_t w = *reinterpret_cast<const uint64_t*>(src);
#pragma unroll
      for (int j = 0; j < 8; ++j) byte |= (((w >> (8 * j)) & 0xFFu) != 0 ? 1u : 0u) << j;
    } else {
      for (int j = 0; j < n; ++j) byte |= (src[j] != 0 ? 1u : 0u) << j;
    }
    packed[idx] = static_cast<uint8_t>(byte);
  }
}

template <int DT>
__global__ void unpack_bits_kernel(const uint8_t* __restrict__ packed, typename Elem<DT>::T* __restrict__ out,
                                   int64_t rows, int64_t cols, int64_t pb) {
  const int64_t total = rows * pb;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / pb;
    const int64_t b = idx - r * pb;
    const int n = static_cast<int>(cols - b * 8 < 8 ? cols - b * 8 : 8);
    const uint32_t byte = packed[idx];
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = static_cast<float>((byte >> j) & 1u);
    typename Elem<DT>::T* dst = out + r * cols + b * 8;
    Chunk<DT>::store(dst, n, (cols & 7) == 0, v);
  }
}

// ---------------------------------------------------------------------------
// Masked backward: one formula for every one-bit activation.
//   kept = bit ? g : 0
//   outside == 0:  out = kept * inside                     (ReLU family: inside 1;
//                                                            Dropout: inside = gain;
//                                                            Hardsigmoid: 1/6)
//   otherwise:     out = g * outside + kept * diff         (LeakyReLU, nn.py:278-282)
// each product and the sum rounded to the dtype, as the tensor expressions are.
// ---------------------------------------------------------------------------

template <int DT>
__global__ void masked_backward_kernel(const typename Elem<DT>::T* __restrict__ grad,
                                       const uint8_t* __restrict__ packed,
                                       typename Elem<DT>::T* __restrict__ out, int64_t rows, int64_t cols,
                                       int64_t pb, float inside, float outside, float diff) {
  using E = Elem<DT>;
  const int64_t total = rows * pb;
  const bool whole = (cols & 7) == 0;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / pb;
    const int64_t b = idx - r * pb;
    const int n = static_cast<int>(cols - b * 8 < 8 ? cols - b * 8 : 8);
    const int64_t off = r * cols + b * 8;
    float g[8], o[8];
    const uint32_t byte = packed[idx];
    Chunk<DT>::load(grad + off, n, whole, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float kept = ((byte >> j) & 1u) ? g[j] : 0.0f;
      if (outside == 0.0f) {
        o[j] = kept * inside;
      } else {
        o[j] = E::round(E::round(g[j] * outside) + E::round(kept * diff));
      }
    }
    Chunk<DT>::store(out + off, n, whole, o);
  }
}

// ---------------------------------------------------------------------------
// Masked forward.
//   CLAMP   out = clamp(x, lower, upper) (upper first, nn.py:121-122),
//           bit = lower < out (< upper)            (ReLU, ReLU6, Hardtanh)
//   LEAKY   out = x > 0 ? x : x * slope, bit = x > 0           (LeakyReLU)
//   INTERVAL bit = lower < x (< upper); out not written       (Hardsigmoid)
// Bounds compare against their value rounded to the dtype, as a comparison of
// a tensor of that dtype with a Python scalar does.
// ---------------------------------------------------------------------------

template <int DT>
__global__ void masked_forward_kernel(const typename Elem<DT>::T* __restrict__ x,
                                      typename Elem<DT>::T* __restrict__ out, uint8_t* __restrict__ packed,
                                      int64_t rows, int64_t cols, int64_t pb, int kind, float lower,
                                      float upper, int has_upper, float slope) {
  using E = Elem<DT>;
  const int64_t total = rows * pb;
  const bool whole = (cols & 7) == 0;
  const float lo_d = E::round(lower);
  const float hi_d = E::round(upper);
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / pb;
    const int64_t b = idx - r * pb;
    const int n = static_cast<int>(cols - b * 8 < 8 ? cols - b * 8 : 8);
    const int64_t off = r * cols + b * 8;
    float v[8], o[8];
    Chunk<DT>::load(x + off, n, whole, v);
    uint32_t byte = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bool keep;
      if (kind == QSTE_MASK_CLAMP) {
        float t = v[j];
        if (has_upper && t > upper) t = hi_d;
        if (t < lower) t = lo_d;
        o[j] = t;
        keep = t > lo_d && (!has_upper || t < hi_d);
      } else if (kind == QSTE_MASK_LEAKY) {
        keep = v[j] > 0.0f;
        o[j] = keep ? v[j] : E::round(v[j] * slope);
      } else {
        keep = v[j] > lo_d && (!has_upper || v[j] < hi_d);
        o[j] = 0.0f;
      }
      byte |= (keep && j < n ? 1u : 0u) << j;
    }
    if (out != nullptr && kind != QSTE_MASK_INTERVAL) Chunk<DT>::store(out + off, n, whole, o);
    packed[idx] = static_cast<uint8_t>(byte);
  }
}

// ---------------------------------------------------------------------------
// Smooth activations.
// ---------------------------------------------------------------------------

struct SmoothParams {
  int kind;
  float a;  // alpha (ELU, CELU) or beta (Softplus)
};

constexpr double kSqrt2 = 1.4142135623730951;
constexpr double kInvSqrt2Pi = 0.3989422804014327;   // 1 / sqrt(2 pi)
constexpr double kSqrt2OverPi = 0.7978845608028654;  // sqrt(2 / pi)
constexpr double kTanhCoefficient = 0.044715;
constexpr double kSeluAlpha = 1.6732632423543772;
constexpr double kSeluScale = 1.0507009873554805;

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float softplus_f(float x, float beta) {
  const float bx = x * beta;
  return bx > 20.0f ? x : log1pf(expf(bx)) / beta;
}

// f(x) in fp32: the value torch's activation computes before its rounding to
// the dtype.
template <int KIND>
__device__ __forceinline__ float value_of(float x, float a) {
  if constexpr (KIND == QSTE_ACT_GELU) {
    return x * 0.5f * (1.0f + erff(x * static_cast<float>(0.70710678118654752440)));
  } else if constexpr (KIND == QSTE_ACT_GELU_TANH) {
    const float beta = static_cast<float>(kSqrt2 * 1.12837916709551257390 * 0.5);
    const float kappa = static_cast<float>(kTanhCoefficient);
    const float cube = x * x * x;
    const float inner = beta * (x + kappa * cube);
    return 0.5f * x * (1.0f + tanhf(inner));
  } else if constexpr (KIND == QSTE_ACT_SILU) {
    return x / (1.0f + expf(-x));
  } else if constexpr (KIND == QSTE_ACT_TANH) {
    return tanhf(x);
  } else if constexpr (KIND == QSTE_ACT_SIGMOID) {
    return 1.0f / (1.0f + expf(-x));
  } else if constexpr (KIND == QSTE_ACT_ELU) {
    return x <= 0.0f ? expm1f(x) * a : x;
  } else if constexpr (KIND == QSTE_ACT_CELU) {
    return x <= 0.0f ? expm1f(x * (1.0f / a)) * a : x;
  } else if constexpr (KIND == QSTE_ACT_SELU) {
    const float scale = static_cast<float>(kSeluScale);
    const float neg = static_cast<float>(kSeluAlpha) * scale;
    return x <= 0.0f ? expm1f(x) * neg : x * scale;
  } else if constexpr (KIND == QSTE_ACT_SOFTPLUS) {
    return softplus_f(x, a);
  } else if constexpr (KIND == QSTE_ACT_MISH) {
    return x * tanhf(log1pf(expf(x)));
  } else if constexpr (KIND == QSTE_ACT_HARDSWISH) {
    return x * fminf(fmaxf(x + 3.0f, 0.0f), 6.0f) / 6.0f;
  } else if constexpr (KIND == QSTE_ACT_RELU_SQUARE) {
    const float r = x < 0.0f ? 0.0f : x;
    return r * r;
  } else {
    return 0.0f;
  }
}

// The derivative the reference retains (nn.py:392-440, 456-481), from the
// input x and the output y as a tensor of the dtype (y already rounded).
template <int KIND>
__device__ __forceinline__ float derivative_of(float x, float y, float a) {
  if constexpr (KIND == QSTE_ACT_GELU) {
    // x / sqrt(2) through the correctly rounded reciprocal (same quotient)
    constexpr float kS2 = static_cast<float>(kSqrt2);
    constexpr float kInvS2 = 1.0f / kS2;
    const float cumulative = 0.5f * (1.0f + erff(div_by(x, kS2, kInvS2)));
    const float e = expf(-0.5f * x * x);
    return cumulative + x * e * static_cast<float>(kInvSqrt2Pi);
  } else if constexpr (KIND == QSTE_ACT_GELU_TANH) {
    const float s = static_cast<float>(kSqrt2OverPi);
    const float cube = x * x * x;
    const float inner = s * (x + static_cast<float>(kTanhCoefficient) * cube);
    const float t = tanhf(inner);
    const float left = 0.5f * (1.0f + t);
    const float right = 0.5f * x * (1.0f - t * t) * s * (1.0f + static_cast<float>(3.0 * kTanhCoefficient) * x * x);
    return left + right;
  } else if constexpr (KIND == QSTE_ACT_SILU) {
    const float s = sigmoid_f(x);
    return s * (1.0f + x * (1.0f - s));
  } else if constexpr (KIND == QSTE_ACT_TANH) {
    return 1.0f - y * y;
  } else if constexpr (KIND == QSTE_ACT_SIGMOID) {
    return y * (1.0f - y);
  } else if constexpr (KIND == QSTE_ACT_ELU) {
    return x > 0.0f ? 1.0f : y + a;
  } else if constexpr (KIND == QSTE_ACT_CELU) {
    return x > 0.0f ? 1.0f : y / a + 1.0f;
  } else if constexpr (KIND == QSTE_ACT_SELU) {
    return x > 0.0f ? static_cast<float>(kSeluScale) : y + static_cast<float>(kSeluScale * kSeluAlpha);
  } else if constexpr (KIND == QSTE_ACT_SOFTPLUS) {
    return sigmoid_f(a * x);
  } else if constexpr (KIND == QSTE_ACT_MISH) {
    const float t = tanhf(softplus_f(x, 1.0f));
    return t + x * (1.0f - t * t) * sigmoid_f(x);
  } else if constexpr (KIND == QSTE_ACT_HARDSWISH) {
    return x <= -3.0f ? 0.0f : (x >= 3.0f ? 1.0f : (2.0f * x + 3.0f) / 6.0f);
  } else if constexpr (KIND == QSTE_ACT_RELU_SQUARE) {
    return x < 0.0f ? 0.0f : x;  // the retained quantity: relu(x), a tensor of the dtype
  } else {
    return 0.0f;
  }
}

// Value (rounded to the dtype) and derivative of one element, sharing the
// subexpressions the two formulas have in common; every shared value is the
// one each formula computes on its own, so the results are unchanged.
template <int KIND, int DT>
__device__ __forceinline__ void value_and_derivative(float x, float a, float& y, float& d) {
  using E = Elem<DT>;
  if constexpr (KIND == QSTE_ACT_SILU) {
    const float denom = 1.0f + expf(-x);  // torch's silu and sigmoid share it
    const float s = 1.0f / denom;         // sigmoid(x) = RN(1 / denom)
    // x / denom from that reciprocal while it stays a normal number
    y = E::round(denom < 0x1p60f ? div_by(x, denom, s) : x / denom);
    d = s * (1.0f + x * (1.0f - s));
  } else if constexpr (KIND == QSTE_ACT_MISH) {
    const float e = expf(x);
    const float t = tanhf(log1pf(e));  // softplus below its threshold is log1p(exp(x))
    y = E::round(x * t);
    const float t2 = x > 20.0f ? tanhf(x) : t;
    d = t2 + x * (1.0f - t2 * t2) * sigmoid_f(x);
  } else if constexpr (KIND == QSTE_ACT_RELU_SQUARE) {
    y = E::round(value_of<KIND>(x, a));
    d = E::round(derivative_of<KIND>(x, y, a));
  } else {
    y = E::round(value_of<KIND>(x, a));
    d = derivative_of<KIND>(x, y, a);
  }
}

// Any kind chosen at run time (the generic path; the hot kinds also have
// specialised instantiations).
constexpr int kDynamic = -1;

// Kinds whose retained derivative reads the output y (the others need only x).
__host__ __device__ constexpr bool derivative_reads_y(int kind) {
  return kind == QSTE_ACT_TANH || kind == QSTE_ACT_SIGMOID || kind == QSTE_ACT_ELU || kind == QSTE_ACT_CELU ||
         kind == QSTE_ACT_SELU;
}

template <int KIND, int DT>
__device__ __forceinline__ void value_and_derivative_any(int kind, float x, float a, float& y, float& d) {
  if constexpr (KIND != kDynamic) {
    value_and_derivative<KIND, DT>(x, a, y, d);
  } else {
    switch (kind) {
#define QSTE_VD(K) case K: value_and_derivative<K, DT>(x, a, y, d); break;
      QSTE_VD(QSTE_ACT_GELU) QSTE_VD(QSTE_ACT_GELU_TANH) QSTE_VD(QSTE_ACT_SILU) QSTE_VD(QSTE_ACT_TANH)
      QSTE_VD(QSTE_ACT_SIGMOID) QSTE_VD(QSTE_ACT_ELU) QSTE_VD(QSTE_ACT_CELU) QSTE_VD(QSTE_ACT_SELU)
      QSTE_VD(QSTE_ACT_SOFTPLUS) QSTE_VD(QSTE_ACT_MISH) QSTE_VD(QSTE_ACT_HARDSWISH) QSTE_VD(QSTE_ACT_RELU_SQUARE)
#undef QSTE_VD
      default: y = 0.0f; d = 0.0f;
    }
  }
}

template <int KIND, int DT>
__device__ __forceinline__ float derivative_any(int kind, float x, float y, float a) {
  using E = Elem<DT>;
  if constexpr (KIND != kDynamic) {
    return KIND == QSTE_ACT_RELU_SQUARE ? E::round(derivative_of<KIND>(x, y, a)) : derivative_of<KIND>(x, y, a);
  } else {
    switch (kind) {
#define QSTE_D(K) case K: return derivative_of<K>(x, y, a);
      QSTE_D(QSTE_ACT_GELU) QSTE_D(QSTE_ACT_GELU_TANH) QSTE_D(QSTE_ACT_SILU) QSTE_D(QSTE_ACT_TANH)
      QSTE_D(QSTE_ACT_SIGMOID) QSTE_D(QSTE_ACT_ELU) QSTE_D(QSTE_ACT_CELU) QSTE_D(QSTE_ACT_SELU)
      QSTE_D(QSTE_ACT_SOFTPLUS) QSTE_D(QSTE_ACT_MISH) QSTE_D(QSTE_ACT_HARDSWISH)
#undef QSTE_D
      case QSTE_ACT_RELU_SQUARE: return E::round(derivative_of<QSTE_ACT_RELU_SQUARE>(x, y, a));
      default: return 0.0f;
    }
  }
}

// Maximum over a row's G threads (G = 64: within the wave; otherwise G is the
// whole workgroup) of |d| as bit patterns: for non-negative floats the bit
// order is the numeric order and every NaN lies above +inf, so the maximum
// keeps a NaN as the reference's amax does.
template <int G>
__device__ __forceinline__ uint32_t group_max_bits(uint32_t v, float* red) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, offset, kWave)));
  if (G == kWave) return v;
  uint32_t* r = reinterpret_cast<uint32_t*>(red);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) r[wave] = v;
  __syncthreads();
  uint32_t m = r[0];
#pragma unroll
  for (int w = 1; w < G / kWave; ++w) m = max(m, r[w]);
  return m;
}

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

// v_cvt_i32_f32: NaN converts to 0 and values beyond the int32 range saturate
// (the quantizer's NaN -> 0 rule in one instruction).
__device__ __forceinline__ int32_t cvt_i32_nan0(float v) {
  int32_t r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// bf16 SiLU table entry: .x the derivative's bits, .y the value's bf16 bits.
using SmoothEntry = uint2;

// The entry of any bf16 input (the table holds those of tab16_index's range).
template <int KIND>
__device__ __forceinline__ SmoothEntry smooth_entry(uint32_t h, float a) {
  float v, d;
  value_and_derivative<KIND, QSTE_BF16>(__uint_as_float(h << 16), a, v, d);
  return make_uint2(__float_as_uint(d), f32_to_bf16(v));
}

// One whole bf16 chunk through the table: derivatives into d, the values'
// bf16 bits packed two to a word into ybits.  Every lane looks up all eight
// entries (inputs outside the tabulated range read entry 0) before the first
// use, and only lanes holding such an input recompute those elements.
template <int KIND>
__device__ __forceinline__ void table_chunk(const uint4& raw, const SmoothEntry* tab, float a, float d[8],
                                            uint32_t ybits[4]) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t idx[8], miss = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t h = (j & 1) ? (w[j / 2] >> 16) : (w[j / 2] & 0xFFFFu);
    uint32_t i;
    const bool in = tab16_index(h, i);
    idx[j] = in ? i : 0u;
    miss |= (in ? 0u : 1u) << j;
  }
  SmoothEntry e[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) e[j] = tab[idx[j]];
  if (miss) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (miss & (1u << j)) e[j] = smooth_entry<KIND>((j & 1) ? (w[j / 2] >> 16) : (w[j / 2] & 0xFFFFu), a);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) d[j] = __uint_as_float(e[j].x);
#pragma unroll
  for (int j = 0; j < 4; ++j) ybits[j] = e[2 * j].y | (e[2 * j + 1].y << 16);
}

// One row per group of G threads: G = 64 is a wave (BLOCK / 64 rows per
// workgroup), G = BLOCK a whole workgroup.  Thread t owns the 8-element
// chunks t, t + G, ...  With CH > 0 a row has at most G * CH chunks and each
// thread's derivatives stay in registers (unrolled, constant indices) between
// the row maximum and the quantization, so the input is read once; with
// CH == 0 (longer rows) they are recomputed from the input, still in L2.
// KIND == kDynamic takes the kind from `kind` at run time.
//
// mode: 0 -- compute y = f(x), store it (when y != NULL), derive from it
//       1 -- y holds the forward output already (computed elsewhere); read it
//       2 -- `provided` holds the fp32 derivative (x, y unused)
// tab (bf16 SiLU in mode 0 with whole chunks, may be NULL): value and
// derivative of the tabulated bf16 inputs (tab16_index), filled by the caller.
template <int DT, int G, int CH, int KIND, int BLOCK>
__device__ __forceinline__ void smooth_row(const typename Elem<DT>::T* __restrict__ x,
                                           typename Elem<DT>::T* __restrict__ y,
                                           const float* __restrict__ provided, int run_mode, int kind, float a,
                                           void* __restrict__ payload, float* __restrict__ scale,
                                           int64_t rows, int64_t cols, float* red, int64_t block,
                                           const SmoothEntry* tab = nullptr) {
  using E = Elem<DT>;
  const bool kUsq = (KIND == kDynamic ? kind : KIND) == QSTE_ACT_RELU_SQUARE;
  // the specialised kinds run in one mode only (smooth_dispatch)
  const int mode = KIND == QSTE_ACT_SILU || KIND == QSTE_ACT_GELU
                       ? 0
                       : (KIND == QSTE_ACT_GELU_TANH || KIND == QSTE_ACT_HARDSWISH ? 1 : run_mode);
  constexpr int kRowsPerBlock = BLOCK / G;
  const int64_t row = block * kRowsPerBlock + threadIdx.x / G;
  const int t = threadIdx.x % G;
  const bool live = row < rows;
  const int64_t nch = (cols + 7) / 8;
  const bool whole = (cols & 7) == 0;
  const int64_t base = (live ? row : 0) * cols;

  // mode 0: v holds the input chunk q on entry and its derivatives on exit
  auto from_input = [&](int64_t q, float v[8], bool write_y) __attribute__((always_inline)) {
    const int n = static_cast<int>(cols - q * 8 < 8 ? cols - q * 8 : 8);
    float yv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float d;
      value_and_derivative_any<KIND, DT>(kind, v[j], a, yv[j], d);
      v[j] = j < n ? d : 0.0f;
    }
    if (write_y && y != nullptr) Chunk<DT>::store(y + base + q * 8, n, whole, yv);
  };

  auto derive = [&](int64_t q, float d[8], bool write_y) __attribute__((always_inline)) {
    const int n = static_cast<int>(cols - q * 8 < 8 ? cols - q * 8 : 8);
    if (mode == 2) {
      Chunk<QSTE_F32>::load(provided + base + q * 8, n, whole, d);
#pragma unroll
      for (int j = 0; j < 8; ++j) d[j] = j < n ? d[j] : 0.0f;
      return;
    }
    float xv[8], yv[8];
    Chunk<DT>::load(x + base + q * 8, n, whole, xv);
    if (mode == 0) {
      from_input(q, xv, write_y);
#pragma unroll
      for (int j = 0; j < 8; ++j) d[j] = xv[j];
      return;
    }
    const bool reads_y = KIND == kDynamic ? derivative_reads_y(kind) : derivative_reads_y(KIND);
    if (reads_y) {
      Chunk<DT>::load(y + base + q * 8, n, whole, yv);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) yv[j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = derivative_any<KIND, DT>(kind, xv[j], yv[j], a);
      d[j] = j < n ? v : 0.0f;
    }
  };

  // d / s through r = RN(1 / s): the row scale lies in [1e-8 / 255, amax / 127]
  // and |d / s| <= 255, so no step leaves the normal range.  A NaN or
  // infinite scale, or an infinite d, gives a NaN or zero quotient here where
  // the division gives NaN or zero, and both store 0.
  auto quantize = [&](int64_t q, const float d[8], float s, float r) __attribute__((always_inline)) {
    const int n = static_cast<int>(cols - q * 8 < 8 ? cols - q * 8 : 8);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q0 = d[j] * r;
      const float quot = fmaf(fmaf(-q0, s, d[j]), r, q0);
      uint32_t byte;
      if (kUsq) {
        const int32_t v = cvt_i32_nan0(rintf(E::round(quot)));
        byte = static_cast<uint32_t>(min(max(v, 0), 255));
      } else {
        const int32_t v = cvt_i32_nan0(rintf(quot));
        byte = static_cast<uint32_t>(min(max(v, -127), 127)) & 0xFFu;
      }
      if (j < 4) lo |= byte << (8 * j);
      else hi |= byte << (8 * (j - 4));
    }
    uint8_t* dst = static_cast<uint8_t*>(payload) + base + q * 8;
    if (whole) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
    } else {
      for (int j = 0; j < n; ++j) dst[j] = static_cast<uint8_t>(((j < 4 ? lo : hi) >> (8 * (j & 3))) & 0xFFu);
    }
  };

  float cache[CH > 0 ? CH : 1][8];
  uint32_t amax = 0;
  if constexpr (CH > 0) {
    if (mode == 0 && whole && nch > 0) {
      // every chunk's load is issued before the first conversion, branch-free
      // (chunks past the row, and dead rows, read chunk 0 of their row or of
      // row 0 and are not used)
      typename Chunk<DT>::Raw raw[CH];
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int64_t q = t + static_cast<int64_t>(k) * G;
        raw[k] = Chunk<DT>::fetch(x + base + (q < nch ? q : 0) * 8);
      }
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int64_t q = t + static_cast<int64_t>(k) * G;
        if (live && q < nch) {
          bool done = false;
          if constexpr (KIND == QSTE_ACT_SILU && DT == QSTE_BF16) {
            if (tab != nullptr) {
              uint32_t ybits[4];
              table_chunk<KIND>(raw[k], tab, a, cache[k], ybits);
              if (y != nullptr)
                *reinterpret_cast<uint4*>(y + base + q * 8) = make_uint4(ybits[0], ybits[1], ybits[2], ybits[3]);
              done = true;
            }
          }
          if (!done) {
            Chunk<DT>::unpack(raw[k], cache[k]);
            from_input(q, cache[k], true);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) amax = max(amax, abs_bits(cache[k][j]));
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int64_t q = t + static_cast<int64_t>(k) * G;
        if (live && q < nch) {
          derive(q, cache[k], true);
#pragma unroll
          for (int j = 0; j < 8; ++j) amax = max(amax, abs_bits(cache[k][j]));
        }
      }
    }
  } else if (live) {
    for (int64_t q = t; q < nch; q += G) {
      float d[8];
      derive(q, d, true);
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = max(amax, abs_bits(d[j]));
    }
  }
  amax = group_max_bits<G>(amax, red);
  if (!live) return;
  float s;
  if (amax > 0x7F800000u) {
    s = __builtin_nanf("");
  } else {
    const float key = __uint_as_float(amax);
    if (kUsq) {
      // relu(x)^2: maximum, clamp and division in the dtype (nn.py:316-318)
      s = E::round(E::round(fmaxf(key, 1e-8f)) / 255.0f);
    } else {
      s = fmaxf(key, 1e-8f) / 127.0f;
    }
  }
  const float r = 1.0f / s;
  if constexpr (CH > 0) {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int64_t q = t + static_cast<int64_t>(k) * G;
      if (q < nch) quantize(q, cache[k], s, r);
    }
  } else {
    for (int64_t q = t; q < nch; q += G) {
      float d[8];
      derive(q, d, false);
      quantize(q, d, s, r);
    }
  }
  if (t == 0) scale[row] = s;
}

// bf16 SiLU takes its value and derivative from an LDS table (4096 entries of
// 8 bytes, tab16_index's range) that each workgroup fills once and then walks
// row blocks, so the exponential and divisions are paid per table entry, not
// per element.
template <int DT, int KIND>
constexpr bool kSmoothTable = KIND == QSTE_ACT_SILU && DT == QSTE_BF16;

template <int DT, int G, int CH, int KIND, int BLOCK>
__global__ __launch_bounds__(BLOCK) void smooth_rows_kernel(
    const typename Elem<DT>::T* __restrict__ x, typename Elem<DT>::T* __restrict__ y,
    const float* __restrict__ provided, int mode, SmoothParams p, void* __restrict__ payload,
    float* __restrict__ scale, int64_t rows, int64_t cols, int64_t blocks) {
  __shared__ float red[BLOCK / kWave];
  if constexpr (kSmoothTable<DT, KIND>) {
    __shared__ SmoothEntry tab[kTab16Entries];
    for (int j = threadIdx.x; j < kTab16Entries; j += BLOCK)
      tab[j] = smooth_entry<KIND>(tab16_bits(static_cast<uint32_t>(j)), p.a);
    __syncthreads();
    // every thread walks the same blocks, so the reductions' barriers match
    for (int64_t b = blockIdx.x; b < blocks; b += gridDim.x)
      smooth_row<DT, G, CH, KIND, BLOCK>(x, y, provided, mode, p.kind, p.a, payload, scale, rows, cols, red, b,
                                         mode == 0 ? tab : nullptr);
  } else {
    smooth_row<DT, G, CH, KIND, BLOCK>(x, y, provided, mode, p.kind, p.a, payload, scale, rows, cols, red,
                                       blockIdx.x);
  }
}

// grad * (payload * scale), each product rounded to the dtype
// (nn.py:504-507; relu(x)^2: grad * 2 * (payload * scale), nn.py:325-330).
template <int DT>
__global__ void smooth_backward_kernel(const typename Elem<DT>::T* __restrict__ grad,
                                       const void* __restrict__ payload, const float* __restrict__ scale,
                                       typename Elem<DT>::T* __restrict__ out, int64_t rows, int64_t cols,
                                       int unsigned_payload) {
  using E = Elem<DT>;
  const int64_t nch = (cols + 7) / 8;
  const int64_t total = rows * nch;
  const bool whole = (cols & 7) == 0;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / nch;
    const int64_t q = idx - r * nch;
    const int n = static_cast<int>(cols - q * 8 < 8 ? cols - q * 8 : 8);
    const int64_t off = r * cols + q * 8;
    const float s = E::round(scale[r]);
    float g[8], o[8];
    Chunk<DT>::load(grad + off, n, whole, g);
    const uint8_t* src = static_cast<const uint8_t*>(payload) + off;
    uint32_t lo = 0, hi = 0;
    if (whole) {
      const uint2 w = *reinterpret_cast<const uint2*>(src);
      lo = w.x;
      hi = w.y;
    } else {
      for (int j = 0; j < n; ++j) (j < 4 ? lo : hi) |= static_cast<uint32_t>(src[j]) << (8 * (j & 3));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t byte = ((j < 4 ? lo : hi) >> (8 * (j & 3))) & 0xFFu;
      const float pv = unsigned_payload ? static_cast<float>(byte)
                                        : static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(byte)));
      const float d = E::round(pv * s);
      o[j] = unsigned_payload ? E::round(E::round(g[j] * 2.0f) * d) : E::round(g[j] * d);
    }
    Chunk<DT>::store(out + off, n, whole, o);
  }
}

inline int grid_for(int64_t items) {
  int64_t blocks = (items + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  return static_cast<int>(blocks < 1 ? 1 : blocks);
}

inline bool dtype_ok(int d) { return d == QSTE_F32 || d == QSTE_F16 || d == QSTE_BF16; }

}  // namespace act
}  // namespace qste

using namespace qste;
using namespace qste::act;

namespace {

#define QSTE_DT_SWITCH(dtype, ...)                                  \
  switch (dtype) {                                                 \
    case QSTE_F32: { constexpr int DT = QSTE_F32; __VA_ARGS__; } break;  \
    case QSTE_F16: { constexpr int DT = QSTE_F16; __VA_ARGS__; } break;  \
    case QSTE_BF16: { constexpr int DT = QSTE_BF16; __VA_ARGS__; } break; \
    default: return QSTE_E_DTYPE;                                  \
  }

bool chunk_aligned(const void* p, int dtype) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  (void)dtype;
  return (a % 16) == 0;
}

template <int DT, int G, int CH, int KIND, int BLOCK>
int smooth_launch(const void* x, void* y, const float* provided, int mode, SmoothParams p, void* payload,
                  float* scale, int64_t rows, int64_t cols, hipStream_t s) {
  using T = typename Elem<DT>::T;
  constexpr int kRows = BLOCK / G;
  const int64_t blocks = (rows + kRows - 1) / kRows;
  // the tabulated kind: a few workgroups per CU, each filling its table once
  const int64_t grid = kSmoothTable<DT, KIND> ? (blocks < 8192 / (BLOCK / kWave) ? blocks : 8192 / (BLOCK / kWave))
                                              : blocks;
  smooth_rows_kernel<DT, G, CH, KIND, BLOCK><<<static_cast<unsigned>(grid), BLOCK, 0, s>>>(
      static_cast<const T*>(x), static_cast<T*>(y), provided, mode, p, payload, scale, rows, cols, blocks);
  return static_cast<int>(hipGetLastError());
}

// Row length -> threads per row, at most two register-cached chunks each:
// <= 1024 columns a wave (4 rows per workgroup), <= 4096 a 256-thread
// workgroup, <= 16384 a 1024-thread workgroup; longer rows recompute.
template <int DT, int KIND>
int smooth_shapes(const void* x, void* y, const float* provided, int mode, SmoothParams p, void* payload,
                  float* scale, int64_t rows, int64_t cols, hipStream_t s) {
  if constexpr (KIND == kDynamic) {
    // every kind in one kernel: derivatives recomputed, no unrolled cache
    if (cols <= 1024) return smooth_launch<DT, 64, 0, KIND, 256>(x, y, provided, mode, p, payload, scale, rows, cols, s);
    if (cols <= 4096) return smooth_launch<DT, 256, 0, KIND, 256>(x, y, provided, mode, p, payload, scale, rows, cols, s);
    return smooth_launch<DT, 1024, 0, KIND, 1024>(x, y, provided, mode, p, payload, scale, rows, cols, s);
  } else {
    if (cols <= 1024) return smooth_launch<DT, 64, 2, KIND, 256>(x, y, provided, mode, p, payload, scale, rows, cols, s);
    if (cols <= 4096) return smooth_launch<DT, 256, 2, KIND, 256>(x, y, provided, mode, p, payload, scale, rows, cols, s);
    if (cols <= 16384)
      return smooth_launch<DT, 1024, 2, KIND, 1024>(x, y, provided, mode, p, payload, scale, rows, cols, s);
    return smooth_launch<DT, 1024, 0, KIND, 1024>(x, y, provided, mode, p, payload, scale, rows, cols, s);
  }
}

// The MLP activations get kernels of their own: GELU and SiLU computing their
// value, tanh-GELU and Hardswish deriving from torch's (which they cannot
// reproduce bit for bit); every other case runs the run-time-kind kernel.
template <int DT>
int smooth_dispatch(const void* x, void* y, const float* provided, int mode, SmoothParams p, void* payload,
                    float* scale, int64_t rows, int64_t cols, hipStream_t s) {
  if (mode == 0 && p.kind == QSTE_ACT_SILU)
    return smooth_shapes<DT, QSTE_ACT_SILU>(x, y, provided, mode, p, payload, scale, rows, cols, s);
  if (mode == 0 && p.kind == QSTE_ACT_GELU)
    return smooth_shapes<DT, QSTE_ACT_GELU>(x, y, provided, mode, p, payload, scale, rows, cols, s);
  if (mode == 1 && p.kind == QSTE_ACT_GELU_TANH)
    return smooth_shapes<DT, QSTE_ACT_GELU_TANH>(x, y, provided, mode, p, payload, scale, rows, cols, s);
  if (mode == 1 && p.kind == QSTE_ACT_HARDSWISH)
    return smooth_shapes<DT, QSTE_ACT_HARDSWISH>(x, y, provided, mode, p, payload, scale, rows, cols, s);
  return smooth_shapes<DT, kDynamic>(x, y, provided, mode, p, payload, scale, rows, cols, s);
}

}  // namespace

extern "C" {

int qste_pack_bits(const uint8_t* mask, uint8_t* packed, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  const int64_t pb = (cols + 7) / 8;
  if (rows * pb == 0) return 0;
  if (!mask || !packed) return QSTE_E_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  pack_bits_kernel<<<grid_for(rows * pb), kThreads, 0, s>>>(mask, packed, rows, cols, pb);
  return static_cast<int>(hipGetLastError());
}

int qste_unpack_bits(const uint8_t* packed, void* out, int out_dtype, int64_t rows, int64_t cols,
                     void* stream) {
  if (!act::dtype_ok(out_dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  const int64_t pb = (cols + 7) / 8;
  if (rows * pb == 0) return 0;
  if (!packed || !out) return QSTE_E_NULL;
  if ((cols & 7) == 0 && !chunk_aligned(out, out_dtype)) return QSTE_E_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QSTE_DT_SWITCH(out_dtype, unpack_bits_kernel<DT><<<grid_for(rows * pb), kThreads, 0, s>>>(
                                packed, static_cast<typename Elem<DT>::T*>(out), rows, cols, pb));
  return static_cast<int>(hipGetLastError());
}

int qste_masked_backward(const void* grad, int dtype, const uint8_t* packed, void* out, int64_t rows,
                         int64_t cols, float inside, float outside, float diff, void* stream) {
  if (!act::dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  const int64_t pb = (cols + 7) / 8;
  if (rows * pb == 0) return 0;
  if (!grad || !packed || !out) return QSTE_E_NULL;
  if ((cols & 7) == 0 && (!chunk_aligned(grad, dtype) || !chunk_aligned(out, dtype))) return QSTE_E_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QSTE_DT_SWITCH(dtype, masked_backward_kernel<DT><<<grid_for(rows * pb), kThreads, 0, s>>>(
                            static_cast<const typename Elem<DT>::T*>(grad), packed,
                            static_cast<typename Elem<DT>::T*>(out), rows, cols, pb, inside, outside, diff));
  return static_cast<int>(hipGetLastError());
}

int qste_apply_bits(const void* values, int dtype, const uint8_t* packed, void* out, int64_t rows,
                    int64_t cols, void* stream) {
  return qste_masked_backward(values, dtype, packed, out, rows, cols, 1.0f, 0.0f, 0.0f, stream);
}

int qste_masked_activation(const void* x, int dtype, int kind, float lower, float upper, int has_upper,
                           float slope, void* out, uint8_t* packed, int64_t rows, int64_t cols,
                           void* stream) {
  if (!act::dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (kind != QSTE_MASK_CLAMP && kind != QSTE_MASK_LEAKY && kind != QSTE_MASK_INTERVAL) return QSTE_E_SHAPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  const int64_t pb = (cols + 7) / 8;
  if (rows * pb == 0) return 0;
  if (!x || !packed || (kind != QSTE_MASK_INTERVAL && !out)) return QSTE_E_NULL;
  if ((cols & 7) == 0 && (!chunk_aligned(x, dtype) || (out && !chunk_aligned(out, dtype)))) return QSTE_E_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QSTE_DT_SWITCH(dtype, masked_forward_kernel<DT><<<grid_for(rows * pb), kThreads, 0, s>>>(
                            static_cast<const typename Elem<DT>::T*>(x), static_cast<typename Elem<DT>::T*>(out),
                            packed, rows, cols, pb, kind, lower, upper, has_upper, slope));
  return static_cast<int>(hipGetLastError());
}

int qste_smooth_activation(const void* x, int dtype, int kind, float param, void* y, int y_given,
                           const float* derivative, void* payload, float* scale, int64_t rows, int64_t cols,
                           void* stream) {
  if (!act::dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (kind < QSTE_ACT_GELU || kind > QSTE_ACT_PROVIDED) return QSTE_E_SHAPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows == 0) return 0;
  if (!scale || (!payload && cols > 0)) return QSTE_E_NULL;
  int mode = 0;
  if (kind == QSTE_ACT_PROVIDED) {
    if (!derivative && cols > 0) return QSTE_E_NULL;
    mode = 2;
  } else {
    if (!x && cols > 0) return QSTE_E_NULL;
    if (y_given) {
      if (!y && cols > 0) return QSTE_E_NULL;
      mode = 1;
    }
  }
  if ((cols & 7) == 0 && cols > 0) {
    if (mode == 2 && !chunk_aligned(derivative, QSTE_F32)) return QSTE_E_ALIGN;
    if (mode != 2 && (!chunk_aligned(x, dtype) || (y && !chunk_aligned(y, dtype)))) return QSTE_E_ALIGN;
    if ((reinterpret_cast<uintptr_t>(payload) & 7) != 0) return QSTE_E_ALIGN;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  SmoothParams p{kind, param};
  const int d = mode == 2 ? QSTE_F32 : dtype;
  QSTE_DT_SWITCH(d, return smooth_dispatch<DT>(x, y, derivative, mode, p, payload, scale, rows, cols, s));
  return 0;
}

int qste_smooth_backward(const void* grad, int dtype, const void* payload, int unsigned_payload,
                         const float* scale, void* out, int64_t rows, int64_t cols, void* stream) {
  if (!act::dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (rows < 0 || cols < 0) return QSTE_E_SHAPE;
  if (rows * cols == 0) return 0;
  if (!grad || !payload || !scale || !out) return QSTE_E_NULL;
  if ((cols & 7) == 0 && (!chunk_aligned(grad, dtype) || !chunk_aligned(out, dtype) ||
                          (reinterpret_cast<uintptr_t>(payload) & 7) != 0))
    return QSTE_E_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nch = (cols + 7) / 8;
  QSTE_DT_SWITCH(dtype, smooth_backward_kernel<DT><<<grid_for(rows * nch), kThreads, 0, s>>>(
                            static_cast<const typename Elem<DT>::T*>(grad), payload, scale,
                            static_cast<typename Elem<DT>::T*>(out), rows, cols, unsigned_payload));
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
