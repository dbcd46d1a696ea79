// The SwiGLU gate h = silu(g) * u and its backward, fused.
//
// A SwiGLU MLP (down(silu(gate(x)) * up(x))) spends, between its GEMMs, one
// elementwise pass per torch operator: silu, the product, and in backward
// two products and silu's backward, each reading and writing a full
// [tokens, ffn] tensor.  Here the forward is one pass (read g and u, write h)
// and the backward one pass (read dh, g and u, write dg and du); u and g are
// what autograd keeps, where torch's chain keeps g, silu(g) and u.
//
// Every value is rounded where torch's operator chain rounds it, so the
// results equal F.silu(g) * u and its autograd gradients in the same dtype:
//   a  = dtype(g / (1 + exp(-g)))                  (silu, ActivationSiluKernel)
//   h  = dtype(a * u)                               (mul)
//   du = dtype(dh * a),  da = dtype(dh * u)         (mul's backward)
//   dg = dtype((da * s) * (1 + g * (1 - s))),  s = 1 / (1 + exp(-g))
//                                                   (silu_backward; torch's
//                                                   build contracts the
//                                                   inner multiply-add)
// The arithmetic is fp32 (torch's opmath for bf16/fp16); a bf16 x bf16
// product is exact in fp32, so only the final rounding matters there.
//
// The forward can also encode each row of h as the next layer's saved
// activation (the one-bit affine encoding, encode.hpp), from the values it
// already holds, so the down projection's forward need not read h again.
#include "common.hpp"
#include "encode.hpp"

namespace qste {
namespace swiglu {

constexpr int kThreads = 256;
constexpr int64_t kEncodeGroups = 1024;  // workgroups of the tabled encoding forward (4 per CU on 256 CUs)
constexpr int64_t kTabRows = 4;          // rows per workgroup from which the table pays for itself

__device__ __forceinline__ float silu_value(float x) { return x / (1.0f + expf(-x)); }

// The two fp32 factors of dg, from the rounded da and the input g
__device__ __forceinline__ void silu_grad_factors(float da, float x, float& ds, float& inner) {
  const float s = 1.0f / (1.0f + expf(-x));
  inner = fmaf(x, 1.0f - s, 1.0f);
  ds = da * s;
}

// dg before its rounding to the dtype (fp32, as torch's silu_backward
// computes it; its vectorized fp16 kernel rounds that fp32 product to fp16)
__device__ __forceinline__ float silu_grad(float da, float x) {
  float ds, inner;
  silu_grad_factors(da, x, ds, inner);
  return ds * inner;
}

template <int DT>
__device__ __forceinline__ float forward_one(float g, float u) {
  using E = Elem<DT>;
  const float a = E::round(silu_value(g));
  return a * u;  // rounded by the caller's store
}

// Generic elementwise forward: any dtype, any alignment.
template <int DT>
__global__ __launch_bounds__(kThreads) void forward_kernel(const typename Elem<DT>::T* __restrict__ g,
                                                           const typename Elem<DT>::T* __restrict__ u,
                                                           typename Elem<DT>::T* __restrict__ h, int64_t n) {
  using E = Elem<DT>;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    E::store(h, i, forward_one<DT>(E::load(g, i), E::load(u, i)));
}

// bf16, 8 values per 16-byte access
__device__ __forceinline__ uint4 forward_chunk(const uint4& gc, const uint4& uc) {
  uint32_t out[4];
  const uint32_t gw[4] = {gc.x, gc.y, gc.z, gc.w}, uw[4] = {uc.x, uc.y, uc.z, uc.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g0 = __uint_as_float(gw[j] << 16), g1 = __uint_as_float(gw[j] & 0xFFFF0000u);
    const float u0 = __uint_as_float(uw[j] << 16), u1 = __uint_as_float(uw[j] & 0xFFFF0000u);
    out[j] = f32x2_to_bf16x2(forward_one<QSTE_BF16>(g0, u0), forward_one<QSTE_BF16>(g1, u1));
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

__global__ __launch_bounds__(kThreads) void forward_bf16x8_kernel(const uint4* __restrict__ g,
                                                                  const uint4* __restrict__ u,
                                                                  uint4* __restrict__ h, int64_t chunks) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; q < chunks;
       q += static_cast<int64_t>(gridDim.x) * kThreads)
    h[q] = forward_chunk(g[q], u[q]);
}

// The forward's table of the rounded silu covers the bf16 gates whose
// magnitude lies in [2^-12, 2^8) (both signs: 2 x 20 binades of 128
// values), wider than the common tables' [2^-12, 2^4): a gate of magnitude
// 16 .. 255 is unusual but not rare enough for the computed path, which
// runs the whole wave through the exponential and the division.
constexpr uint32_t kFwdExps = 20;
constexpr uint32_t kFwdHalf = kFwdExps * 128;
constexpr int kFwdEntries = 2 * kFwdHalf;

__device__ __forceinline__ uint32_t fwd_tab_bits(uint32_t j) {
  const uint32_t neg = j >= kFwdHalf ? 1u : 0u;
  return (neg << 15) | ((kTab16ExpLo << 7) + (j - neg * kFwdHalf));
}

// The rounded silu of bf16 gate bits `bits` (value x): from the table when
// tabulated, else computed the same way the table was filled.
__device__ __forceinline__ float silu_rounded_bf16(uint32_t bits, float x, const uint16_t* tab_a) {
  const uint32_t off = (bits & 0x7FFFu) - (kTab16ExpLo << 7);  // wraps above the range when below it
  return off < kFwdHalf ? bf16_to_f32(tab_a[off + ((bits >> 15) ? kFwdHalf : 0u)])
                        : Elem<QSTE_BF16>::round(silu_value(x));
}

// forward_chunk with the rounded silu looked up
__device__ __forceinline__ uint4 forward_chunk_tab(const uint4& gc, const uint4& uc, const uint16_t* tab_a) {
  uint32_t out[4];
  const uint32_t gw[4] = {gc.x, gc.y, gc.z, gc.w}, uw[4] = {uc.x, uc.y, uc.z, uc.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g0 = __uint_as_float(gw[j] << 16), g1 = __uint_as_float(gw[j] & 0xFFFF0000u);
    const float u0 = __uint_as_float(uw[j] << 16), u1 = __uint_as_float(uw[j] & 0xFFFF0000u);
    const float a0 = silu_rounded_bf16(gw[j] & 0xFFFFu, g0, tab_a);
    const float a1 = silu_rounded_bf16(gw[j] >> 16, g1, tab_a);
    out[j] = f32x2_to_bf16x2(a0 * u0, a1 * u1);
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

// bf16 rows of `stride` 8-value chunks (stride <= CH * kThreads); workgroup
// b takes rows b, b + gridDim.x, ...: h is written and its row encoded from
// the registers.  With TAB the rounded silu of tabulated gates comes from an
// LDS table the workgroup fills once for all its rows (the exponential and
// the correctly rounded division per entry, not per element); without, for
// grids of about one row per workgroup, every element computes it.
template <int CH, bool TAB>
__global__ __launch_bounds__(kThreads) void forward_encode_kernel(const uint16_t* __restrict__ g,
                                                                  const uint16_t* __restrict__ u,
                                                                  uint16_t* __restrict__ h,
                                                                  uint8_t* __restrict__ packed,
                                                                  float* __restrict__ offset,
                                                                  float* __restrict__ scale, int64_t rows,
                                                                  int64_t cols, int64_t stride) {
  __shared__ double red[kThreads / kWave];
  __shared__ uint16_t tab_a[TAB ? kFwdEntries : 1];
  if (TAB) {
    for (int j = threadIdx.x; j < kFwdEntries; j += kThreads) {
      const float x = __uint_as_float(fwd_tab_bits(static_cast<uint32_t>(j)) << 16);
      tab_a[j] = f32_to_bf16(silu_value(x));
    }
    __syncthreads();
  }
  const int t = threadIdx.x;
  // with TAB the grid is four workgroups per CU of one wave per SIMD, the
  // i-th quarter of the grid taking the i-th slot on every CU: a rank per
  // SIMD for the priority rotation (measured 302 -> 288 us at 16384 x 14336)
  int turn = TAB ? static_cast<int>(blockIdx.x / (kEncodeGroups / 4)) : 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    if (TAB) rotate_priority(turn++);
    const uint4* gr = reinterpret_cast<const uint4*>(g + row * cols);
    const uint4* ur = reinterpret_cast<const uint4*>(u + row * cols);
    uint4* hr = reinterpret_cast<uint4*>(h + row * cols);
    uint4 gv[CH], uv[CH], v[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int64_t q = t + static_cast<int64_t>(k) * kThreads;
      gv[k] = q < stride ? gr[q] : make_uint4(0, 0, 0, 0);
      uv[k] = q < stride ? ur[q] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int64_t q = t + static_cast<int64_t>(k) * kThreads;
      v[k] = q >= stride ? make_uint4(0, 0, 0, 0)
                         : TAB ? forward_chunk_tab(gv[k], uv[k], tab_a) : forward_chunk(gv[k], uv[k]);
      if (q < stride) hr[q] = v[k];
    }
    encode_row_chunks<kThreads, CH>(v, packed + row * stride, offset + row, scale + row, cols, stride, red);
  }
}

template <int DT>
__device__ __forceinline__ void backward_one(float dh, float g, float u, float& dg, float& du) {
  using E = Elem<DT>;
  const float a = E::round(silu_value(g));
  du = dh * a;
  const float da = E::round(dh * u);
  dg = silu_grad(da, g);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void backward_kernel(const typename Elem<DT>::T* __restrict__ dh,
                                                            const typename Elem<DT>::T* __restrict__ g,
                                                            const typename Elem<DT>::T* __restrict__ u,
                                                            typename Elem<DT>::T* __restrict__ dg,
                                                            typename Elem<DT>::T* __restrict__ du, int64_t n) {
  using E = Elem<DT>;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    float a, b;
    backward_one<DT>(E::load(dh, i), E::load(g, i), E::load(u, i), a, b);
    E::store(dg, i, a);
    E::store(du, i, b);
  }
}

__global__ __launch_bounds__(kThreads) void backward_bf16x8_kernel(const uint4* __restrict__ dh,
                                                                   const uint4* __restrict__ g,
                                                                   const uint4* __restrict__ u,
                                                                   uint4* __restrict__ dg,
                                                                   uint4* __restrict__ du, int64_t chunks) {
  for (int64_t q = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; q < chunks;
       q += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint4 hc = dh[q], gc = g[q], uc = u[q];
    const uint32_t hw[4] = {hc.x, hc.y, hc.z, hc.w}, gw[4] = {gc.x, gc.y, gc.z, gc.w};
    const uint32_t uw[4] = {uc.x, uc.y, uc.z, uc.w};
    uint32_t og[4], ou[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float dg0, du0, dg1, du1;
      backward_one<QSTE_BF16>(__uint_as_float(hw[j] << 16), __uint_as_float(gw[j] << 16),
                              __uint_as_float(uw[j] << 16), dg0, du0);
      backward_one<QSTE_BF16>(__uint_as_float(hw[j] & 0xFFFF0000u), __uint_as_float(gw[j] & 0xFFFF0000u),
                              __uint_as_float(uw[j] & 0xFFFF0000u), dg1, du1);
      og[j] = f32x2_to_bf16x2(dg0, dg1);
      ou[j] = f32x2_to_bf16x2(du0, du1);
    }
    dg[q] = make_uint4(og[0], og[1], og[2], og[3]);
    du[q] = make_uint4(ou[0], ou[1], ou[2], ou[3]);
  }
}

// Backward plus the column sums the two binary layers before the gate need.
// In a SwiGLU MLP the gate and up projections that produced g and u read one
// input; each layer's backward forms v[c] = sum_t dY[t, c] * offset[t], the
// offset correction of its evidence (functional.py:139-144), by reading its
// dY again.  This pass writes dg and du and sums them as it goes, with the
// chunking and order of colsum_partial_x8_kernel (reduce.hip): chunks of
// kSumChunk samples, kSumWaves waves per chunk each summing a run of
// consecutive samples with fmaf in sample order, the waves' sums added in
// wave order, and the chunk partials [chunk][2][cols] summed in chunk order
// by sum_partials_kernel.  The sums therefore equal, bit for bit, what the
// layers' backward computes from dg and du.
// Lane l of a workgroup owns columns 8 (64 b + l) .. + 7; needs cols % 8 == 0
// and 16-byte aligned operands.
constexpr int kSumChunk = 256;
constexpr int kSumWaves = 4;
constexpr int kSumThreads = kSumWaves * 64;

// bf16 gates in the tabulated range (tab16_index) take sigmoid(g) and the
// rounded silu(g) from LDS tables that the workgroup fills first with the
// arithmetic above, so the exponential and the two correctly rounded
// divisions are paid once per table entry, not once per element; other
// gates compute them.
__device__ __forceinline__ void fill_silu_table(float* tab_s, uint16_t* tab_a, int tid, int threads) {
  for (int j = tid; j < kTab16Entries; j += threads) {
    const float x = __uint_as_float(tab16_bits(static_cast<uint32_t>(j)) << 16);
    tab_a[j] = f32_to_bf16(silu_value(x));
    tab_s[j] = 1.0f / (1.0f + expf(-x));
  }
}

// backward_one with a = the rounded silu(g) and s = sigmoid(g) given
template <int DT>
__device__ __forceinline__ void backward_given(float dh, float g, float u, float a, float s, float& dg,
                                               float& du) {
  using E = Elem<DT>;
  du = dh * a;
  const float da = E::round(dh * u);
  const float inner = fmaf(g, 1.0f - s, 1.0f);
  const float ds = da * s;
  dg = ds * inner;
}

template <int DT>
__device__ __forceinline__ void backward_x8(const uint4& hc, const uint4& gc, const uint4& uc, uint4& og,
                                            uint4& ou, float (&fg)[8], float (&fu)[8], const float* tab_s,
                                            const uint16_t* tab_a) {
  using E = Elem<DT>;
  const uint16_t* h = reinterpret_cast<const uint16_t*>(&hc);
  const uint16_t* g = reinterpret_cast<const uint16_t*>(&gc);
  const uint16_t* u = reinterpret_cast<const uint16_t*>(&uc);
  uint16_t* rg = reinterpret_cast<uint16_t*>(&og);
  uint16_t* ru = reinterpret_cast<uint16_t*>(&ou);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float a, b;
    if constexpr (DT == QSTE_BF16) {
      uint32_t idx;
      if (tab16_index(g[i], idx)) {
        backward_given<DT>(E::load(h, i), E::load(g, i), E::load(u, i), bf16_to_f32(tab_a[idx]), tab_s[idx], a,
                           b);
      } else {
        backward_one<DT>(E::load(h, i), E::load(g, i), E::load(u, i), a, b);
      }
    } else {
      backward_one<DT>(E::load(h, i), E::load(g, i), E::load(u, i), a, b);
    }
    E::store(rg, i, a);
    E::store(ru, i, b);
    fg[i] = E::load(rg, i);  // the stored (rounded) values are what is summed
    fu[i] = E::load(ru, i);
  }
}

template <int DT>
__global__ __launch_bounds__(kSumThreads) void backward_sums_kernel(
    const uint16_t* __restrict__ dh, const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
    uint16_t* __restrict__ dg, uint16_t* __restrict__ du, const float* __restrict__ off_g,
    const float* __restrict__ off_u, int64_t samples, int64_t cols, int64_t ldo, float* __restrict__ part) {
  constexpr int UNROLL = 4;
  constexpr int kPad = 17;
  constexpr int kRed = kSumWaves * 64 * kPad;
  constexpr int kTab = DT == QSTE_BF16 ? kTab16Entries + kTab16Entries / 2 : 0;  // floats: s, then a as bf16
  // the tables while the samples are summed, then the waves' partial sums
  __shared__ float lds[kRed > kTab ? kRed : kTab];
  float* red = lds;
  float* tab_s = lds;
  uint16_t* tab_a = reinterpret_cast<uint16_t*>(lds + kTab16Entries);
  if constexpr (DT == QSTE_BF16) {
    fill_silu_table(tab_s, tab_a, threadIdx.x, kSumThreads);
    __syncthreads();
  }
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 512;
  const int64_t c = base + lane * 8;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kSumChunk;
  const int64_t c1 = c0 + kSumChunk < samples ? c0 + kSumChunk : samples;
  constexpr int kPer = kSumChunk / kSumWaves;
  const int64_t t0 = c0 + wave * kPer < c1 ? c0 + wave * kPer : c1;
  const int64_t t1 = t0 + kPer < c1 ? t0 + kPer : c1;
  float vg[8], vu[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) vg[i] = vu[i] = 0.0f;
  auto one = [&](const uint4& hc, const uint4& gc, const uint4& uc, int64_t t, float og_, float ou_) {
    uint4 rg, ru;
    float fg[8], fu[8];
    backward_x8<DT>(hc, gc, uc, rg, ru, fg, fu, tab_s, tab_a);
    *reinterpret_cast<uint4*>(dg + t * ldo + c) = rg;
    *reinterpret_cast<uint4*>(du + t * ldo + c) = ru;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vg[i] = fmaf(fg[i], og_, vg[i]);
      vu[i] = fmaf(fu[i], ou_, vu[i]);
    }
  };
  if (c < cols) {
    int64_t t = t0;
    for (; t + UNROLL <= t1; t += UNROLL) {
      uint4 hq[UNROLL], gq[UNROLL], uq[UNROLL];
      float og[UNROLL], ou[UNROLL];
#pragma unroll
      for (int k = 0; k < UNROLL; ++k) {
        const int64_t at = (t + k) * cols + c;
        hq[k] = *reinterpret_cast<const uint4*>(dh + at);
        gq[k] = *reinterpret_cast<const uint4*>(g + at);
        uq[k] = *reinterpret_cast<const uint4*>(u + at);
        og[k] = off_g[t + k];
        ou[k] = off_u[t + k];
      }
#pragma unroll
      for (int k = 0; k < UNROLL; ++k) one(hq[k], gq[k], uq[k], t + k, og[k], ou[k]);
    }
    for (; t < t1; ++t) {
      const int64_t at = t * cols + c;
      one(*reinterpret_cast<const uint4*>(dh + at), *reinterpret_cast<const uint4*>(g + at),
          *reinterpret_cast<const uint4*>(u + at), t, off_g[t], off_u[t]);
    }
  }
  __syncthreads();  // every wave is done with the tables
  float* mine = red + (wave * 64 + lane) * kPad;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mine[i] = vg[i];
    mine[8 + i] = vu[i];
  }
  __syncthreads();
  // 1024 results per workgroup (512 columns of the gate sums, then of the up
  // sums), the waves added in order 0..kSumWaves-1
  for (int j = threadIdx.x; j < 2 * 512; j += kSumThreads) {
    const int which = j / 512;
    const int cc = j % 512;
    const int64_t col = base + cc;
    const int slot = (cc / 8) * kPad + which * 8 + cc % 8;
    float sum = red[slot];
#pragma unroll
    for (int w = 1; w < kSumWaves; ++w) sum += red[w * 64 * kPad + slot];
    if (col < cols) part[(static_cast<int64_t>(blockIdx.y) * 2 + which) * cols + col] = sum;
  }
}

inline int grid_of(int64_t work) {
  int64_t b = (work + kThreads - 1) / kThreads;
  if (b > 8192) b = 8192;  // a grid-stride loop covers the rest
  return static_cast<int>(b < 1 ? 1 : b);
}

inline bool aligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace swiglu

int launch_pack_affine_rows(const void*, int, uint8_t*, float*, float*, int64_t, int64_t, hipStream_t);

int launch_swiglu_forward(const void* g, const void* u, int dtype, void* h, uint8_t* packed, float* offset,
                          float* scale, int64_t rows, int64_t cols, hipStream_t s) {
  using namespace swiglu;
  const int64_t n = rows * cols;
  if (n == 0) return 0;
  const int64_t stride = cols / 8;
  const bool vec = dtype == QSTE_BF16 && cols % 8 == 0 && aligned(g) && aligned(u) && aligned(h);
  if (packed && vec && stride <= 8 * kThreads) {
    // with at least kTabRows rows per workgroup of kEncodeGroups, each fills
    // the table once for its rows; fewer rows take a workgroup per row
    const bool tab = rows >= kTabRows * kEncodeGroups;
    const unsigned grid = static_cast<unsigned>(tab ? kEncodeGroups : rows);
    const auto* gp = static_cast<const uint16_t*>(g);
    const auto* upp = static_cast<const uint16_t*>(u);
    auto* hp = static_cast<uint16_t*>(h);
    if (stride <= 2 * kThreads && tab)
      forward_encode_kernel<2, true>
          <<<grid, kThreads, 0, s>>>(gp, upp, hp, packed, offset, scale, rows, cols, stride);
    else if (stride <= 2 * kThreads)
      forward_encode_kernel<2, false>
          <<<grid, kThreads, 0, s>>>(gp, upp, hp, packed, offset, scale, rows, cols, stride);
    else if (tab)
      forward_encode_kernel<8, true>
          <<<grid, kThreads, 0, s>>>(gp, upp, hp, packed, offset, scale, rows, cols, stride);
    else
      forward_encode_kernel<8, false>
          <<<grid, kThreads, 0, s>>>(gp, upp, hp, packed, offset, scale, rows, cols, stride);
    return static_cast<int>(hipGetLastError());
  }
  if (vec) {
    forward_bf16x8_kernel<<<grid_of(n / 8), kThreads, 0, s>>>(static_cast<const uint4*>(g),
                                                               static_cast<const uint4*>(u), static_cast<uint4*>(h),
                                                               n / 8);
  } else {
    switch (dtype) {
      case QSTE_F32:
        forward_kernel<QSTE_F32><<<grid_of(n), kThreads, 0, s>>>(static_cast<const float*>(g),
                                                                 static_cast<const float*>(u),
                                                                 static_cast<float*>(h), n);
        break;
      case QSTE_F16:
        forward_kernel<QSTE_F16><<<grid_of(n), kThreads, 0, s>>>(static_cast<const uint16_t*>(g),
                                                                 static_cast<const uint16_t*>(u),
                                                                 static_cast<uint16_t*>(h), n);
        break;
      default:
        forward_kernel<QSTE_BF16><<<grid_of(n), kThreads, 0, s>>>(static_cast<const uint16_t*>(g),
                                                                  static_cast<const uint16_t*>(u),
                                                                  static_cast<uint16_t*>(h), n);
        break;
    }
  }
  int rc = static_cast<int>(hipGetLastError());
  if (rc || !packed) return rc;
  // rows too wide (or not bf16) for the fused encoding: encode h as written
  return launch_pack_affine_rows(h, dtype, packed, offset, scale, rows, cols, s);
}

int launch_swiglu_backward(const void* dh, const void* g, const void* u, int dtype, void* dg, void* du, int64_t n,
                           hipStream_t s) {
  using namespace swiglu;
  if (n == 0) return 0;
  if (dtype == QSTE_BF16 && n % 8 == 0 && aligned(dh) && aligned(g) && aligned(u) && aligned(dg) && aligned(du)) {
    backward_bf16x8_kernel<<<grid_of(n / 8), kThreads, 0, s>>>(
        static_cast<const uint4*>(dh), static_cast<const uint4*>(g), static_cast<const uint4*>(u),
        static_cast<uint4*>(dg), static_cast<uint4*>(du), n / 8);
    return static_cast<int>(hipGetLastError());
  }
  switch (dtype) {
    case QSTE_F32:
      backward_kernel<QSTE_F32><<<grid_of(n), kThreads, 0, s>>>(
          static_cast<const float*>(dh), static_cast<const float*>(g), static_cast<const float*>(u),
          static_cast<float*>(dg), static_cast<float*>(du), n);
      break;
    case QSTE_F16:
      backward_kernel<QSTE_F16><<<grid_of(n), kThreads, 0, s>>>(
          static_cast<const uint16_t*>(dh), static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
          static_cast<uint16_t*>(dg), static_cast<uint16_t*>(du), n);
      break;
    default:
      backward_kernel<QSTE_BF16><<<grid_of(n), kThreads, 0, s>>>(
          static_cast<const uint16_t*>(dh), static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
          static_cast<uint16_t*>(dg), static_cast<uint16_t*>(du), n);
      break;
  }
  return static_cast<int>(hipGetLastError());
}

int launch_colsums(const void*, int, const float*, int64_t, int64_t, float*, float*, float*, float*, hipStream_t);
int launch_sum_partials(const float*, int64_t, int64_t, float*, hipStream_t);

size_t swiglu_backward_sums_workspace(int64_t rows, int64_t cols) {
  const int64_t chunks = (rows + swiglu::kSumChunk - 1) / swiglu::kSumChunk;
  return static_cast<size_t>(chunks * 2 * cols) * sizeof(float);
}

// sums [2][cols]: sum_t dg[t, c] * off_g[t], then sum_t du[t, c] * off_u[t];
// part: swiglu_backward_sums_workspace(rows, cols) bytes.
int launch_swiglu_backward_sums(const void* dh, const void* g, const void* u, int dtype, void* dg, void* du,
                                const float* off_g, const float* off_u, int64_t rows, int64_t cols, float* sums,
                                float* part, hipStream_t s, int64_t ld_out) {
  using namespace swiglu;
  if (rows * cols == 0) return 0;
  const int64_t chunks = (rows + kSumChunk - 1) / kSumChunk;
  const bool x8 = (dtype == QSTE_BF16 || dtype == QSTE_F16) && cols % 8 == 0 && aligned(dh) && aligned(g) &&
                  aligned(u) && aligned(dg) && aligned(du) && ld_out % 8 == 0;
  // outputs with a row pitch of their own are written by the 8-wide pass only
  if (ld_out != cols && !x8) return QSTE_E_ALIGN;
  if (x8) {
    const dim3 grid(static_cast<unsigned>((cols + 511) / 512), static_cast<unsigned>(chunks));
    if (dtype == QSTE_BF16)
      backward_sums_kernel<QSTE_BF16><<<grid, kSumThreads, 0, s>>>(
          static_cast<const uint16_t*>(dh), static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
          static_cast<uint16_t*>(dg), static_cast<uint16_t*>(du), off_g, off_u, rows, cols, ld_out, part);
    else
      backward_sums_kernel<QSTE_F16><<<grid, kSumThreads, 0, s>>>(
          static_cast<const uint16_t*>(dh), static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
          static_cast<uint16_t*>(dg), static_cast<uint16_t*>(du), off_g, off_u, rows, cols, ld_out, part);
    const int rc = static_cast<int>(hipGetLastError());
    if (rc) return rc;
    return launch_sum_partials(part, chunks, 2 * cols, sums, s);
  }
  // any other dtype or layout: the plain pass, then the layers' own column
  // sums over what it wrote
  int rc = launch_swiglu_backward(dh, g, u, dtype, dg, du, rows * cols, s);
  if (rc) return rc;
  if ((rc = launch_colsums(dg, dtype, off_g, rows, cols, part, nullptr, sums, nullptr, s))) return rc;
  return launch_colsums(du, dtype, off_u, rows, cols, part, nullptr, sums + cols, nullptr, s);
}

}  // namespace qste
