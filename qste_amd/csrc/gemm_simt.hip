// Generic tiled products over packed signs, fp32 accumulation on the VALU.
//
// This family takes every dtype and every shape (ragged widths, widths that
// are not a multiple of 64, fp32 activations).  bf16 / fp16 operands at
// MFMA-friendly shapes go to gemm_mfma.hip instead.
//
//   forward   y[m, n]  = (sum_k x[m, k] * sign_w[n, k]) * scale[n] + bias[n]
//             (fallback.py:95-108, epilogue applied in fp32 after the sum)
//   dgrad     dx[m, n] = sum_k dy[m, k] * rnd(scale[k]) * sign_w[k, n]
//             (fallback.py:111-123; rnd rounds the folded scale to the
//             operand dtype as cuda.py:1585-1586 does; identity for fp32)
//   evidence  E[m, n]  = sum_k dy[k, m] * rnd(xs[k]) * sign_x[k, n]
//             (fallback.py:126-138) with an optional fused epilogue:
//             + v[m] (offset correction, functional.py:139-144),
//             partial row inner products against sign_w (packed_row_inner,
//             fallback.py:141-148), then * scale[m] (functional.py:190).
#include "common.hpp"

namespace qste {

constexpr int kTM = 64, kTN = 64, kTK = 16, kThreads = 256;

enum AMode { A_MK = 0, A_KM = 1 };      // A[m][k] at a[m*lda+k] or a[k*lda+m]
enum BMode { B_BITS_NK = 0, B_BITS_KN = 1 };  // sign bits of row n (col k) or row k (col n)

struct SimtArgs {
  const void* a;
  int64_t lda;
  const uint8_t* bits;
  int64_t bits_stride;
  const float* k_scale;   // per-k folded scale (B_BITS_KN), may be null
  void* out;
  int64_t ldo;
  int64_t M, N, K;
  // epilogue
  const float* n_scale;   // forward: scale[n]
  const float* n_bias;    // forward: bias[n]
  const float* m_add;     // evidence: + v[m]
  const float* m_scale;   // evidence: * scale[m] after the row inner product
  const uint8_t* w_bits;  // evidence: sign_w for the row inner product
  int64_t w_stride;
  float* gs_partial;      // evidence: [n_tiles][M]
};

template <int DT, int AM, int BM, int EPI>
__global__ __launch_bounds__(kThreads) void simt_gemm_kernel(SimtArgs p) {
  using E = Elem<DT>;
  __shared__ float As[kTK][kTM + 4];
  __shared__ float Bs[kTK][kTN + 4];
  __shared__ float red[kTM][17];

  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kTM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kTN;
  const typename E::T* A = static_cast<const typename E::T*>(p.a);

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

  for (int64_t k0 = 0; k0 < p.K; k0 += kTK) {
    // A tile: 64 x 16 values, 4 per thread
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * kThreads;
      int mm, kk;
      if (AM == A_MK) { mm = idx / kTK; kk = idx % kTK; } else { kk = idx / kTM; mm = idx % kTM; }
      const int64_t gm = m0 + mm, gk = k0 + kk;
      float v = 0.0f;
      if (gm < p.M && gk < p.K) v = (AM == A_MK) ? E::load(A, gm * p.lda + gk) : E::load(A, gk * p.lda + gm);
      As[kk][mm] = v;
    }
    // B tile: 16 x 64 signs, 4 per thread
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * kThreads;
      int nn, kk;
      if (BM == B_BITS_NK) { nn = idx / kTK; kk = idx % kTK; } else { kk = idx / kTN; nn = idx % kTN; }
      const int64_t gn = n0 + nn, gk = k0 + kk;
      float v = 0.0f;
      if (gn < p.N && gk < p.K) {
        if (BM == B_BITS_NK) {
          v = sign_of(p.bits + gn * p.bits_stride, gk);
        } else {
          v = sign_of(p.bits + gk * p.bits_stride, gn);
          if (p.k_scale) v *= E::round(p.k_scale[gk]);
        }
      }
      Bs[kk][nn] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kTK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }

  // epilogue
  if (EPI == 0) {  // forward / dgrad: optional n-scale and n-bias, dtype store
    typename E::T* out = static_cast<typename E::T*>(p.out);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t gm = m0 + ty * 4 + i;
      if (gm >= p.M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t gn = n0 + tx * 4 + j;
        if (gn >= p.N) continue;
        float v = acc[i][j];
        if (p.n_scale) v = v * p.n_scale[gn];
        if (p.n_bias) v = v + p.n_bias[gn];
        E::store(out, gm * p.ldo + gn, v);
      }
    }
  } else {  // evidence: fp32 output with the fused row epilogue
    float* out = static_cast<float*>(p.out);
    float rowpart[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t gm = m0 + ty * 4 + i;
      if (gm >= p.M) continue;
      const float add = p.m_add ? p.m_add[gm] : 0.0f;
      const float mul = p.m_scale ? p.m_scale[gm] : 1.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t gn = n0 + tx * 4 + j;
        if (gn >= p.N) continue;
        const float e0 = acc[i][j] + add;
        if (p.w_bits) rowpart[i] += e0 * sign_of(p.w_bits + gm * p.w_stride, gn);
        out[gm * p.ldo + gn] = e0 * mul;
      }
    }
    if (p.gs_partial) {
#pragma unroll
      for (int i = 0; i < 4; ++i) red[ty * 4 + i][tx] = rowpart[i];
      __syncthreads();
      if (tid < kTM) {
        float s = 0.0f;
        for (int j = 0; j < 16; ++j) s += red[tid][j];
        const int64_t gm = m0 + tid;
        if (gm < p.M) p.gs_partial[static_cast<int64_t>(blockIdx.x) * p.M + gm] = s;
      }
    }
  }
}

template <int DT, int AM, int BM, int EPI>
static int launch_simt(const SimtArgs& p, hipStream_t stream) {
  dim3 grid(ceil_div(p.N, kTN), ceil_div(p.M, kTM));
  simt_gemm_kernel<DT, AM, BM, EPI><<<grid, kThreads, 0, stream>>>(p);
  return static_cast<int>(hipGetLastError());
}

#define QSTE_DISPATCH_DT(dtype, CALL)            \
  switch (dtype) {                               \
    case QSTE_F32: { constexpr int DT = QSTE_F32; CALL; } \
    case QSTE_F16: { constexpr int DT = QSTE_F16; CALL; } \
    case QSTE_BF16: { constexpr int DT = QSTE_BF16; CALL; } \
    default: return QSTE_E_DTYPE;                \
  }

int simt_linear_forward(const void* x, int dtype, const uint8_t* packed, const float* scale,
                        const float* bias, void* y, int64_t m, int64_t rows, int64_t cols,
                        hipStream_t stream) {
  SimtArgs p{};
  p.a = x; p.lda = cols; p.bits = packed; p.bits_stride = (cols + 7) / 8;
  p.out = y; p.ldo = rows; p.M = m; p.N = rows; p.K = cols;
  p.n_scale = scale; p.n_bias = bias;
  QSTE_DISPATCH_DT(dtype, return (launch_simt<DT, A_MK, B_BITS_NK, 0>(p, stream)));
}

int simt_linear_dgrad(const void* dy, int dtype, const uint8_t* packed, const float* row_scale,
                      void* dx, int64_t m, int64_t rows, int64_t cols, hipStream_t stream) {
  SimtArgs p{};
  p.a = dy; p.lda = rows; p.bits = packed; p.bits_stride = (cols + 7) / 8; p.k_scale = row_scale;
  p.out = dx; p.ldo = cols; p.M = m; p.N = cols; p.K = rows;
  QSTE_DISPATCH_DT(dtype, return (launch_simt<DT, A_MK, B_BITS_KN, 0>(p, stream)));
}

int simt_evidence(const void* dy, int dtype, const uint8_t* packed_x, const float* x_scale,
                  float* evidence, int64_t samples, int64_t rows, int64_t cols,
                  const float* m_add, const float* m_scale, const uint8_t* w_bits,
                  float* gs_partial, hipStream_t stream) {
  SimtArgs p{};
  p.a = dy; p.lda = rows; p.bits = packed_x; p.bits_stride = (cols + 7) / 8; p.k_scale = x_scale;
  p.out = evidence; p.ldo = cols; p.M = rows; p.N = cols; p.K = samples;
  p.m_add = m_add; p.m_scale = m_scale; p.w_bits = w_bits; p.w_stride = (cols + 7) / 8;
  p.gs_partial = gs_partial;
  QSTE_DISPATCH_DT(dtype, return (launch_simt<DT, A_KM, B_BITS_KN, 1>(p, stream)));
}

int simt_evidence_tiles(int64_t cols) { return ceil_div(cols, kTN); }

}  // namespace qste
