// Binary embedding: row lookup into packed signs, and its evidence.
//
// Reference behaviour (BleedingXiko/QSTE):
//   packed_embedding        -- src/qste/kernels/fallback.py:151-155
//                              (out[n] = sign(packed[ids[n]]) * scale[ids[n]])
//   QSTEEmbeddingFn.backward -- src/qste/functional.py:274-286: evidence =
//                              zeros(R, C).index_add_(0, ids, grad), row
//                              inner product with the signs (scale gradient),
//                              then evidence *= scale[r]
//
// The lookup is byte work: one thread per packed byte of an output row writes
// its eight +-scale values.  The backward has no atomics on floats: the token
// ids are sorted stably (rocPRIM radix sort, token index as the value), each
// vocabulary row finds its run of tokens by binary search, and one workgroup
// per vocabulary row sums its tokens' gradient rows in ascending token order
// -- the order of a sequential index_add_, so the fp32 sums are the CPU
// reference's bit for bit -- then forms the scale gradient and the scaled
// evidence in the same pass.  Every row of the evidence is written once
// (zero rows for ids that do not occur).
#include <hipcub/hipcub.hpp>

#include "common.hpp"

namespace qste {
namespace emb {

constexpr int kThreads = 256;

template <int DT>
__global__ void lookup_kernel(const int64_t* __restrict__ ids, const uint8_t* __restrict__ packed,
                              const float* __restrict__ scale, typename Elem<DT>::T* __restrict__ out,
                              int64_t count, int64_t rows, int64_t cols, int64_t pb) {
  const int64_t total = count * pb;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = idx / pb;
    const int64_t b = idx - n * pb;
    const int64_t id = ids[n];
    const bool ok = id >= 0 && id < rows;  // the host rejects bad ids; never read out of bounds
    const uint32_t byte = ok ? packed[id * pb + b] : 0u;
    const float s = ok ? scale[id] : 0.0f;
    const int m = static_cast<int>(cols - b * 8 < 8 ? cols - b * 8 : 8);
    typename Elem<DT>::T* dst = out + n * cols + b * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < m) Elem<DT>::store(dst, j, ((byte >> j) & 1u) ? s : -s);
  }
}

// keys = ids as int32 (an invalid id sorts after every row and is ignored),
// values = token positions
__global__ void keys_kernel(const int64_t* __restrict__ ids, int32_t* __restrict__ keys,
                            int32_t* __restrict__ order, int64_t count, int64_t rows) {
  const int64_t n = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (n >= count) return;
  const int64_t id = ids[n];
  keys[n] = (id >= 0 && id < rows) ? static_cast<int32_t>(id) : static_cast<int32_t>(rows);
  order[n] = static_cast<int32_t>(n);
}

// start[r] = first position of key r in the sorted keys (lower bound), for
// r in [0, rows]; the run of row r is [start[r], start[r + 1]).
__global__ void bounds_kernel(const int32_t* __restrict__ sorted, int32_t* __restrict__ start,
                              int64_t count, int64_t rows) {
  const int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (r > rows) return;
  int64_t lo = 0, hi = count;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (sorted[mid] < r) lo = mid + 1;
    else hi = mid;
  }
  start[r] = static_cast<int32_t>(lo);
}

// One workgroup per vocabulary row r; columns spread over the threads.
template <int DT>
__global__ __launch_bounds__(kThreads) void evidence_rows_kernel(
    const typename Elem<DT>::T* __restrict__ grad, const int32_t* __restrict__ order,
    const int32_t* __restrict__ start, const uint8_t* __restrict__ packed, const float* __restrict__ scale,
    float* __restrict__ evidence, float* __restrict__ grad_scale, int64_t cols, int64_t pb) {
  __shared__ double red[kThreads / kWave];
  const int64_t r = blockIdx.x;
  const int32_t s0 = start[r];
  const int32_t s1 = start[r + 1];
  const float sr = scale[r];
  const uint8_t* bits = packed + r * pb;
  float* dst = evidence + r * cols;
  double inner = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    float acc = 0.0f;
    for (int32_t j = s0; j < s1; ++j) acc += Elem<DT>::load(grad + static_cast<int64_t>(order[j]) * cols, c);
    inner += static_cast<double>(acc) * static_cast<double>(sign_of(bits, c));
    dst[c] = acc * sr;
  }
  inner = block_sum(inner, red);
  if (threadIdx.x == 0) grad_scale[r] = static_cast<float>(inner);
}

inline int grid_for(int64_t items) {
  int64_t blocks = (items + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  return static_cast<int>(blocks < 1 ? 1 : blocks);
}

inline size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

int key_bits(int64_t rows) {
  int bits = 1;
  while ((int64_t{1} << bits) <= rows) ++bits;  // keys lie in [0, rows]
  return bits;
}

struct Layout {
  size_t keys_in, keys_out, order_in, order_out, start, sort_tmp, sort_bytes, total;
};

Layout layout(int64_t count, int64_t rows) {
  Layout l{};
  size_t sort_bytes = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<const int32_t*>(nullptr),
                                     static_cast<int32_t*>(nullptr), static_cast<const int32_t*>(nullptr),
                                     static_cast<int32_t*>(nullptr), static_cast<int>(count), 0,
                                     key_bits(rows));
  size_t at = 0;
  const size_t n4 = align_up(sizeof(int32_t) * static_cast<size_t>(count > 0 ? count : 1));
  l.keys_in = at; at += n4;
  l.keys_out = at; at += n4;
  l.order_in = at; at += n4;
  l.order_out = at; at += n4;
  l.start = at; at += align_up(sizeof(int32_t) * static_cast<size_t>(rows + 1));
  l.sort_tmp = at; at += align_up(sort_bytes > 0 ? sort_bytes : 1);
  l.sort_bytes = sort_bytes;
  l.total = at;
  return l;
}

inline bool dtype_ok(int d) { return d == QSTE_F32 || d == QSTE_F16 || d == QSTE_BF16; }

}  // namespace emb
}  // namespace qste

using namespace qste;
using namespace qste::emb;

#define QSTE_EMB_DT_SWITCH(dtype, ...)                                    \
  switch (dtype) {                                                       \
    case QSTE_F32: { constexpr int DT = QSTE_F32; __VA_ARGS__; } break;  \
    case QSTE_F16: { constexpr int DT = QSTE_F16; __VA_ARGS__; } break;  \
    case QSTE_BF16: { constexpr int DT = QSTE_BF16; __VA_ARGS__; } break; \
    default: return QSTE_E_DTYPE;                                        \
  }

extern "C" {

int qste_packed_embedding(const int64_t* ids, int64_t count, const uint8_t* packed, const float* scale,
                          void* out, int out_dtype, int64_t rows, int64_t cols, void* stream) {
  if (!emb::dtype_ok(out_dtype)) return QSTE_E_DTYPE;
  if (count < 0 || rows < 0 || cols < 0) return QSTE_E_SHAPE;
  const int64_t pb = (cols + 7) / 8;
  if (count * pb == 0) return 0;
  if (!ids || !packed || !scale || !out) return QSTE_E_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QSTE_EMB_DT_SWITCH(out_dtype, lookup_kernel<DT><<<grid_for(count * pb), kThreads, 0, s>>>(
                                    ids, packed, scale, static_cast<typename Elem<DT>::T*>(out), count,
                                    rows, cols, pb));
  return static_cast<int>(hipGetLastError());
}

size_t qste_embedding_backward_workspace_bytes(int64_t count, int64_t rows) {
  if (count < 0 || rows < 0 || count > INT32_MAX || rows >= INT32_MAX) return 0;
  return layout(count, rows).total;
}

int qste_embedding_backward(const int64_t* ids, int64_t count, const void* grad, int dtype,
                            const uint8_t* packed, const float* scale, float* evidence, float* grad_scale,
                            int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (!emb::dtype_ok(dtype)) return QSTE_E_DTYPE;
  if (count < 0 || rows <= 0 || cols <= 0 || count > INT32_MAX || rows >= INT32_MAX) return QSTE_E_SHAPE;
  if (!packed || !scale || !evidence || !grad_scale || (count > 0 && (!ids || !grad))) return QSTE_E_NULL;
  const Layout l = layout(count, rows);
  if (!workspace || workspace_bytes < l.total) return QSTE_E_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(workspace);
  int32_t* keys_in = reinterpret_cast<int32_t*>(base + l.keys_in);
  int32_t* keys_out = reinterpret_cast<int32_t*>(base + l.keys_out);
  int32_t* order_in = reinterpret_cast<int32_t*>(base + l.order_in);
  int32_t* order_out = reinterpret_cast<int32_t*>(base + l.order_out);
  int32_t* start = reinterpret_cast<int32_t*>(base + l.start);
  hipError_t e;
  if (count > 0) {
    keys_kernel<<<ceil_div(count, kThreads), kThreads, 0, s>>>(ids, keys_in, order_in, count, rows);
    if ((e = hipGetLastError()) != hipSuccess) return static_cast<int>(e);
    size_t sort_bytes = l.sort_bytes;
    e = hipcub::DeviceRadixSort::SortPairs(base + l.sort_tmp, sort_bytes, keys_in, keys_out, order_in, order_out,
                                           static_cast<int>(count), 0, key_bits(rows), s);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  bounds_kernel<<<ceil_div(rows + 1, kThreads), kThreads, 0, s>>>(keys_out, start, count, rows);
  if ((e = hipGetLastError()) != hipSuccess) return static_cast<int>(e);
  const int64_t pb = (cols + 7) / 8;
  QSTE_EMB_DT_SWITCH(dtype, evidence_rows_kernel<DT><<<static_cast<unsigned>(rows), kThreads, 0, s>>>(
                                static_cast<const typename Elem<DT>::T*>(grad), order_out, start, packed, scale,
                                evidence, grad_scale, cols, pb));
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
