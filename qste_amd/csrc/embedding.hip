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
// ids are sorted stably (a least-significant-digit radix sort written here,
// 8 bits per pass, token index as the value), each
// vocabulary row finds its run of tokens by binary search, and one workgroup
// per vocabulary row sums its tokens' gradient rows in ascending token order
// -- the order of a sequential index_add_, so the fp32 sums are the CPU
// reference's bit for bit -- then forms the scale gradient and the scaled
// evidence in the same pass.  Every row of the evidence is written once
// (zero rows for ids that do not occur).
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

// One wave per vocabulary row r (kRowWaves rows a workgroup), columns spread
// over the lanes, four at a time (16-byte evidence stores) when the layout
// allows.  Each element sums its row's tokens in ascending token order, from
// +0, in fp32.
constexpr int kRowWaves = 4;

template <int DT>
__device__ __forceinline__ void load4(const typename Elem<DT>::T* p, float (&v)[4]) {
  if constexpr (DT == QSTE_F32) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
  } else {
    const uint2 q = *reinterpret_cast<const uint2*>(p);
    const uint16_t h[4] = {static_cast<uint16_t>(q.x), static_cast<uint16_t>(q.x >> 16),
                           static_cast<uint16_t>(q.y), static_cast<uint16_t>(q.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = Elem<DT>::load(h, i);
  }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kRowWaves* kWave) void evidence_rows_kernel(
    const typename Elem<DT>::T* __restrict__ grad, const int32_t* __restrict__ order,
    const int32_t* __restrict__ start, const uint8_t* __restrict__ packed, const float* __restrict__ scale,
    float* __restrict__ evidence, float* __restrict__ grad_scale, int64_t rows, int64_t cols, int64_t pb) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
  if (r >= rows) return;  // the whole wave: no workgroup barrier follows
  const int32_t s0 = start[r];
  const int32_t s1 = start[r + 1];
  const float sr = scale[r];
  const uint8_t* bits = packed + r * pb;
  float* dst = evidence + r * cols;
  double inner = 0.0;
  if constexpr (VEC) {
    for (int64_t c = 4 * lane; c < cols; c += 4 * kWave) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int32_t j = s0; j < s1; ++j) {
        float v[4];
        load4<DT>(grad + static_cast<int64_t>(order[j]) * cols + c, v);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += v[q];
      }
      *reinterpret_cast<float4*>(dst + c) = make_float4(acc[0] * sr, acc[1] * sr, acc[2] * sr, acc[3] * sr);
      const uint32_t byte = bits[c >> 3] >> (c & 7);
#pragma unroll
      for (int q = 0; q < 4; ++q) inner += static_cast<double>(acc[q]) * (((byte >> q) & 1u) ? 1.0 : -1.0);
    }
  } else {
    for (int64_t c = lane; c < cols; c += kWave) {
      float acc = 0.0f;
      for (int32_t j = s0; j < s1; ++j) acc += Elem<DT>::load(grad + static_cast<int64_t>(order[j]) * cols, c);
      inner += static_cast<double>(acc) * static_cast<double>(sign_of(bits, c));
      dst[c] = acc * sr;
    }
  }
  inner = wave_sum(inner);
  if (lane == 0) grad_scale[r] = static_cast<float>(inner);
}

// -- stable LSD radix sort of (key, value) int32 pairs, 8 bits a pass --------
// Each pass: every block of kSortItems consecutive items counts its digits
// (LDS integer atomics: only the counts are kept); one workgroup scans the
// counts digit-major then block-major, giving each (digit, block) its first
// output slot; then every block places its items, kSortThreads at a time in
// item order: an item's slot is its (digit, block) start, plus the items of
// its digit placed by earlier rounds of the block, by earlier waves of this
// round and by lower lanes of its wave (eight ballots match the lanes of one
// digit).  Items keep their order within a digit, so each pass is stable and
// the sort deterministic.
constexpr int kSortThreads = 256;  // one per digit in the count and the scan of a block
constexpr int kSortRounds = 4;
constexpr int kSortItems = kSortThreads * kSortRounds;
constexpr int kSortWaves = kSortThreads / kWave;

__global__ __launch_bounds__(kSortThreads) void digit_count_kernel(const int32_t* __restrict__ keys, int64_t count,
                                                                   int shift, int32_t* __restrict__ counts,
                                                                   int64_t blocks) {
  __shared__ int32_t hist[256];
  hist[threadIdx.x] = 0;
  __syncthreads();
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kSortItems;
  for (int i = threadIdx.x; i < kSortItems; i += kSortThreads) {
    const int64_t n = b0 + i;
    if (n < count) atomicAdd(&hist[(static_cast<uint32_t>(keys[n]) >> shift) & 255u], 1);
  }
  __syncthreads();
  counts[static_cast<int64_t>(threadIdx.x) * blocks + blockIdx.x] = hist[threadIdx.x];
}

// Exclusive scan, in place, of n int32 counts (n % 4 == 0; one workgroup of
// 1024 threads, 4096 counts a tile: four per thread, a wave scan by
// shuffles, the waves' totals through LDS, a running carry between tiles).
constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void scan_counts_kernel(int32_t* __restrict__ counts, int64_t n) {
  __shared__ int32_t wave_total[kScanThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  int32_t carry = 0;
  for (int64_t base = 0; base < n; base += 4 * kScanThreads) {
    const int64_t i = base + 4 * static_cast<int64_t>(threadIdx.x);
    int4 v = make_int4(0, 0, 0, 0);
    if (i < n) v = *reinterpret_cast<const int4*>(counts + i);
    const int32_t own = v.x + v.y + v.z + v.w;
    int32_t incl = own;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int32_t y = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += y;
    }
    if (lane == kWave - 1) wave_total[w] = incl;
    __syncthreads();
    int32_t before = carry + incl - own, tile = 0;
    for (int q = 0; q < kScanThreads / kWave; ++q) {
      const int32_t t = wave_total[q];
      if (q < w) before += t;
      tile += t;
    }
    if (i < n)
      *reinterpret_cast<int4*>(counts + i) =
          make_int4(before, before + v.x, before + v.x + v.y, before + v.x + v.y + v.z);
    carry += tile;
    __syncthreads();  // wave_total is rewritten by the next tile
  }
}

__global__ __launch_bounds__(kSortThreads) void digit_place_kernel(const int32_t* __restrict__ keys_in,
                                                                   const int32_t* __restrict__ vals_in,
                                                                   int32_t* __restrict__ keys_out,
                                                                   int32_t* __restrict__ vals_out, int64_t count,
                                                                   int shift, const int32_t* __restrict__ offsets,
                                                                   int64_t blocks) {
  __shared__ int32_t run[256];                  // next slot of each digit for this block
  __shared__ int32_t wave_count[kSortWaves][256];  // items of each digit in each wave this round
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int w = t / kWave;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kSortItems;
  const int m = static_cast<int>(count - b0 < kSortItems ? count - b0 : kSortItems);
  int32_t key[kSortRounds], val[kSortRounds];
#pragma unroll
  for (int c = 0; c < kSortRounds; ++c) {
    const int i = c * kSortThreads + t;
    key[c] = i < m ? keys_in[b0 + i] : 0;
    val[c] = i < m ? vals_in[b0 + i] : 0;
  }
  run[t] = offsets[static_cast<int64_t>(t) * blocks + blockIdx.x];
#pragma unroll
  for (int c = 0; c < kSortRounds; ++c) {
#pragma unroll
    for (int q = 0; q < kSortWaves; ++q) wave_count[q][t] = 0;
    __syncthreads();
    const bool valid = c * kSortThreads + t < m;
    const uint32_t d = (static_cast<uint32_t>(key[c]) >> shift) & 255u;
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t ones = __ballot((d >> b) & 1u);
      same &= ((d >> b) & 1u) ? ones : ~ones;
    }
    if (valid && (same >> lane) == 1ull) wave_count[w][d] = __popcll(same);  // the digit's highest lane
    __syncthreads();
    if (valid) {
      int32_t at = run[d] + __popcll(same & ((1ull << lane) - 1ull));
      for (int q = 0; q < w; ++q) at += wave_count[q][d];
      keys_out[at] = key[c];
      vals_out[at] = val[c];
    }
    __syncthreads();
    int32_t placed = 0;
#pragma unroll
    for (int q = 0; q < kSortWaves; ++q) placed += wave_count[q][t];
    run[t] += placed;
  }
}

inline int64_t sort_blocks(int64_t count) { return (count + kSortItems - 1) / kSortItems; }

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
  size_t keys_in, keys_out, order_in, order_out, start, counts, total;
};

Layout layout(int64_t count, int64_t rows) {
  Layout l{};
  size_t at = 0;
  const size_t n4 = align_up(sizeof(int32_t) * static_cast<size_t>(count > 0 ? count : 1));
  l.keys_in = at; at += n4;
  l.keys_out = at; at += n4;
  l.order_in = at; at += n4;
  l.order_out = at; at += n4;
  l.start = at; at += align_up(sizeof(int32_t) * static_cast<size_t>(rows + 1));
  l.counts = at; at += align_up(sizeof(int32_t) * 256 * static_cast<size_t>(sort_blocks(count > 0 ? count : 1)));
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
  int32_t* counts = reinterpret_cast<int32_t*>(base + l.counts);
  hipError_t e;
  if (count > 0) {
    keys_kernel<<<ceil_div(count, kThreads), kThreads, 0, s>>>(ids, keys_in, order_in, count, rows);
    if ((e = hipGetLastError()) != hipSuccess) return static_cast<int>(e);
    const int64_t blocks = sort_blocks(count);
    const int bits = key_bits(rows);
    for (int shift = 0; shift < bits; shift += 8) {
      digit_count_kernel<<<static_cast<unsigned>(blocks), kSortThreads, 0, s>>>(keys_in, count, shift, counts,
                                                                               blocks);
      scan_counts_kernel<<<1, kScanThreads, 0, s>>>(counts, 256 * blocks);
      digit_place_kernel<<<static_cast<unsigned>(blocks), kSortThreads, 0, s>>>(keys_in, order_in, keys_out,
                                                                               order_out, count, shift, counts,
                                                                               blocks);
      if ((e = hipGetLastError()) != hipSuccess) return static_cast<int>(e);
      std::swap(keys_in, keys_out);
      std::swap(order_in, order_out);
    }
    // the sorted pairs are in the *_in arrays after the last swap
    std::swap(keys_in, keys_out);
    std::swap(order_in, order_out);
  }
  bounds_kernel<<<ceil_div(rows + 1, kThreads), kThreads, 0, s>>>(keys_out, start, count, rows);
  if ((e = hipGetLastError()) != hipSuccess) return static_cast<int>(e);
  const int64_t pb = (cols + 7) / 8;
  const unsigned row_groups = static_cast<unsigned>((rows + kRowWaves - 1) / kRowWaves);
  const bool vec = cols % 4 == 0 && reinterpret_cast<uintptr_t>(grad) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(evidence) % 16 == 0;
  QSTE_EMB_DT_SWITCH(dtype, {
    const auto* g = static_cast<const typename Elem<DT>::T*>(grad);
    if (vec)
      evidence_rows_kernel<DT, true><<<row_groups, kRowWaves * kWave, 0, s>>>(
          g, order_out, start, packed, scale, evidence, grad_scale, rows, cols, pb);
    else
      evidence_rows_kernel<DT, false><<<row_groups, kRowWaves * kWave, 0, s>>>(
          g, order_out, start, packed, scale, evidence, grad_scale, rows, cols, pb);
  });
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
