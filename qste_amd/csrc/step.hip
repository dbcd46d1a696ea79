// The fused QSTE coordinate step (spec: src/qste/kernels/fallback.py:158-242).
//
// The step has three global dependencies -- the factored row/column second
// moments, the global RMS of the normalized update, and the global RMS of
// the new momentum -- so it runs as a short chain of passes over the fp32
// evidence, none of which writes the evidence:
//
//   stats     row and column sums of g^2 + 1e-12         -> row_part, col_part
//   cols      column EMA, fp16 col_v, column factor       (one thread/column)
//   rows      row EMA, fp16 row_v, mean row statistic, row factor (1 group)
//   usq       sum of U^2, U = g * rf * cf                 -> usq_part
//   scalars   RMS clip divisor
//   moment    m = q*S*b1 + (1-b1)*U/div per block: new fp16 scale, sum m^2
//   scalars   coordinate step size lr / rms(m)
//   final     stochastic rounding, momentum requantization, sign repack,
//             flip count (one thread per packed byte)
//   finish    new block scales into place, flip total
//
// Float semantics follow the specification operation by operation: every
// element-wise product and sum rounds in fp32 (this file is compiled with
// -ffp-contract=off), torch's `add_(x, alpha=a)` is a fused multiply-add
// (fmaf), divisions and square roots are correctly rounded.  Reductions
// accumulate in double in a fixed order and round once, so the result does
// not depend on launch geometry and equals the correctly rounded sum but in
// vanishingly rare cases.
#include "common.hpp"

namespace qste {

namespace step {

constexpr int kThreads = 256;
constexpr int kChunkCols = 1024;  // columns per stats workgroup (4 per thread)
constexpr int kStrip = 64;        // rows per stats workgroup
constexpr int kUsqGroups = 1024;
constexpr int kMomentGroups = 1024;

struct Params {
  float b1, a1, b2, a2, clip, lr;
  int64_t rows, cols, count, blocks, block_size;
  int block_shift;
  uint32_t seed_part;
  int64_t step;
  const int64_t* step_device;
  const uint8_t* enabled;
};

struct Work {
  double* row_part;   // [nchunks][rows]
  double* col_part;   // [nstrips][cols]
  float* new_row;     // [rows]
  float* row_factor;  // [rows]
  float* new_col;     // [cols]
  float* col_factor;  // [cols]
  double* usq_part;   // [kUsqGroups]
  double* msq_part;   // [kMomentGroups * waves]
  float* scalars;     // [0] divisor, [1] step size
  uint16_t* s_new;    // [blocks]
  int64_t* flips_part;// [final groups]
  int64_t nchunks, nstrips, final_groups;
};

__device__ __forceinline__ bool enabled(const Params& p) {
  return p.enabled == nullptr || *p.enabled != 0;
}

// -- stats -------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void stats_kernel(const float* __restrict__ g, Params p,
                                                         Work w) {
  __shared__ double red[kStrip][kThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t chunk = blockIdx.x;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kStrip;
  const int64_t c0 = chunk * kChunkCols + threadIdx.x * 4;
  const float eps = 1e-12f;
  double col_acc[4] = {0.0, 0.0, 0.0, 0.0};
  const int rows_here = static_cast<int>(p.rows - r0 < kStrip ? p.rows - r0 : kStrip);
  for (int rr = 0; rr < rows_here; ++rr) {
    const float* line = g + (r0 + rr) * p.cols;
    double rp = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = c0 + j;
      if (c < p.cols) {
        const float v = line[c];
        float sq = v * v;
        sq = sq + eps;
        col_acc[j] += static_cast<double>(sq);
        rp += static_cast<double>(sq);
      }
    }
    rp = wave_sum(rp);
    if (lane == 0) red[rr][wave] = rp;
  }
  __syncthreads();
  if (threadIdx.x < rows_here) {
    double s = 0.0;
    for (int k = 0; k < kThreads / kWave; ++k) s += red[threadIdx.x][k];
    w.row_part[chunk * p.rows + r0 + threadIdx.x] = s;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c = c0 + j;
    if (c < p.cols) w.col_part[static_cast<int64_t>(blockIdx.y) * p.cols + c] = col_acc[j];
  }
}

// -- column and row statistics ----------------------------------------------
__global__ void cols_kernel(uint16_t* __restrict__ col_v, Params p, Work w) {
  const int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (c >= p.cols) return;
  double s = 0.0;
  for (int64_t k = 0; k < w.nstrips; ++k) s += w.col_part[k * p.cols + c];
  const float mean = static_cast<float>(s) / static_cast<float>(p.rows);
  const float decayed = f16_to_f32(col_v[c]) * p.b2;
  const float nc = fmaf(mean, p.a2, decayed);
  w.new_col[c] = nc;
  w.col_factor[c] = 1.0f / sqrtf(fmaxf(nc, 1e-10f));
  if (enabled(p)) col_v[c] = f32_to_f16(nc);
}

__global__ __launch_bounds__(1024) void rows_kernel(uint16_t* __restrict__ row_v, Params p, Work w) {
  __shared__ double red[1024 / kWave];
  double acc = 0.0;
  const bool on = enabled(p);
  for (int64_t r = threadIdx.x; r < p.rows; r += blockDim.x) {
    double s = 0.0;
    for (int64_t k = 0; k < w.nchunks; ++k) s += w.row_part[k * p.rows + r];
    const float mean = static_cast<float>(s) / static_cast<float>(p.cols);
    const float decayed = f16_to_f32(row_v[r]) * p.b2;
    const float nr = fmaf(mean, p.a2, decayed);
    w.new_row[r] = nr;
    acc += static_cast<double>(fmaxf(nr, 1e-10f));
    if (on) row_v[r] = f32_to_f16(nr);
  }
  acc = block_sum(acc, red);
  const float sqrt_mean = sqrtf(static_cast<float>(acc) / static_cast<float>(p.rows));
  for (int64_t r = threadIdx.x; r < p.rows; r += blockDim.x)
    w.row_factor[r] = sqrt_mean / sqrtf(fmaxf(w.new_row[r], 1e-10f));
}

// -- update RMS ---------------------------------------------------------------
__device__ __forceinline__ float normalized(float g, float rf, float cf) {
  float u = g * rf;
  u = u * cf;
  return u;
}

__global__ __launch_bounds__(kThreads) void usq_kernel(const float* __restrict__ g, Params p,
                                                       Work w) {
  __shared__ double red[kThreads / kWave];
  double acc = 0.0;
  for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const float rf = w.row_factor[r];
    const float* line = g + r * p.cols;
    for (int64_t c = threadIdx.x; c < p.cols; c += kThreads) {
      const float u = normalized(line[c], rf, w.col_factor[c]);
      const float s = u * u;
      acc += static_cast<double>(s);
    }
  }
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) w.usq_part[blockIdx.x] = acc;
}

__global__ __launch_bounds__(kThreads) void divisor_kernel(Params p, Work w, int64_t parts) {
  __shared__ double red[kThreads / kWave];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < parts; i += kThreads) acc += w.usq_part[i];
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) {
    float rms = sqrtf(static_cast<float>(acc) / static_cast<float>(p.count));
    rms = fmaxf(rms, 1e-8f);
    const float ratio = rms / p.clip;
    w.scalars[0] = ratio > 1.0f ? ratio : 1.0f;
  }
}

// -- momentum -------------------------------------------------------------------
__device__ __forceinline__ float moment_of(float g, float rf, float cf, float divisor, float prev,
                                           float s_old, const Params& p) {
  const float u = normalized(g, rf, cf) / divisor;
  float decoded = prev * s_old;
  decoded = decoded * p.b1;
  return fmaf(u, p.a1, decoded);
}

// One wave per momentum block at a time; lanes stride the block's elements.
__global__ __launch_bounds__(kThreads) void moment_kernel(const float* __restrict__ g,
                                                          const int8_t* __restrict__ moment_q,
                                                          const uint16_t* __restrict__ moment_scale,
                                                          Params p, Work w) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  const float divisor = w.scalars[0];
  double msq = 0.0;
  for (int64_t b = wave_id; b < p.blocks; b += waves) {
    const float s_old = f16_to_f32(moment_scale[b]);
    float amax = 0.0f;
    for (int64_t j = lane; j < p.block_size; j += kWave) {
      const int64_t i = b * p.block_size + j;
      float m = 0.0f;
      if (i < p.count) {
        const int64_t r = i / p.cols;
        const int64_t c = i - r * p.cols;
        m = moment_of(g[i], w.row_factor[r], w.col_factor[c], divisor,
                      static_cast<float>(moment_q[i]), s_old, p);
      }
      amax = fmaxf(amax, fabsf(m));
      const float s = m * m;
      msq += static_cast<double>(s);
    }
    amax = wave_max(amax);
    if (lane == 0) w.s_new[b] = f32_to_f16(fmaxf(amax, 1e-6f) / 127.0f);
  }
  msq = wave_sum(msq);
  if (lane == 0) w.msq_part[wave_id] = msq;
}

__global__ __launch_bounds__(kThreads) void step_size_kernel(Params p, Work w, int64_t parts) {
  __shared__ double red[kThreads / kWave];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < parts; i += kThreads) acc += w.msq_part[i];
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) {
    const float padded = static_cast<float>(p.blocks * p.block_size);
    float mrms = sqrtf(static_cast<float>(acc) / padded);
    mrms = fmaxf(mrms, 1e-8f);
    w.scalars[1] = p.lr / mrms;
  }
}

// -- final element pass -------------------------------------------------------
__global__ __launch_bounds__(kThreads) void final_kernel(const float* __restrict__ g,
                                                         int8_t* __restrict__ coord,
                                                         uint8_t* __restrict__ packed,
                                                         int8_t* __restrict__ moment_q,
                                                         const uint16_t* __restrict__ moment_scale,
                                                         Params p, Work w) {
  __shared__ int64_t red[kThreads / kWave];
  const int64_t stride = (p.cols + 7) / 8;
  const int64_t total = p.rows * stride;
  const int64_t idx = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const float divisor = w.scalars[0];
  const float step_size = w.scalars[1];
  const int64_t step = p.step_device ? *p.step_device : p.step;
  const uint32_t combined = p.seed_part ^ step_hash(step);
  const bool on = enabled(p);
  int64_t flips = 0;
  if (idx < total) {
    const int64_t r = idx / stride;
    const int64_t b = idx - r * stride;
    const int64_t c0 = b * 8;
    const int n = static_cast<int>(p.cols - c0 < 8 ? p.cols - c0 : 8);
    const float rf = w.row_factor[r];
    uint32_t byte = 0;
    int8_t cnew[8], qnew[8];
    for (int j = 0; j < n; ++j) {
      const int64_t c = c0 + j;
      const int64_t i = r * p.cols + c;
      const int64_t blk = i >> p.block_shift;
      const float m = moment_of(g[i], rf, w.col_factor[c], divisor,
                                static_cast<float>(moment_q[i]), f16_to_f32(moment_scale[blk]), p);
      const float delta = m * step_size;
      const float target = static_cast<float>(coord[i]) - delta;
      const float lower = floorf(target);
      const float u = static_cast<float>(scramble(static_cast<uint32_t>(static_cast<uint64_t>(i)) ^ combined)) *
                      (1.0f / 4294967296.0f);
      const float frac = target - lower;
      float rounded = lower + (u < frac ? 1.0f : 0.0f);
      rounded = fminf(127.0f, fmaxf(-127.0f, rounded));
      cnew[j] = static_cast<int8_t>(rounded);
      const float decode = fmaxf(f16_to_f32(w.s_new[blk]), 1e-12f);
      float q = rintf(m / decode);
      q = fminf(127.0f, fmaxf(-127.0f, q));
      qnew[j] = static_cast<int8_t>(q);
      byte |= (rounded >= 0.0f ? 1u : 0u) << j;
    }
    const uint32_t mask = n >= 8 ? 0xFFu : ((1u << n) - 1u);
    flips = __popc((static_cast<uint32_t>(packed[idx]) ^ byte) & mask);
    if (on) {
      for (int j = 0; j < n; ++j) {
        const int64_t i = r * p.cols + c0 + j;
        coord[i] = cnew[j];
        moment_q[i] = qnew[j];
      }
      packed[idx] = static_cast<uint8_t>(byte);
    }
  }
  flips = block_sum(flips, red);
  if (threadIdx.x == 0) w.flips_part[blockIdx.x] = on ? flips : 0;
}

__global__ __launch_bounds__(kThreads) void finish_kernel(uint16_t* __restrict__ moment_scale,
                                                          int64_t* __restrict__ flips_out, Params p,
                                                          Work w) {
  __shared__ int64_t red[kThreads / kWave];
  if (enabled(p)) {
    for (int64_t b = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; b < p.blocks;
         b += static_cast<int64_t>(gridDim.x) * kThreads)
      moment_scale[b] = w.s_new[b];
  }
  if (blockIdx.x == 0 && flips_out) {
    int64_t acc = 0;
    for (int64_t i = threadIdx.x; i < w.final_groups; i += kThreads) acc += w.flips_part[i];
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) *flips_out = acc;
  }
}

// -- plan ------------------------------------------------------------------------
struct Layout {
  size_t off[11];
  size_t total;
};

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static Layout layout(int64_t rows, int64_t cols, int64_t block_size, Work* w) {
  const int64_t nchunks = (cols + kChunkCols - 1) / kChunkCols;
  const int64_t nstrips = (rows + kStrip - 1) / kStrip;
  const int64_t count = rows * cols;
  const int64_t blocks = (count + block_size - 1) / block_size;
  const int64_t stride = (cols + 7) / 8;
  const int64_t final_groups = (rows * stride + kThreads - 1) / kThreads;
  const size_t sizes[11] = {
      sizeof(double) * static_cast<size_t>(nchunks * rows),
      sizeof(double) * static_cast<size_t>(nstrips * cols),
      sizeof(float) * static_cast<size_t>(rows),
      sizeof(float) * static_cast<size_t>(rows),
      sizeof(float) * static_cast<size_t>(cols),
      sizeof(float) * static_cast<size_t>(cols),
      sizeof(double) * kUsqGroups,
      sizeof(double) * kMomentGroups * (kThreads / kWave),
      sizeof(float) * 4,
      sizeof(uint16_t) * static_cast<size_t>(blocks),
      sizeof(int64_t) * static_cast<size_t>(final_groups > 0 ? final_groups : 1),
  };
  Layout l{};
  size_t at = 0;
  for (int i = 0; i < 11; ++i) {
    l.off[i] = at;
    at += align_up(sizes[i]);
  }
  l.total = at;
  if (w) {
    w->nchunks = nchunks;
    w->nstrips = nstrips;
    w->final_groups = final_groups;
  }
  return l;
}

}  // namespace step

size_t coordinate_update_workspace(int64_t rows, int64_t cols, int64_t block_size) {
  if (rows <= 0 || cols <= 0 || block_size <= 0) return 0;
  return step::layout(rows, cols, block_size, nullptr).total;
}

int launch_coordinate_update(const float* g, int8_t* coord, uint8_t* packed, int8_t* moment_q,
                             uint16_t* moment_scale, uint16_t* row_v, uint16_t* col_v, int64_t rows,
                             int64_t cols, double beta1, double beta2, double update_clip,
                             double coordinate_lr, int64_t block_size, int64_t seed, int64_t step_,
                             const int64_t* step_device, int64_t* flips_out,
                             const uint8_t* update_enabled, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  using namespace step;
  if (rows == 0 || cols == 0) return 0;  // the C entry handles empty surfaces
  Work w{};
  const Layout l = layout(rows, cols, block_size, &w);
  if (workspace_bytes < l.total || workspace == nullptr) return QSTE_E_WORKSPACE;
  char* base = static_cast<char*>(workspace);
  w.row_part = reinterpret_cast<double*>(base + l.off[0]);
  w.col_part = reinterpret_cast<double*>(base + l.off[1]);
  w.new_row = reinterpret_cast<float*>(base + l.off[2]);
  w.row_factor = reinterpret_cast<float*>(base + l.off[3]);
  w.new_col = reinterpret_cast<float*>(base + l.off[4]);
  w.col_factor = reinterpret_cast<float*>(base + l.off[5]);
  w.usq_part = reinterpret_cast<double*>(base + l.off[6]);
  w.msq_part = reinterpret_cast<double*>(base + l.off[7]);
  w.scalars = reinterpret_cast<float*>(base + l.off[8]);
  w.s_new = reinterpret_cast<uint16_t*>(base + l.off[9]);
  w.flips_part = reinterpret_cast<int64_t*>(base + l.off[10]);

  Params p{};
  p.b1 = static_cast<float>(beta1);
  p.a1 = static_cast<float>(1.0 - beta1);
  p.b2 = static_cast<float>(beta2);
  p.a2 = static_cast<float>(1.0 - beta2);
  p.clip = static_cast<float>(update_clip);
  p.lr = static_cast<float>(coordinate_lr);
  p.rows = rows;
  p.cols = cols;
  p.count = rows * cols;
  p.block_size = block_size;
  p.blocks = (p.count + block_size - 1) / block_size;
  int shift = 0;
  while ((int64_t{1} << shift) < block_size) ++shift;
  p.block_shift = shift;
  p.seed_part = seed_hash(seed);
  p.step = step_;
  p.step_device = step_device;
  p.enabled = update_enabled;

  int rc;
  stats_kernel<<<dim3(static_cast<unsigned>(w.nchunks), static_cast<unsigned>(w.nstrips)), kThreads, 0,
                 stream>>>(g, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  cols_kernel<<<ceil_div(cols, 256), 256, 0, stream>>>(col_v, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  rows_kernel<<<1, 1024, 0, stream>>>(row_v, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  usq_kernel<<<kUsqGroups, kThreads, 0, stream>>>(g, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  divisor_kernel<<<1, kThreads, 0, stream>>>(p, w, kUsqGroups);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  moment_kernel<<<kMomentGroups, kThreads, 0, stream>>>(g, moment_q, moment_scale, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  step_size_kernel<<<1, kThreads, 0, stream>>>(p, w, kMomentGroups * (kThreads / kWave));
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  final_kernel<<<static_cast<unsigned>(w.final_groups), kThreads, 0, stream>>>(
      g, coord, packed, moment_q, moment_scale, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  finish_kernel<<<ceil_div(p.blocks, kThreads) < 1024 ? ceil_div(p.blocks, kThreads) : 1024, kThreads, 0,
                  stream>>>(moment_scale, flips_out, p, w);
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
