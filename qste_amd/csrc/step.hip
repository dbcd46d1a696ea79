// The fused QSTE coordinate step (spec: src/qste/kernels/fallback.py:158-242).
//
// The step has three global dependencies -- the factored row/column second
// moments, the global RMS of the normalized update, and the global RMS of
// the new momentum -- so it runs as a short chain of passes over the fp32
// evidence, none of which writes the evidence:
//
//   stats    one workgroup per strip of rows and chunk of 1024 columns: row
//            sums of g^2 + 1e-12 (finished here when one chunk holds the
//            row), column partial sums per strip
//   colrow   column EMA, fp16 col_v, column factor; its last workgroups
//            finish rows split over chunks (row EMA, fp16 row_v) and sum
//            the clamped row statistic
//   usq      (prologue: mean row statistic) sum of U^2, U = g * rf * cf,
//            per workgroup; on the vector path also the momentum
//            m = q*S*b1 + (1-b1)*U as if the clip divisor were 1: new fp16
//            block scales and sum of m^2
//   moment   (prologue: RMS clip divisor) returns at once when the divisor
//            is exactly 1 (then U / div == U and the usq pass's momentum is
//            the exact result, which is the usual case: the clip engages
//            only when rms(U) > update_clip); otherwise
//            m = q*S*b1 + (1-b1)*U/div for one momentum block per wave:
//            new fp16 block scale, sum of m^2
//   final    (prologue: step size 1/rms(m) * lr) stochastic rounding, momentum
//            requantization, sign repack and flip count, 8 columns (one
//            packed byte) per thread
//   finish   new block scales into place, flip total
//
// Float semantics follow the specification operation by operation: every
// element-wise product and sum rounds in fp32 (this file is compiled with
// -ffp-contract=off), torch's `add_(x, alpha=a)` is a fused multiply-add
// (fmaf), divisions and square roots are correctly rounded.  Reductions
// accumulate in double, each in a fixed order, and round once, so results
// equal the correctly rounded sums but in vanishingly rare cases, whichever
// kernel (and so whichever order) a shape takes.
//
// Fast paths (vector loads) need cols % 8 == 0 and a power-of-two
// block_size >= 8; other shapes and block sizes (any positive size, as the
// specification allows) take scalar code with the same arithmetic.  Shapes with cols % 256
// == 0 and block_size <= 256 take the row kernels for the stats, usq and
// momentum passes: a wave owns a 1024-column chunk of one row at a time,
// keeps its column factors in registers, and finds a momentum block's
// maximum among block_size / 4 consecutive lanes with DPP lane moves.
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace qste {

namespace step {

constexpr int kThreads = 256;
constexpr int kStrip = 64;        // rows per stats workgroup
constexpr int kColChunk = 1024;   // columns per stats workgroup (4 per thread)
constexpr int kUsqGroups = 1024;
constexpr int kMomentGroups = kUsqGroups;  // the momentum partials share the usq layout
constexpr int kFinalGroups = 2048;
constexpr int kRowsGroups = 64;   // workgroups finishing the row statistics

struct Params {
  float b1, a1, b2, a2, clip, lr;
  int64_t rows, cols, count, blocks, block_size;
  int block_shift;  // log2(block_size), or -1 when block_size is not a power of two
  uint32_t seed_part;
  int64_t step;
  const int64_t* step_device;
  const uint8_t* enabled;
  bool vec;       // cols % 8 == 0, block_size a power of two >= 8
  bool small;     // rows * cols < 2^32: 32-bit index arithmetic
  uint32_t bpr;   // momentum blocks per row when cols % block_size == 0, else 0
  bool spec;      // the usq pass also computes the momentum as if the clip divisor were 1
};

// Momentum block of flat index i.
__device__ __forceinline__ int64_t block_of(int64_t i, const Params& p) {
  return p.block_shift >= 0 ? (i >> p.block_shift) : i / p.block_size;
}

// Row and column of flat index i.
__device__ __forceinline__ void row_col(int64_t i, const Params& p, int64_t& r, int64_t& c) {
  if (p.small) {
    const uint32_t ii = static_cast<uint32_t>(i), cc = static_cast<uint32_t>(p.cols);
    const uint32_t rr = ii / cc;
    r = rr;
    c = ii - rr * cc;
  } else {
    r = i / p.cols;
    c = i - r * p.cols;
  }
}

struct Work {
  double* col_part;    // [nstrips][cols]
  double* clamp_part;  // [kRowsGroups] partial sums of max(new_row, 1e-10)
  double* row_part;    // [nchunks][rows]
  float* new_row;      // [rows]
  float* row_factor;   // [rows] (written by the usq pass)
  float* new_col;      // [cols]
  float* col_factor;   // [cols]
  double* usq_part;    // [kUsqGroups]
  double* msq_part;    // [kMomentGroups]
  float* scalars;      // [0] sqrt(mean row stat), [1] divisor, [2] step size, [3] rms(m)
  uint16_t* s_new;     // [blocks]
  float* s_rcp;        // [blocks] 1 / max(s_new, 1e-12), correctly rounded (row path)
  int64_t* flips_part; // [kFinalGroups]
  int64_t nstrips, nchunks;
  int64_t parts;       // slots of usq_part and msq_part written (<= kUsqGroups)
  int64_t fparts;      // slots of flips_part written (<= kFinalGroups)
};

__device__ __forceinline__ bool enabled(const Params& p) {
  return p.enabled == nullptr || *p.enabled != 0;
}

__device__ __forceinline__ float square_eps(float v) {
  float sq = v * v;
  return sq + 1e-12f;
}

__device__ __forceinline__ float normalized(float g, float rf, float cf) {
  float u = g * rf;
  return u * cf;
}

__device__ __forceinline__ float row_factor_of(float sqrt_mean, float new_row) {
  return sqrt_mean / sqrtf(fmaxf(new_row, 1e-10f));
}

__device__ __forceinline__ float moment_of(float u2, float prev, float s_old, const Params& p) {
  float decoded = prev * s_old;
  decoded = decoded * p.b1;
  return fmaf(u2, p.a1, decoded);
}

// DPP lane moves (v_mov_b32 with a data-parallel-primitive control): lane i
// receives the value of the lane CTRL names; a lane whose source lies outside
// its row of 16 lanes, or whose row is not in ROWS, receives 0.
constexpr int kShr1 = 0x111, kShr2 = 0x112, kShr4 = 0x114, kShr8 = 0x118;  // row_shr:n
constexpr int kBcast15 = 0x142, kBcast31 = 0x143;                         // row_bcast:15, :31
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROWS, 0xF, true));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL, ROWS>(__float_as_uint(v)));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = dpp_u32<CTRL, ROWS>(static_cast<uint32_t>(b));
  const uint64_t hi = dpp_u32<CTRL, ROWS>(static_cast<uint32_t>(b >> 32));
  return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}

// Maximum of nonnegative values over aligned groups of n lanes (n a power of
// two, 1..64): after the shift by 2^j every lane holds the maximum of the
// 2^(j+1) lanes ending at it within its row; the broadcasts join rows.  The
// last lane of each group receives the group's maximum.
__device__ __forceinline__ float group_max_last(float v, int n) {
  if (n >= 2) v = fmaxf(v, dpp_f32<kShr1>(v));
  if (n >= 4) v = fmaxf(v, dpp_f32<kShr2>(v));
  if (n >= 8) v = fmaxf(v, dpp_f32<kShr4>(v));
  if (n >= 16) v = fmaxf(v, dpp_f32<kShr8>(v));
  if (n >= 32) v = fmaxf(v, dpp_f32<kBcast15, 0xA>(v));
  if (n >= 64) v = fmaxf(v, dpp_f32<kBcast31, 0xC>(v));
  return v;
}

template <int N>
__device__ __forceinline__ float group_max_last_n(float v) {
  if (N >= 2) v = fmaxf(v, dpp_f32<kShr1>(v));
  if (N >= 4) v = fmaxf(v, dpp_f32<kShr2>(v));
  if (N >= 8) v = fmaxf(v, dpp_f32<kShr4>(v));
  if (N >= 16) v = fmaxf(v, dpp_f32<kShr8>(v));
  if (N >= 32) v = fmaxf(v, dpp_f32<kBcast15, 0xA>(v));
  if (N >= 64) v = fmaxf(v, dpp_f32<kBcast31, 0xC>(v));
  return v;
}

// Sum over the wave in a fixed tree (the same shifts and broadcasts), read
// back from the last lane: every lane receives the total.
__device__ __forceinline__ double wave_total(double v) {
  v += dpp_f64<kShr1>(v);
  v += dpp_f64<kShr2>(v);
  v += dpp_f64<kShr4>(v);
  v += dpp_f64<kShr8>(v);
  v += dpp_f64<kBcast15, 0xA>(v);
  v += dpp_f64<kBcast31, 0xC>(v);
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), 63));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), 63));
  return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}

// -- stats: strip of rows x chunk of columns --------------------------------
// Thread t owns columns c0 + 4t .. c0 + 4t + 3 of the chunk.  When the whole
// row fits one chunk (cols <= 1024) the row sums complete here; otherwise
// per-chunk row partials go to row_part and are combined in `colrow`.
__global__ __launch_bounds__(kThreads) void stats_kernel(const float* __restrict__ g,
                                                         uint16_t* __restrict__ row_v, Params p,
                                                         Work w) {
  __shared__ double red[kStrip][kThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t chunk = blockIdx.x;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kStrip;
  const int64_t c0 = chunk * kColChunk + threadIdx.x * 4;
  const int rows_here = static_cast<int>(p.rows - r0 < kStrip ? p.rows - r0 : kStrip);
  double col_acc[4] = {0.0, 0.0, 0.0, 0.0};
  const bool full4 = p.vec && c0 + 4 <= p.cols;
  for (int rr0 = 0; rr0 < rows_here; rr0 += 4) {
    // four rows' loads in flight before any reduction
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (full4 && rr0 + u < rows_here) v[u] = *reinterpret_cast<const float4*>(g + (r0 + rr0 + u) * p.cols + c0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rr = rr0 + u;
      if (rr >= rows_here) break;
      double rp = 0.0;
      if (full4) {
        const float s0 = square_eps(v[u].x), s1 = square_eps(v[u].y);
        const float s2 = square_eps(v[u].z), s3 = square_eps(v[u].w);
        col_acc[0] += s0; col_acc[1] += s1; col_acc[2] += s2; col_acc[3] += s3;
        rp = (static_cast<double>(s0) + static_cast<double>(s1)) +
             (static_cast<double>(s2) + static_cast<double>(s3));
      } else {
        const float* line = g + (r0 + rr) * p.cols;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (c0 + j < p.cols) {
            const float sq = square_eps(line[c0 + j]);
            col_acc[j] += static_cast<double>(sq);
            rp += static_cast<double>(sq);
          }
        }
      }
      rp = wave_sum(rp);
      if (lane == 0) red[rr][wave] = rp;
    }
  }
  __syncthreads();
  if (threadIdx.x < rows_here) {
    double s = 0.0;
    for (int k = 0; k < kThreads / kWave; ++k) s += red[threadIdx.x][k];
    const int64_t r = r0 + threadIdx.x;
    if (w.nchunks == 1) {
      const float mean = static_cast<float>(s) / static_cast<float>(p.cols);
      const float nr = fmaf(mean, p.a2, f16_to_f32(row_v[r]) * p.b2);
      w.new_row[r] = nr;
      if (enabled(p)) row_v[r] = f32_to_f16(nr);
    } else {
      w.row_part[chunk * p.rows + r] = s;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (c0 + j < p.cols) w.col_part[static_cast<int64_t>(blockIdx.y) * p.cols + c0 + j] = col_acc[j];
}

// -- column statistics and the rows split over chunks --------------------------
// Workgroups below `col_groups` own 16 columns each: thread t sums strips
// t/16, t/16 + 16, ... of column 16 b + t % 16 and a column's 16 partials
// are combined in a fixed order.  The kRowsGroups workgroups after them
// finish rows whose sums were split over chunks and sum the clamped row
// statistic (finished by the next pass).
__global__ __launch_bounds__(kThreads) void colrow_kernel(uint16_t* __restrict__ col_v,
                                                          uint16_t* __restrict__ row_v, Params p, Work w,
                                                          int col_groups) {
  const bool on = enabled(p);
  if (static_cast<int>(blockIdx.x) >= col_groups) {
    __shared__ double red[kThreads / kWave];
    const int64_t group = static_cast<int64_t>(blockIdx.x) - col_groups;
    double acc = 0.0;
    for (int64_t r = group * kThreads + threadIdx.x; r < p.rows; r += static_cast<int64_t>(kRowsGroups) * kThreads) {
      float nr;
      if (w.nchunks > 1) {
        double s = 0.0;
        for (int64_t k = 0; k < w.nchunks; ++k) s += w.row_part[k * p.rows + r];
        const float mean = static_cast<float>(s) / static_cast<float>(p.cols);
        nr = fmaf(mean, p.a2, f16_to_f32(row_v[r]) * p.b2);
        w.new_row[r] = nr;
        if (on) row_v[r] = f32_to_f16(nr);
      } else {
        nr = w.new_row[r];
      }
      acc += static_cast<double>(fmaxf(nr, 1e-10f));
    }
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) w.clamp_part[group] = acc;
    return;
  }
  __shared__ double part[16][17];
  const int cl = threadIdx.x & 15, sg = threadIdx.x >> 4;
  const int64_t c = blockIdx.x * 16ll + cl;
  double s = 0.0;
  if (c < p.cols)
    for (int64_t k = sg; k < w.nstrips; k += 16) s += w.col_part[k * p.cols + c];
  part[sg][cl] = s;
  __syncthreads();
  if (threadIdx.x < 16 && c < p.cols) {
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += part[k][cl];
    const float mean = static_cast<float>(t) / static_cast<float>(p.rows);
    const float nc = fmaf(mean, p.a2, f16_to_f32(col_v[c]) * p.b2);
    w.new_col[c] = nc;
    w.col_factor[c] = 1.0f / sqrtf(fmaxf(nc, 1e-10f));
    if (on) col_v[c] = f32_to_f16(nc);
  }
}

// sqrt of the mean clamped row statistic (the same value in every workgroup)
__device__ __forceinline__ float sqrt_mean_of(const Params& p, const Work& w, double* red) {
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < kRowsGroups; i += kThreads) acc += w.clamp_part[i];
  acc = block_sum(acc, red);
  const float v = sqrtf(static_cast<float>(acc) / static_cast<float>(p.rows));
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) w.scalars[0] = v;
  return v;
}

// -- sum of U^2, one row at a time per workgroup -----------------------------
// On the vector path with spec set, lane l of wave w holds columns
// 4 (64 w' + l) .. + 3 of a 1024-column slice: its 4 elements share one
// momentum block (block_size in 4..256, a power of two, dividing cols), and
// the block_size / 4 lanes of a block reduce its |m| maximum.
__global__ __launch_bounds__(kThreads) void usq_kernel(const float* __restrict__ g,
                                                       const int8_t* __restrict__ moment_q,
                                                       const uint16_t* __restrict__ moment_scale, Params p,
                                                       Work w) {
  __shared__ double red[kThreads / kWave];
  const float sqrt_mean = sqrt_mean_of(p, w, red);
  const int lane = threadIdx.x & (kWave - 1);
  double acc = 0.0, msq = 0.0;
  for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const float rf = row_factor_of(sqrt_mean, w.new_row[r]);
    if (threadIdx.x == 0) w.row_factor[r] = rf;
    const float* line = g + r * p.cols;
    if (p.vec) {
      const float4* l4 = reinterpret_cast<const float4*>(line);
      const float4* cf4 = reinterpret_cast<const float4*>(w.col_factor);
      const uint32_t* q4p = reinterpret_cast<const uint32_t*>(moment_q + r * p.cols);
      for (int64_t q = threadIdx.x; q < p.cols / 4; q += kThreads) {
        const float4 v = l4[q], cf = cf4[q];
        uint32_t q4 = 0;
        float s_old = 0.0f;
        const int64_t blk = (r * p.cols + 4 * q) >> p.block_shift;
        if (p.spec) {
          q4 = q4p[q];
          s_old = f16_to_f32(moment_scale[blk]);
        }
        const float u[4] = {normalized(v.x, rf, cf.x), normalized(v.y, rf, cf.y), normalized(v.z, rf, cf.z),
                            normalized(v.w, rf, cf.w)};
        const float s0 = u[0] * u[0], s1 = u[1] * u[1], s2 = u[2] * u[2], s3 = u[3] * u[3];
        acc += (static_cast<double>(s0) + static_cast<double>(s1)) +
               (static_cast<double>(s2) + static_cast<double>(s3));
        if (p.spec) {
          float amax = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float prev = static_cast<float>(static_cast<int8_t>(q4 >> (8 * e)));
            const float m = moment_of(u[e], prev, s_old, p);
            amax = fmaxf(amax, fabsf(m));
            const float sq = m * m;
            msq += static_cast<double>(sq);
          }
          // maximum over the block's block_size / 4 lanes
          for (int o = 1; o < static_cast<int>(p.block_size >> 2); o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
          if ((lane & ((p.block_size >> 2) - 1)) == 0) w.s_new[blk] = f32_to_f16(fmaxf(amax, 1e-6f) / 127.0f);
        }
      }
    } else {
      for (int64_t c = threadIdx.x; c < p.cols; c += kThreads) {
        const float u = normalized(line[c], rf, w.col_factor[c]);
        const float s = u * u;
        acc += static_cast<double>(s);
      }
    }
  }
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) w.usq_part[blockIdx.x] = acc;
  if (p.spec) {
    __syncthreads();
    msq = block_sum(msq, red);
    if (threadIdx.x == 0) w.msq_part[blockIdx.x] = msq;
  }
}

__device__ __forceinline__ float divisor_of(const double* usq_part, int64_t parts, int64_t count,
                                            float clip, double* red) {
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < parts; i += kThreads) acc += usq_part[i];
  acc = block_sum(acc, red);
  float rms = sqrtf(static_cast<float>(acc) / static_cast<float>(count));
  rms = fmaxf(rms, 1e-8f);
  const float ratio = rms / clip;
  return ratio > 1.0f ? ratio : 1.0f;
}

// -- momentum: one wave per block at a time, 4 elements per lane ------------
__global__ __launch_bounds__(kThreads) void moment_kernel(const float* __restrict__ g,
                                                          const int8_t* __restrict__ moment_q,
                                                          const uint16_t* __restrict__ moment_scale,
                                                          Params p, Work w) {
  __shared__ double red[kThreads / kWave];
  __shared__ double wsum[kThreads / kWave];
  const float divisor = divisor_of(w.usq_part, w.parts, p.count, p.clip, red);
  if (blockIdx.x == 0 && threadIdx.x == 0) w.scalars[1] = divisor;
  // the usq pass's momentum assumed a divisor of 1: exact if it is
  if (p.spec && divisor == 1.0f) return;
  const float rdiv = 1.0f / divisor;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave;
  double msq = 0.0;
  constexpr int G = 4;  // blocks per wave iteration: four independent loads per lane
  for (int64_t g0 = wave_id * G; g0 < p.blocks; g0 += waves * G) {
    float amax[G] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t j = 4 * lane; j < p.block_size; j += 4 * kWave) {
      float4 v[G], cf[G];
      uint32_t q4[G];
      float rf[G];
      bool fast[G];
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int64_t b = g0 + k;
        const int64_t i = b * p.block_size + j;
        fast[k] = p.vec && b < p.blocks && i + 4 <= p.count;
        if (fast[k]) {
          int64_t r, c;
          if (p.bpr) {
            const uint32_t bb = static_cast<uint32_t>(b);
            const uint32_t br = bb / p.bpr;
            r = br;
            c = static_cast<int64_t>(bb - br * p.bpr) * p.block_size + j;
          } else {
            row_col(i, p, r, c);
          }
          v[k] = *reinterpret_cast<const float4*>(g + i);
          cf[k] = *reinterpret_cast<const float4*>(w.col_factor + c);
          q4[k] = *reinterpret_cast<const uint32_t*>(moment_q + i);
          rf[k] = w.row_factor[r];
        }
      }
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int64_t b = g0 + k;
        if (b >= p.blocks) break;
        const float s_old = f16_to_f32(moment_scale[b]);
        const int64_t i = b * p.block_size + j;
        float m[4] = {0.f, 0.f, 0.f, 0.f};
        if (fast[k]) {
          const float gv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
          const float cv[4] = {cf[k].x, cf[k].y, cf[k].z, cf[k].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float u2 = div_by(normalized(gv[e], rf[k], cv[e]), divisor, rdiv);
            const float prev = static_cast<float>(static_cast<int8_t>(q4[k] >> (8 * e)));
            m[e] = moment_of(u2, prev, s_old, p);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t ie = i + e;
            if (j + e < p.block_size && ie < p.count) {
              int64_t r, c;
              row_col(ie, p, r, c);
              const float u2 = div_by(normalized(g[ie], w.row_factor[r], w.col_factor[c]), divisor, rdiv);
              m[e] = moment_of(u2, static_cast<float>(moment_q[ie]), s_old, p);
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          amax[k] = fmaxf(amax[k], fabsf(m[e]));
          const float sq = m[e] * m[e];
          msq += static_cast<double>(sq);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int64_t b = g0 + k;
      const float a = wave_max(amax[k]);
      if (lane == 0 && b < p.blocks) w.s_new[b] = f32_to_f16(fmaxf(a, 1e-6f) / 127.0f);
    }
  }
  msq = wave_sum(msq);
  __syncthreads();
  if (lane == 0) wsum[wave] = msq;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int k = 0; k < kThreads / kWave; ++k) t += wsum[k];
    w.msq_part[blockIdx.x] = t;
  }
}

// -- row path --------------------------------------------------------------------
// cols % 256 == 0, block_size 8..256, vector-aligned operands.  A wave owns a
// kRowChunk-column chunk of one row at a time: lane l holds the float4
// slots at columns c0 + 4 l + 256 k, k = 0..3, and a slot is present in
// every lane or in none (chunk_slots).  A momentum block of block_size
// columns is then block_size / 4 consecutive lanes of one slot.
constexpr int kRowChunk = kColChunk;

__device__ __forceinline__ int chunk_slots(int64_t cols, int64_t c0) {
  const int64_t left = (cols - c0) >> 8;
  return left >= 4 ? 4 : static_cast<int>(left);
}

// stats on the row path: workgroup (b, chunk) takes rows 4 b + wave,
// + 4 gridDim.x, ... of its chunk, the next row's loads issued before the
// current row is reduced; one wave sum per row and chunk, and the column
// partials of the four waves combined through LDS into strip b.  Same
// outputs as stats_kernel with gridDim.x strips.
__global__ __launch_bounds__(kThreads) void stats_row_kernel(const float* __restrict__ g,
                                                             uint16_t* __restrict__ row_v, Params p, Work w) {
  __shared__ double colsum[kThreads / kWave][kRowChunk];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t chunk = blockIdx.y;
  const int64_t c0 = chunk * kRowChunk;
  const int ns = chunk_slots(p.cols, c0);
  // slots past the chunk's end re-read its last slot (results dropped)
  int64_t sc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) sc[k] = c0 + 4 * lane + 256 * (k < ns ? k : ns - 1);
  double col[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) col[k][e] = 0.0;
  const int64_t rstep = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave;
  float4 cur[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) cur[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (r < p.rows) {
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = *reinterpret_cast<const float4*>(g + r * p.cols + sc[k]);
  }
  for (; r < p.rows; r += rstep) {
    // the last row re-reads itself (a cache hit) rather than branch
    const int64_t rn = r + rstep < p.rows ? r + rstep : r;
    float4 nxt[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) nxt[k] = *reinterpret_cast<const float4*>(g + rn * p.cols + sc[k]);
    __builtin_amdgcn_sched_barrier(0);  // the next row's loads in flight during this row's arithmetic
    double rp = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k >= ns) break;
      const double d0 = square_eps(cur[k].x), d1 = square_eps(cur[k].y);
      const double d2 = square_eps(cur[k].z), d3 = square_eps(cur[k].w);
      col[k][0] += d0; col[k][1] += d1; col[k][2] += d2; col[k][3] += d3;
      rp += (d0 + d1) + (d2 + d3);
    }
    rp = wave_total(rp);
    if (lane == 0) {
      if (w.nchunks == 1) {
        const float mean = static_cast<float>(rp) / static_cast<float>(p.cols);
        const float nr = fmaf(mean, p.a2, f16_to_f32(row_v[r]) * p.b2);
        w.new_row[r] = nr;
        if (enabled(p)) row_v[r] = f32_to_f16(nr);
      } else {
        w.row_part[chunk * p.rows + r] = rp;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = nxt[k];
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) colsum[wave][256 * k + 4 * lane + e] = col[k][e];
  __syncthreads();
  for (int c = threadIdx.x; c < 256 * ns; c += kThreads)
    w.col_part[static_cast<int64_t>(blockIdx.x) * p.cols + c0 + c] =
        (colsum[0][c] + colsum[1][c]) + (colsum[2][c] + colsum[3][c]);
}

// usq (MOMENT false) and momentum (MOMENT true) passes on the row path:
// workgroup (b, chunk) takes rows 4 b + wave, + 4 gridDim.x, ... of its
// chunk and writes partial slot chunk * gridDim.x + b.  The usq pass also
// computes the momentum when p.spec is set (as usq_kernel does), the
// momentum pass returns at once when that result stands.
template <bool MOMENT>
__global__ __launch_bounds__(kThreads) void elem_row_kernel(const float* __restrict__ g,
                                                            const int8_t* __restrict__ moment_q,
                                                            const uint16_t* __restrict__ moment_scale,
                                                            Params p, Work w) {
  __shared__ double red[kThreads / kWave];
  float divisor = 1.0f, sqrt_mean = 0.0f;
  if (MOMENT) {
    divisor = divisor_of(w.usq_part, w.parts, p.count, p.clip, red);
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) w.scalars[1] = divisor;
    if (p.spec && divisor == 1.0f) return;
  } else {
    sqrt_mean = sqrt_mean_of(p, w, red);
  }
  const bool with_m = MOMENT || p.spec;
  const float rdiv = 1.0f / divisor;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t chunk = blockIdx.y;
  const int64_t c0 = chunk * kRowChunk;
  const int ns = chunk_slots(p.cols, c0);
  const int gsize = static_cast<int>(p.block_size >> 2);  // lanes per momentum block
  // loads are unconditional (straight-line code keeps the compiler's waits
  // per load): slots past the chunk's end re-read its last slot, and those
  // results are dropped
  int64_t sc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) sc[k] = c0 + 4 * lane + 256 * (k < ns ? k : ns - 1);
  float4 cf[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) cf[k] = *reinterpret_cast<const float4*>(w.col_factor + sc[k]);
  double acc = 0.0, msq = 0.0;
  const int64_t rstep = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave; r < p.rows; r += rstep) {
    float rf;
    if (MOMENT) {
      rf = w.row_factor[r];
    } else {
      rf = row_factor_of(sqrt_mean, w.new_row[r]);
      if (chunk == 0 && lane == 0) w.row_factor[r] = rf;
    }
    const int64_t rb = r * p.cols;
    float4 v[4];
    uint32_t q4[4];
    float so[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = *reinterpret_cast<const float4*>(g + rb + sc[k]);
      if (with_m) {
        q4[k] = *reinterpret_cast<const uint32_t*>(moment_q + rb + sc[k]);
        so[k] = f16_to_f32(moment_scale[(rb + sc[k]) >> p.block_shift]);
      } else {
        q4[k] = 0u;
        so[k] = 0.f;
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the arithmetic
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k >= ns) break;
      const float gv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
      const float cv[4] = {cf[k].x, cf[k].y, cf[k].z, cf[k].w};
      float uu[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uu[e] = normalized(gv[e], rf, cv[e]);
        if (MOMENT) uu[e] = div_by(uu[e], divisor, rdiv);
      }
      if (!MOMENT) {
        const float s0 = uu[0] * uu[0], s1 = uu[1] * uu[1], s2 = uu[2] * uu[2], s3 = uu[3] * uu[3];
        acc += (static_cast<double>(s0) + static_cast<double>(s1)) +
               (static_cast<double>(s2) + static_cast<double>(s3));
      }
      if (with_m) {
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float prev = static_cast<float>(static_cast<int8_t>(q4[k] >> (8 * e)));
          const float m = moment_of(uu[e], prev, so[k], p);
          amax = fmaxf(amax, fabsf(m));
          const float sq = m * m;
          msq += static_cast<double>(sq);
        }
        amax = group_max_last(amax, gsize);
        if ((lane & (gsize - 1)) == gsize - 1) {
          const int64_t blk = (rb + sc[k]) >> p.block_shift;
          const uint16_t s16 = f32_to_f16(fmaxf(amax, 1e-6f) / 127.0f);
          w.s_new[blk] = s16;
          w.s_rcp[blk] = 1.0f / fmaxf(f16_to_f32(s16), 1e-12f);
        }
      }
    }
  }
  const int64_t slot = chunk * gridDim.x + blockIdx.x;
  if (!MOMENT) {
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) w.usq_part[slot] = acc;
  }
  if (with_m) {
    __syncthreads();
    msq = block_sum(msq, red);
    if (threadIdx.x == 0) w.msq_part[slot] = msq;
  }
}

// -- final element pass: one packed byte (8 columns) per thread ---------------

// Step size of the spec (fallback.py:204-206): `coordinate_lr / moment_rms`
// divides a Python float by an fp32 tensor, which torch evaluates as
// Tensor.__rtruediv__, `reciprocal(moment_rms) * fp32(lr)`: two roundings,
// not one division (they differ for a learning rate that is not a power of
// two).
__device__ __forceinline__ float step_size_of(float mrms, float lr) {
  const float inverse = 1.0f / mrms;
  return inverse * lr;
}

struct FinalScalars {
  float step_size, divisor, rdiv;
  uint32_t combined;
  bool on;
};

// Prologue shared by the final kernels: momentum RMS -> step size (stored in
// scalars[2] with the RMS in scalars[3] by the first workgroup), the clip
// divisor of the momentum pass, and the hash key of (seed, step).
__device__ __forceinline__ FinalScalars final_prologue(const Params& p, const Work& w, double* red) {
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < w.parts; i += kThreads) acc += w.msq_part[i];
  acc = block_sum(acc, red);
  const float padded = static_cast<float>(p.blocks * p.block_size);
  float mrms = sqrtf(static_cast<float>(acc) / padded);
  mrms = fmaxf(mrms, 1e-8f);
  FinalScalars f;
  f.step_size = step_size_of(mrms, p.lr);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    w.scalars[2] = f.step_size;
    w.scalars[3] = mrms;
  }
  f.divisor = w.scalars[1];
  f.rdiv = 1.0f / f.divisor;
  const int64_t step = p.step_device ? *p.step_device : p.step;
  f.combined = p.seed_part ^ step_hash(step);
  f.on = enabled(p);
  return f;
}
__device__ __forceinline__ uint32_t final_byte(const float* __restrict__ g, int8_t* __restrict__ coord,
                                               int8_t* __restrict__ moment_q,
                                               const uint16_t* __restrict__ moment_scale, const Params& p,
                                               const Work& w, int64_t r, int64_t b, float rf, float divisor,
                                               float rdiv, float step_size, uint32_t combined, bool on) {
  const int64_t c0 = b * 8;
  const int64_t i0 = r * p.cols + c0;
  const int n = static_cast<int>(p.cols - c0 < 8 ? p.cols - c0 : 8);
  float gv[8], cv[8], prev[8], cur[8];
  float s_old = 0.f, s_new = 0.f, rdec = 1.0f;
  if (p.vec) {
    const float4 ga = *reinterpret_cast<const float4*>(g + i0);
    const float4 gb = *reinterpret_cast<const float4*>(g + i0 + 4);
    const float4 ca = *reinterpret_cast<const float4*>(w.col_factor + c0);
    const float4 cb = *reinterpret_cast<const float4*>(w.col_factor + c0 + 4);
    const uint64_t q8 = *reinterpret_cast<const uint64_t*>(moment_q + i0);
    const uint64_t c8 = *reinterpret_cast<const uint64_t*>(coord + i0);
    gv[0] = ga.x; gv[1] = ga.y; gv[2] = ga.z; gv[3] = ga.w; gv[4] = gb.x; gv[5] = gb.y; gv[6] = gb.z; gv[7] = gb.w;
    cv[0] = ca.x; cv[1] = ca.y; cv[2] = ca.z; cv[3] = ca.w; cv[4] = cb.x; cv[5] = cb.y; cv[6] = cb.z; cv[7] = cb.w;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      prev[j] = static_cast<float>(static_cast<int8_t>(q8 >> (8 * j)));
      cur[j] = static_cast<float>(static_cast<int8_t>(c8 >> (8 * j)));
    }
    const int64_t blk = i0 >> p.block_shift;  // block_size >= 8: one block for the byte
    s_old = f16_to_f32(moment_scale[blk]);
    s_new = f16_to_f32(w.s_new[blk]);
    rdec = 1.0f / fmaxf(s_new, 1e-12f);
  } else {
    for (int j = 0; j < 8; ++j) {
      if (j < n) {
        gv[j] = g[i0 + j];
        cv[j] = w.col_factor[c0 + j];
        prev[j] = static_cast<float>(moment_q[i0 + j]);
        cur[j] = static_cast<float>(coord[i0 + j]);
      } else {
        gv[j] = cv[j] = prev[j] = cur[j] = 0.f;
      }
    }
  }
  uint32_t byte = 0;
  uint64_t cnew8 = 0, qnew8 = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j >= n) continue;
    const int64_t i = i0 + j;
    float so = s_old, sn = s_new;
    if (!p.vec) {
      const int64_t blk = block_of(i, p);
      so = f16_to_f32(moment_scale[blk]);
      sn = f16_to_f32(w.s_new[blk]);
    }
    const float u2 = div_by(normalized(gv[j], rf, cv[j]), divisor, rdiv);
    const float m = moment_of(u2, prev[j], so, p);
    const float delta = m * step_size;
    const float target = cur[j] - delta;
    const float lower = floorf(target);
    const float u = static_cast<float>(scramble(static_cast<uint32_t>(static_cast<uint64_t>(i)) ^ combined)) *
                    (1.0f / 4294967296.0f);
    const float frac = target - lower;
    float rounded = lower + (u < frac ? 1.0f : 0.0f);
    rounded = fminf(127.0f, fmaxf(-127.0f, rounded));
    const float decode = fmaxf(sn, 1e-12f);
    float q = rintf(div_by(m, decode, p.vec ? rdec : 1.0f / decode));
    q = fminf(127.0f, fmaxf(-127.0f, q));
    const int8_t cn = static_cast<int8_t>(rounded), qn = static_cast<int8_t>(q);
    cnew8 |= static_cast<uint64_t>(static_cast<uint8_t>(cn)) << (8 * j);
    qnew8 |= static_cast<uint64_t>(static_cast<uint8_t>(qn)) << (8 * j);
    byte |= (rounded >= 0.0f ? 1u : 0u) << j;
    if (on && !p.vec) {
      coord[i] = cn;
      moment_q[i] = qn;
    }
  }
  if (on && p.vec) {
    *reinterpret_cast<uint64_t*>(coord + i0) = cnew8;
    *reinterpret_cast<uint64_t*>(moment_q + i0) = qnew8;
  }
  return byte;
}

__global__ __launch_bounds__(kThreads) void final_kernel(const float* __restrict__ g,
                                                         int8_t* __restrict__ coord,
                                                         uint8_t* __restrict__ packed,
                                                         int8_t* __restrict__ moment_q,
                                                         const uint16_t* __restrict__ moment_scale,
                                                         Params p, Work w) {
  __shared__ double red[kThreads / kWave];
  __shared__ int64_t ired[kThreads / kWave];
  const FinalScalars f = final_prologue(p, w, red);
  const float step_size = f.step_size, divisor = f.divisor, rdiv = f.rdiv;
  const uint32_t combined = f.combined;
  const bool on = f.on;

  const int64_t stride = (p.cols + 7) / 8;
  const int64_t total = p.rows * stride;
  int64_t flips = 0;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kThreads) {
    int64_t r, b;
    if (p.small) {
      const uint32_t ii = static_cast<uint32_t>(idx), ss = static_cast<uint32_t>(stride);
      const uint32_t rr = ii / ss;
      r = rr;
      b = ii - rr * ss;
    } else {
      r = idx / stride;
      b = idx - r * stride;
    }
    const float rf = w.row_factor[r];
    const uint32_t old_byte = packed[idx];
    const uint32_t byte = final_byte(g, coord, moment_q, moment_scale, p, w, r, b, rf, divisor, rdiv, step_size,
                                     combined, on);
    const int64_t c0 = b * 8;
    const int n = static_cast<int>(p.cols - c0 < 8 ? p.cols - c0 : 8);
    const uint32_t mask = n >= 8 ? 0xFFu : ((1u << n) - 1u);
    flips += __popc((old_byte ^ byte) & mask);
    if (on) packed[idx] = static_cast<uint8_t>(byte);
  }
  flips = block_sum(flips, ired);
  if (threadIdx.x == 0) w.flips_part[blockIdx.x] = on ? flips : 0;
}

// Vector path of the final pass (cols % 8 == 0, block_size >= 8, aligned
// pointers): one packed byte per thread per iteration, straight-line code
// for its 8 elements, the same arithmetic as final_byte.  With a clip
// divisor of exactly 1 the correction U / div is the identity and is
// skipped (a uniform choice per workgroup).
template <bool DIV1>
__device__ __forceinline__ int64_t final_vec_loop(const float* __restrict__ g, int8_t* __restrict__ coord,
                                                  uint8_t* __restrict__ packed, int8_t* __restrict__ moment_q,
                                                  const uint16_t* __restrict__ moment_scale, const Params& p,
                                                  const Work& w, float divisor, float rdiv, float step_size,
                                                  uint32_t combined, bool on) {
  const int64_t stride = p.cols >> 3;
  const int64_t total = p.rows * stride;
  int64_t flips = 0;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kThreads) {
    int64_t r, b;
    if (p.small) {
      const uint32_t ii = static_cast<uint32_t>(idx), ss = static_cast<uint32_t>(stride);
      const uint32_t rr = ii / ss;
      r = rr;
      b = ii - rr * ss;
    } else {
      r = idx / stride;
      b = idx - r * stride;
    }
    const int64_t c0 = b * 8;
    const int64_t i0 = r * p.cols + c0;
    const float4 ga = *reinterpret_cast<const float4*>(g + i0);
    const float4 gb = *reinterpret_cast<const float4*>(g + i0 + 4);
    const float4 ca = *reinterpret_cast<const float4*>(w.col_factor + c0);
    const float4 cb = *reinterpret_cast<const float4*>(w.col_factor + c0 + 4);
    const uint64_t q8 = *reinterpret_cast<const uint64_t*>(moment_q + i0);
    const uint64_t c8 = *reinterpret_cast<const uint64_t*>(coord + i0);
    const uint32_t old_byte = packed[idx];
    const float rf = w.row_factor[r];
    const int64_t blk = i0 >> p.block_shift;  // block_size >= 8: one block for the byte
    const float s_old = f16_to_f32(moment_scale[blk]);
    const float decode = fmaxf(f16_to_f32(w.s_new[blk]), 1e-12f);
    const float rdec = 1.0f / decode;
    const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
    const float cv[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
    uint32_t byte = 0, cn_lo = 0, cn_hi = 0, qn_lo = 0, qn_hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float u2 = normalized(gv[j], rf, cv[j]);
      if (!DIV1) u2 = div_by(u2, divisor, rdiv);
      const float prev = static_cast<float>(static_cast<int8_t>(q8 >> (8 * j)));
      const float cur = static_cast<float>(static_cast<int8_t>(c8 >> (8 * j)));
      const float m = moment_of(u2, prev, s_old, p);
      const float delta = m * step_size;
      const float target = cur - delta;
      const float lower = floorf(target);
      const float u = static_cast<float>(scramble(static_cast<uint32_t>(i0 + j) ^ combined)) *
                      (1.0f / 4294967296.0f);
      const float frac = target - lower;
      float rounded = lower + (u < frac ? 1.0f : 0.0f);
      rounded = fminf(127.0f, fmaxf(-127.0f, rounded));
      float q = rintf(div_by(m, decode, rdec));
      q = fminf(127.0f, fmaxf(-127.0f, q));
      const uint32_t cb8 = static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(rounded)));
      const uint32_t qb8 = static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(q)));
      if (j < 4) {
        cn_lo |= cb8 << (8 * j);
        qn_lo |= qb8 << (8 * j);
      } else {
        cn_hi |= cb8 << (8 * (j - 4));
        qn_hi |= qb8 << (8 * (j - 4));
      }
      byte |= (rounded >= 0.0f ? 1u : 0u) << j;
    }
    if (on) {
      *reinterpret_cast<uint64_t*>(coord + i0) = (static_cast<uint64_t>(cn_hi) << 32) | cn_lo;
      *reinterpret_cast<uint64_t*>(moment_q + i0) = (static_cast<uint64_t>(qn_hi) << 32) | qn_lo;
      packed[idx] = static_cast<uint8_t>(byte);
    }
    flips += __popc(old_byte ^ byte);
  }
  return flips;
}

__global__ __launch_bounds__(kThreads) void final_vec_kernel(const float* __restrict__ g,
                                                             int8_t* __restrict__ coord,
                                                             uint8_t* __restrict__ packed,
                                                             int8_t* __restrict__ moment_q,
                                                             const uint16_t* __restrict__ moment_scale,
                                                             Params p, Work w) {
  __shared__ double red[kThreads / kWave];
  __shared__ int64_t ired[kThreads / kWave];
  const FinalScalars f = final_prologue(p, w, red);
  const float step_size = f.step_size, divisor = f.divisor, rdiv = f.rdiv;
  const uint32_t combined = f.combined;
  const bool on = f.on;
  const int64_t flips =
      divisor == 1.0f
          ? final_vec_loop<true>(g, coord, packed, moment_q, moment_scale, p, w, divisor, rdiv, step_size, combined, on)
          : final_vec_loop<false>(g, coord, packed, moment_q, moment_scale, p, w, divisor, rdiv, step_size, combined,
                                  on);
  const int64_t total = block_sum(flips, ired);
  if (threadIdx.x == 0) w.flips_part[blockIdx.x] = on ? total : 0;
}

// Final pass on the row path: workgroup (b, chunk) takes kFinalChunk
// columns of rows 4 b + wave, + 4 gridDim.x, ..., the next row's loads
// issued before the current row's arithmetic;
// lane l owns the packed byte of columns c0 + 8 l .. + 7 (lanes past the
// row's end idle).  Column factors stay in registers, the row factor is one
// load per row, the block scale's reciprocal comes from the momentum pass,
// and the eight elements of a byte share the first step of their hash.
// The same arithmetic as final_byte.
constexpr int kFinalChunk = 512;

template <bool DIV1>
__device__ __forceinline__ int64_t final_row_loop(const float* __restrict__ g, int8_t* __restrict__ coord,
                                                  uint8_t* __restrict__ packed, int8_t* __restrict__ moment_q,
                                                  const uint16_t* __restrict__ moment_scale, const Params& p,
                                                  const Work& w, float divisor, float rdiv, float step_size,
                                                  uint32_t combined, bool on) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kFinalChunk + 8 * lane;
  const bool lane_on = c0 < p.cols;
  const int64_t stride = p.cols >> 3;
  float cv[8];
  {
    const int64_t cl = lane_on ? c0 : p.cols - 8;
    const float4 ca = *reinterpret_cast<const float4*>(w.col_factor + cl);
    const float4 cb = *reinterpret_cast<const float4*>(w.col_factor + cl + 4);
    cv[0] = ca.x; cv[1] = ca.y; cv[2] = ca.z; cv[3] = ca.w; cv[4] = cb.x; cv[5] = cb.y; cv[6] = cb.z; cv[7] = cb.w;
  }
  int64_t flips = 0;
  const int64_t rstep = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  // loads are unconditional (straight-line code keeps the compiler's waits
  // per load): idle lanes read their row's last byte, rows past the end the
  // last row, and those results are dropped
  const int64_t cc = lane_on ? c0 : p.cols - 8;
  struct RowIn {
    float4 ga, gb;
    uint64_t q8, c8;
    uint32_t old_byte;
    float rf, s_old, decode, rdec;
  };
  auto load_row = [&](int64_t r, RowIn& in) {
    const int64_t i0 = r * p.cols + cc;
    in.ga = *reinterpret_cast<const float4*>(g + i0);
    in.gb = *reinterpret_cast<const float4*>(g + i0 + 4);
    in.q8 = *reinterpret_cast<const uint64_t*>(moment_q + i0);
    in.c8 = *reinterpret_cast<const uint64_t*>(coord + i0);
    in.old_byte = packed[r * stride + (cc >> 3)];
    in.rf = w.row_factor[r];
    const int64_t blk = i0 >> p.block_shift;  // block_size >= 8: one block for the byte
    in.s_old = f16_to_f32(moment_scale[blk]);
    in.decode = fmaxf(f16_to_f32(w.s_new[blk]), 1e-12f);
    in.rdec = w.s_rcp[blk];
  };
  int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave;
  RowIn cur;
  load_row(r < p.rows ? r : 0, cur);
  for (; r < p.rows; r += rstep) {
    // the next row's loads in flight during this row's arithmetic; the last
    // row re-reads itself (a cache hit) rather than branch
    RowIn nxt;
    load_row(r + rstep < p.rows ? r + rstep : r, nxt);
    __builtin_amdgcn_sched_barrier(0);
    const int64_t i0 = r * p.cols + cc;
    const uint32_t head = scramble_head(static_cast<uint32_t>(i0) ^ combined);
    const float gv[8] = {cur.ga.x, cur.ga.y, cur.ga.z, cur.ga.w, cur.gb.x, cur.gb.y, cur.gb.z, cur.gb.w};
    uint32_t byte = 0, cn_lo = 0, cn_hi = 0, qn_lo = 0, qn_hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float u2 = normalized(gv[j], cur.rf, cv[j]);
      if (!DIV1) u2 = div_by(u2, divisor, rdiv);
      const float prev = static_cast<float>(static_cast<int8_t>(cur.q8 >> (8 * j)));
      const float cval = static_cast<float>(static_cast<int8_t>(cur.c8 >> (8 * j)));
      const float m = moment_of(u2, prev, cur.s_old, p);
      const float delta = m * step_size;
      const float target = cval - delta;
      const float lower = floorf(target);
      const float uu = static_cast<float>(scramble_tail(head ^ static_cast<uint32_t>(j))) * (1.0f / 4294967296.0f);
      const float frac = target - lower;
      float rounded = lower + (uu < frac ? 1.0f : 0.0f);
      rounded = fminf(127.0f, fmaxf(-127.0f, rounded));
      float q = rintf(div_by(m, cur.decode, cur.rdec));
      q = fminf(127.0f, fmaxf(-127.0f, q));
      const uint32_t cb8 = static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(rounded)));
      const uint32_t qb8 = static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(q)));
      if (j < 4) {
        cn_lo |= cb8 << (8 * j);
        qn_lo |= qb8 << (8 * j);
      } else {
        cn_hi |= cb8 << (8 * (j - 4));
        qn_hi |= qb8 << (8 * (j - 4));
      }
      byte |= (rounded >= 0.0f ? 1u : 0u) << j;
    }
    if (lane_on) {
      if (on) {
        *reinterpret_cast<uint64_t*>(coord + i0) = (static_cast<uint64_t>(cn_hi) << 32) | cn_lo;
        *reinterpret_cast<uint64_t*>(moment_q + i0) = (static_cast<uint64_t>(qn_hi) << 32) | qn_lo;
        packed[r * stride + (cc >> 3)] = static_cast<uint8_t>(byte);
      }
      flips += __popc(cur.old_byte ^ byte);
    }
    cur = nxt;
  }
  return flips;
}

__global__ __launch_bounds__(kThreads) void final_row_kernel(const float* __restrict__ g,
                                                             int8_t* __restrict__ coord,
                                                             uint8_t* __restrict__ packed,
                                                             int8_t* __restrict__ moment_q,
                                                             const uint16_t* __restrict__ moment_scale,
                                                             Params p, Work w) {
  __shared__ double red[kThreads / kWave];
  __shared__ int64_t ired[kThreads / kWave];
  const FinalScalars f = final_prologue(p, w, red);
  const float step_size = f.step_size, divisor = f.divisor, rdiv = f.rdiv;
  const uint32_t combined = f.combined;
  const bool on = f.on;
  const int64_t flips =
      divisor == 1.0f
          ? final_row_loop<true>(g, coord, packed, moment_q, moment_scale, p, w, divisor, rdiv, step_size, combined, on)
          : final_row_loop<false>(g, coord, packed, moment_q, moment_scale, p, w, divisor, rdiv, step_size, combined,
                                  on);
  const int64_t total = block_sum(flips, ired);
  if (threadIdx.x == 0) w.flips_part[static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = on ? total : 0;
}

__global__ __launch_bounds__(kThreads) void finish_kernel(uint16_t* __restrict__ moment_scale,
                                                          int64_t* __restrict__ flips_out, Params p, Work w) {
  __shared__ int64_t red[kThreads / kWave];
  if (enabled(p)) {
    for (int64_t b = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; b < p.blocks;
         b += static_cast<int64_t>(gridDim.x) * kThreads)
      moment_scale[b] = w.s_new[b];
  }
  if (blockIdx.x == 0 && flips_out) {
    int64_t acc = 0;
    for (int64_t i = threadIdx.x; i < w.fparts; i += kThreads) acc += w.flips_part[i];
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) *flips_out = acc;
  }
}

// -- one-launch step --------------------------------------------------------------
// Shapes with cols % 2048 == 0, a power-of-two block_size in 8..256 and at
// most kMaxRows rows per workgroup run the whole step as one launch of
// kPerCU workgroups per compute unit, every workgroup resident at once, with
// grid barriers between the passes.  Workgroup b owns a strip: rows [r0, r1)
// of one 2048-column group; wave w of it owns the strip's columns
// 2048 cg + 256 w .. + 255, four consecutive columns per lane.  The first
// lds_rows rows of the strip stay in LDS from the statistics pass on; every
// pass streams the other rows through buffer loads, two batches of kBatch
// rows in flight per wave (registers go to loads in flight rather than to
// holding evidence: with fewer loads in flight the passes wait on memory
// latency), and walks them against the previous pass's direction so that it
// starts on the rows the Infinity Cache received last.
//
//   A  row partials (per wave, combined over the waves in order) and column
//      partials (per lane over the strip's rows in order)
//   -- barrier --
//      column sums (each workgroup a slice of the columns) -> col_v, column
//      factors; row statistics of the strip's rows -> row_v (by the first
//      column group's workgroup), clamped-row partial
//   -- barrier --
//   B  sqrt of the mean row statistic, row factors; sum of U^2 (and, with
//      spec, the momentum at divisor 1: new block scales, sum of m^2)
//   -- barrier --
//   C  clip divisor; unless spec held it to 1: the momentum, new block
//      scales, sum of m^2
//   -- barrier --
//   D  step size; stochastic rounding, requantization, packing, flips; the
//      new block scales into moment_scale; one 64-bit atomic per workgroup
//      adds its flips and its arrival, and the last to arrive writes the
//      total.
//
// Every value that crosses workgroups (partials, factors) is written with
// agent-scope atomic stores and read with agent-scope atomic loads, which are
// coherent across the XCDs' L2 caches, and every thread waits for its stores
// to complete before its workgroup arrives at a barrier; the evidence, read
// only, and values a workgroup passes to itself take ordinary loads and
// stores.  A barrier that waits longer than kSpinLimit polls (seconds) sets
// the error word and lets the workgroup go on, so every launch ends; the
// flip count is then -1.  The arithmetic is the multi-launch path's,
// element by element; reductions are in double and in a fixed order, so a
// call is deterministic.
namespace fused {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;  // 8
constexpr int kTile = 256 * kWaves;       // columns per workgroup
constexpr int kMaxRows = 128;             // rows per workgroup
constexpr int kPerCU = 2;                 // workgroups per compute unit (4 waves per SIMD)
constexpr int kBatch = 4;                 // rows of a wave's strip loaded together (two batches in flight)
constexpr int kLdsTotal = 160 * 1024 / kPerCU;  // LDS per workgroup (gfx950: 160 KiB per compute unit)
constexpr uint32_t kSpinLimit = 1u << 21;  // polls of about 1 us
constexpr int kSyncWords = 64 * 11;       // [0] barrier total, [64 (1 + g)] group g, [576] flips (64 bits), [640] error
constexpr int kSyncFlips = 64 * 9, kSyncError = 64 * 10;
constexpr uint32_t kDead = 0x80000000u;   // lane offset past every strip: the load returns 0, reads nothing

struct FWork {
  unsigned* sync;       // kSyncWords, zeroed by sync_clear_kernel
  double* colpart;      // [nwg][kTile]
  double* rowpart;      // [cgs][rows]
  float* col_factor;    // [cols]
  double* clamp_part;   // [wpc]
  double* usq_part;     // [nwg]
  double* msq_part;     // [nwg]
  uint16_t* s_new;      // [blocks]
  float* s_rcp;         // [blocks]
  float* scalars;       // [4]
  int wpc;              // workgroups per column group
  int cgs;              // column groups
  int lds_rows;         // rows of a wave's strip held in LDS
};

__device__ __forceinline__ void st_agent(double* p, double v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int64_t* p, int64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), static_cast<uint64_t>(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_agent(const double* p) {
  return __builtin_bit_cast(double, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ int64_t ld_agent(const int64_t* p) {
  return static_cast<int64_t>(
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ unsigned add_agent(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every load and store this thread issued has completed.
__device__ __forceinline__ void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Grid barrier number `gen` (1, 2, ...) of this launch.  Workgroups arrive
// at one of eight group counters (b % 8); the last of a group adds one to
// the total, which every workgroup then polls.
__device__ __forceinline__ void grid_barrier(unsigned* sync, unsigned gen) {
  drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned g = blockIdx.x & 7u;
    const unsigned gsize = (gridDim.x - g + 7u) >> 3;
    const unsigned groups = gridDim.x < 8u ? gridDim.x : 8u;
    if (add_agent(sync + 64 * (1 + g), 1u) + 1u == gen * gsize) add_agent(sync, 1u);
    uint32_t spins = 0;
    while (ld_agent(sync) < gen * groups) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSpinLimit) {
        add_agent(sync + kSyncError, 1u);
        break;
      }
    }
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__global__ void sync_clear_kernel(unsigned* sync) {
  for (int i = threadIdx.x; i < kSyncWords; i += blockDim.x) sync[i] = 0u;
}

typedef __attribute__((address_space(3))) void lds_t;

// Buffer resource over `bytes` bytes at `base` (loads past the end read 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t strip_rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFll ? 0xFFFFFFFFu : static_cast<uint32_t>(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(n), 0x00020000);
}

// What a pass reads of one row of a wave's strip.
enum : int { kNeedE = 1, kNeedQ = 2, kNeedFinal = 4 };

struct RowIn {
  float4 v;          // evidence (rows in memory; LDS rows are read when used)
  uint32_t q4, c4;   // int8 momentum, int8 coordinates
  uint32_t old;      // packed byte holding this lane's four signs
  uint32_t s16;      // new fp16 block scale
  float s_old, rdec;
};

__global__ __launch_bounds__(kThreads, kPerCU) void fused_step_kernel(const float* __restrict__ g, int8_t* __restrict__ coord,
                                                              uint8_t* __restrict__ packed,
                                                              int8_t* __restrict__ moment_q,
                                                              uint16_t* __restrict__ moment_scale,
                                                              uint16_t* __restrict__ row_v,
                                                              uint16_t* __restrict__ col_v, Params p, FWork w,
                                                              int64_t* __restrict__ flips_out) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red[kMaxRows * kWaves];  // row partials per wave; later the column-sum slots
  __shared__ float rowf[kMaxRows];           // new row statistic, then the row factor
  __shared__ float rowv_prev[kMaxRows];      // row_v before this step
  __shared__ double bred[kWaves];
  __shared__ int64_t ired[kWaves];
  float4* stage = reinterpret_cast<float4*>(dyn);

  const bool on = enabled(p);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x;
  const int cg = b / w.wpc, part = b - cg * w.wpc;
  const int64_t r0 = p.rows * part / w.wpc;
  const int nrows = static_cast<int>(p.rows * (part + 1) / w.wpc - r0);
  const int nL = nrows < w.lds_rows ? nrows : w.lds_rows;  // strip rows 0 .. nL-1 stay in LDS
  const int64_t cols = p.cols;
  const int64_t col = static_cast<int64_t>(cg) * kTile + 256 * wave + 4 * lane;
  const int64_t flat0 = r0 * cols + col;  // flat index of this lane's first element of the strip
  const uint32_t row_bytes = static_cast<uint32_t>(cols * 4);
  const __amdgpu_buffer_rsrc_t strip = strip_rsrc(g + r0 * cols, static_cast<int64_t>(nrows) * cols * 4);
  const uint32_t voff = static_cast<uint32_t>(col * 4);
  float4* st = stage + wave * kWave + lane;  // LDS row j of this lane: st[j * kThreads]
  const int nb = (nrows + kBatch - 1) / kBatch;
  // A SIMD holds four waves of this kernel: waves w and w + 4 of two
  // workgroups.  With priority ties everywhere the oldest of them streamed
  // its rows ~40% faster than the youngest, so every pass ended on a tail of
  // young waves; the passes rotate each wave's priority per batch of rows
  // (rotate_priority), offset by its rank among the four.  The grid holds
  // two workgroups per CU, its first half taking one slot on every CU and
  // the second half the other.
  const int prank = __builtin_amdgcn_readfirstlane((wave >> 2) + 2 * (b >= static_cast<int>(gridDim.x >> 1)));

  for (int t = threadIdx.x; t < nrows; t += kThreads) rowv_prev[t] = f16_to_f32(row_v[r0 + t]);

  // Strip row at position `pos` of a pass's walk: forward, or backward so
  // that a pass starts on the rows the previous one read last.
  auto row_at = [&](int pos, bool fwd) { return __builtin_amdgcn_readfirstlane(fwd ? pos : nrows - 1 - pos); };
  // Per-row operands through buffer instructions: a wave-uniform byte
  // offset per row (scalar), the lane's column offset (vector).  The block
  // scales of row i start at block (r0 + i) * cols >> shift (cols is a
  // multiple of 256 and block_size divides 256, so rows hold whole blocks).
  const int bshift = p.block_shift;
  const int64_t blk0 = (r0 * cols) >> bshift;                 // first block of the strip
  const int64_t nblk = (static_cast<int64_t>(nrows) * cols) >> bshift;
  const uint32_t row_blocks = static_cast<uint32_t>(cols >> bshift);
  const __amdgpu_buffer_rsrc_t rq = strip_rsrc(moment_q + r0 * cols, static_cast<int64_t>(nrows) * cols);
  const __amdgpu_buffer_rsrc_t rc8 = strip_rsrc(coord + r0 * cols, static_cast<int64_t>(nrows) * cols);
  const __amdgpu_buffer_rsrc_t rpk = strip_rsrc(packed + (r0 * cols >> 3), static_cast<int64_t>(nrows) * cols / 8);
  const __amdgpu_buffer_rsrc_t rso = strip_rsrc(moment_scale + blk0, nblk * 2);
  const __amdgpu_buffer_rsrc_t rsn = strip_rsrc(w.s_new + blk0, nblk * 2);
  const __amdgpu_buffer_rsrc_t rsr = strip_rsrc(w.s_rcp + blk0, nblk * 4);
  const uint32_t vq = static_cast<uint32_t>(col);             // byte offset of the lane's 4 int8 values
  const uint32_t vpk = static_cast<uint32_t>(col >> 3);       // its packed byte
  const uint32_t vblk = static_cast<uint32_t>(col >> bshift); // its block within the row
  // Loads of strip row i (i < 0: nothing; evidence only for rows in memory).
  auto load = [&](auto need_tag, int i, RowIn& in) {
    constexpr int NEED = decltype(need_tag)::value;
    const bool live = i >= 0;
    const uint32_t ic = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(live ? i : 0));
    if (NEED & kNeedE) {
      // LDS rows and positions past the strip read nothing: a lane offset
      // past the buffer's end returns zeros without a memory access
      const bool mem = live && static_cast<int>(ic) >= nL;
      in.v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(strip, mem ? voff : kDead, ic * row_bytes, 0));
    }
    const uint32_t rowb = ic * static_cast<uint32_t>(cols);  // byte offset of the row's int8 values
    const uint32_t rblk = ic * row_blocks;                    // the row's first block
    if (NEED & (kNeedQ | kNeedFinal)) {
      in.q4 = __builtin_amdgcn_raw_buffer_load_b32(rq, vq, rowb, 0);
      in.s_old = f16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rso, 2 * vblk, 2 * rblk, 0));
    }
    if (NEED & kNeedFinal) {
      in.c4 = __builtin_amdgcn_raw_buffer_load_b32(rc8, vq, rowb, 0);
      in.old = __builtin_amdgcn_raw_buffer_load_b8(rpk, vpk, rowb >> 3, 0);
      in.s16 = __builtin_amdgcn_raw_buffer_load_b16(rsn, 2 * vblk, 2 * rblk, 0);
      in.rdec = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsr, 4 * vblk, 4 * rblk, 0));
    }
  };
  // One pass over the strip: two batches of kBatch rows in flight, the
  // evidence of LDS rows read from LDS when used.
  auto sweep = [&](auto need_tag, bool fwd, auto&& op) {
    RowIn cur[kBatch], nxt[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) load(need_tag, u < nrows ? row_at(u, fwd) : -1, cur[u]);
    for (int k = 0; k < nb; ++k) {
      rotate_priority(k + prank);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int pos = (k + 1) * kBatch + u;
        load(need_tag, pos < nrows ? row_at(pos, fwd) : -1, nxt[u]);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int pos = k * kBatch + u;
        if (pos < nrows) {
          const int i = row_at(pos, fwd);
          if (i < nL) cur[u].v = st[i * kThreads];
          op(i, cur[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) cur[u] = nxt[u];
    }
    __builtin_amdgcn_s_setprio(0);
  };
  using E_ = std::integral_constant<int, kNeedE>;
  using EQ_ = std::integral_constant<int, kNeedE | kNeedQ>;
  using EF_ = std::integral_constant<int, kNeedE | kNeedFinal>;

  // ---- A: statistics -----------------------------------------------------------
  double c0 = 0.0, c1 = 0.0, c2 = 0.0, c3 = 0.0;
  auto stats = [&](int i, const RowIn& in) {
    const float4 v = in.v;
    const double d0 = square_eps(v.x), d1 = square_eps(v.y), d2 = square_eps(v.z), d3 = square_eps(v.w);
    c0 += d0; c1 += d1; c2 += d2; c3 += d3;
    const double rp = wave_total((d0 + d1) + (d2 + d3));
    if (lane == 0) red[i * kWaves + wave] = rp;
  };
  // the LDS rows by direct loads (no registers), all in flight together;
  // lane l of a wave lands at the wave's row base + 16 l
  for (int j = 0; j < nL; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(strip, (lds_t*)(stage + j * kThreads + wave * kWave), 16, voff,
                                             static_cast<int>(static_cast<uint32_t>(j) * row_bytes), 0, 0);
  // rows in memory first (the walk skips the LDS rows), then the LDS rows
  {
    const int nm = nrows - nL, nbm = (nm + kBatch - 1) / kBatch;
    RowIn cur[kBatch], nxt[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) load(E_{}, u < nm ? nL + u : -1, cur[u]);
    for (int k = 0; k < nbm; ++k) {
      rotate_priority(k + prank);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int pos = (k + 1) * kBatch + u;
        load(E_{}, pos < nm ? nL + pos : -1, nxt[u]);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (k * kBatch + u < nm) stats(nL + k * kBatch + u, cur[u]);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) cur[u] = nxt[u];
    }
  }
  __builtin_amdgcn_s_setprio(0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads have landed in LDS
  for (int j = 0; j < nL; ++j) {
    RowIn in;
    in.v = st[j * kThreads];
    stats(j, in);
  }
  {
    double* cp = w.colpart + (static_cast<int64_t>(cg) * w.wpc + part) * kTile + 256 * wave + 4 * lane;
    st_agent(cp + 0, c0);
    st_agent(cp + 1, c1);
    st_agent(cp + 2, c2);
    st_agent(cp + 3, c3);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nrows; t += kThreads) {
    const double* rr = red + t * kWaves;
    const double s = ((rr[0] + rr[1]) + (rr[2] + rr[3])) + ((rr[4] + rr[5]) + (rr[6] + rr[7]));
    st_agent(w.rowpart + static_cast<int64_t>(cg) * p.rows + r0 + t, s);
  }
  grid_barrier(w.sync, 1);

  // ---- column and row statistics --------------------------------------------------
  {
    // workgroup b sums columns [b cpw, (b + 1) cpw): thread (cl, sub) the
    // partials sub, sub + nsub, ... of column cl, then the nsub sums in order
    const int cpw = static_cast<int>((cols + gridDim.x - 1) / gridDim.x);
    const int nsub = kThreads / cpw;
    const int cl = threadIdx.x % cpw, sub = threadIdx.x / cpw;
    const int64_t c = static_cast<int64_t>(b) * cpw + cl;
    double s = 0.0;
    if (sub < nsub && c < cols) {
      const int ccg = static_cast<int>(c / kTile);
      const double* src = w.colpart + static_cast<int64_t>(ccg) * w.wpc * kTile + (c - static_cast<int64_t>(ccg) * kTile);
      for (int k0 = sub; k0 < w.wpc; k0 += 8 * nsub) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = k0 + u * nsub;
          v[u] = k < w.wpc ? ld_agent(src + static_cast<int64_t>(k) * kTile) : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
      }
    }
    __syncthreads();  // every row partial in red was read before the barrier
    if (sub < nsub) red[sub * cpw + cl] = s;
    __syncthreads();
    if (threadIdx.x < cpw && c < cols) {
      double t = 0.0;
      for (int k = 0; k < nsub; ++k) t += red[k * cpw + threadIdx.x];
      const float mean = static_cast<float>(t) / static_cast<float>(p.rows);
      const float nc = fmaf(mean, p.a2, f16_to_f32(col_v[c]) * p.b2);
      if (on) col_v[c] = f32_to_f16(nc);
      st_agent(w.col_factor + c, 1.0f / sqrtf(fmaxf(nc, 1e-10f)));
    }
  }
  {
    double acc = 0.0;
    for (int t = threadIdx.x; t < nrows; t += kThreads) {
      double v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[k] = k < w.cgs ? ld_agent(w.rowpart + static_cast<int64_t>(k) * p.rows + r0 + t) : 0.0;
      double s = 0.0;
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[k];
      const float mean = static_cast<float>(s) / static_cast<float>(cols);
      const float nr = fmaf(mean, p.a2, rowv_prev[t] * p.b2);
      if (cg == 0 && on) row_v[r0 + t] = f32_to_f16(nr);
      rowf[t] = nr;
      acc += static_cast<double>(fmaxf(nr, 1e-10f));
    }
    acc = block_sum(acc, bred);
    if (cg == 0 && threadIdx.x == 0) st_agent(w.clamp_part + part, acc);
  }
  grid_barrier(w.sync, 2);

  // ---- B: factors, sum of U^2 ------------------------------------------------------
  {
    double a = 0.0;
    for (int k = threadIdx.x; k < w.wpc; k += kThreads) a += ld_agent(w.clamp_part + k);
    a = block_sum(a, bred);
    const float sqrt_mean = sqrtf(static_cast<float>(a) / static_cast<float>(p.rows));
    if (b == 0 && threadIdx.x == 0) w.scalars[0] = sqrt_mean;
    for (int t = threadIdx.x; t < nrows; t += kThreads) rowf[t] = row_factor_of(sqrt_mean, rowf[t]);
  }
  float cf[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) cf[e] = ld_agent(w.col_factor + col + e);
  __syncthreads();

  const int gsize = static_cast<int>(p.block_size >> 2);  // lanes per momentum block
  double usq = 0.0, msq = 0.0;
  // U of one row; with MOM the momentum (DIV: U / divisor), block scales,
  // m^2.  GS: lanes per momentum block when known at compile time (64 for
  // the default block of 256), 0 for the run-time gsize.
  auto row_op = [&](auto usq_on, auto mom_on, auto div_on, auto gs_tag, int i, const RowIn& in, float divisor,
                    float rdiv) {
    constexpr bool USQ = decltype(usq_on)::value, MOM = decltype(mom_on)::value, DIV = decltype(div_on)::value;
    constexpr int GS = decltype(gs_tag)::value;
    const float rf = rowf[i];
    const float4 v = in.v;
    const float u[4] = {normalized(v.x, rf, cf[0]), normalized(v.y, rf, cf[1]), normalized(v.z, rf, cf[2]),
                        normalized(v.w, rf, cf[3])};
    if (USQ) {
      const float s0 = u[0] * u[0], s1 = u[1] * u[1], s2 = u[2] * u[2], s3 = u[3] * u[3];
      usq += (static_cast<double>(s0) + static_cast<double>(s1)) + (static_cast<double>(s2) + static_cast<double>(s3));
    }
    if (MOM) {
      float amax = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float ue = DIV ? div_by(u[e], divisor, rdiv) : u[e];
        const float prev = static_cast<float>(static_cast<int8_t>(in.q4 >> (8 * e)));
        const float m = moment_of(ue, prev, in.s_old, p);
        amax = fmaxf(amax, fabsf(m));
        const float sq = m * m;
        msq += static_cast<double>(sq);
      }
      const int gs = GS ? GS : gsize;
      amax = GS ? group_max_last_n<GS>(amax) : group_max_last(amax, gsize);
      if ((lane & (gs - 1)) == gs - 1) {
        const uint32_t ic = static_cast<uint32_t>(i);
        const uint16_t s16 = f32_to_f16(fmaxf(amax, 1e-6f) / 127.0f);
        __builtin_amdgcn_raw_buffer_store_b16(s16, rsn, 2 * vblk, 2 * ic * row_blocks, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, 1.0f / fmaxf(f16_to_f32(s16), 1e-12f)),
                                              rsr, 4 * vblk, 4 * ic * row_blocks, 0);
      }
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using G64_ = std::integral_constant<int, 64>;
  using G0_ = std::integral_constant<int, 0>;
  const bool spec = p.spec, g64 = gsize == 64;
  if (spec && g64)
    sweep(EQ_{}, false, [&](int i, const RowIn& in) { row_op(T_{}, T_{}, F_{}, G64_{}, i, in, 1.0f, 1.0f); });
  else if (spec)
    sweep(EQ_{}, false, [&](int i, const RowIn& in) { row_op(T_{}, T_{}, F_{}, G0_{}, i, in, 1.0f, 1.0f); });
  else
    sweep(E_{}, false, [&](int i, const RowIn& in) { row_op(T_{}, F_{}, F_{}, G0_{}, i, in, 1.0f, 1.0f); });
  usq = block_sum(usq, bred);
  if (threadIdx.x == 0) st_agent(w.usq_part + b, usq);
  if (spec) {
    msq = block_sum(msq, bred);
    if (threadIdx.x == 0) st_agent(w.msq_part + b, msq);
  }
  grid_barrier(w.sync, 3);

  // ---- C: clip divisor, momentum -----------------------------------------------------
  float divisor;
  {
    double a = 0.0;
    for (int k = threadIdx.x; k < static_cast<int>(gridDim.x); k += kThreads) a += ld_agent(w.usq_part + k);
    a = block_sum(a, bred);
    float rms = sqrtf(static_cast<float>(a) / static_cast<float>(p.count));
    rms = fmaxf(rms, 1e-8f);
    const float ratio = rms / p.clip;
    divisor = ratio > 1.0f ? ratio : 1.0f;
    if (b == 0 && threadIdx.x == 0) w.scalars[1] = divisor;
  }
  const float rdiv = 1.0f / divisor;
  bool fwd_d = true;  // the final pass walks against the pass before it
  if (!(spec && divisor == 1.0f)) {
    msq = 0.0;
    if (g64)
      sweep(EQ_{}, true, [&](int i, const RowIn& in) { row_op(F_{}, T_{}, T_{}, G64_{}, i, in, divisor, rdiv); });
    else
      sweep(EQ_{}, true, [&](int i, const RowIn& in) { row_op(F_{}, T_{}, T_{}, G0_{}, i, in, divisor, rdiv); });
    msq = block_sum(msq, bred);
    if (threadIdx.x == 0) st_agent(w.msq_part + b, msq);
    grid_barrier(w.sync, 4);
    fwd_d = false;
  }

  // ---- D: rounding, requantization, packing --------------------------------------------
  float step_size;
  {
    double a = 0.0;
    for (int k = threadIdx.x; k < static_cast<int>(gridDim.x); k += kThreads) a += ld_agent(w.msq_part + k);
    a = block_sum(a, bred);
    const float padded = static_cast<float>(p.blocks * p.block_size);
    float mrms = sqrtf(static_cast<float>(a) / padded);
    mrms = fmaxf(mrms, 1e-8f);
    step_size = step_size_of(mrms, p.lr);
    if (b == 0 && threadIdx.x == 0) {
      w.scalars[2] = step_size;
      w.scalars[3] = mrms;
    }
  }
  const int64_t step = p.step_device ? *p.step_device : p.step;
  const uint32_t combined = p.seed_part ^ step_hash(step);
  const int shift_nib = 4 * (lane & 1);
  int64_t flips = 0;
  auto final_row = [&](auto div1_tag, int i, const RowIn& in) {
    constexpr bool DIV1 = decltype(div1_tag)::value;
    const float rf = rowf[i];
    const int64_t i0 = flat0 + static_cast<int64_t>(i) * cols;  // flat index of the lane's first element
    const uint32_t head = scramble_head(static_cast<uint32_t>(i0) ^ combined);
    const float decode = fmaxf(f16_to_f32(static_cast<uint16_t>(in.s16)), 1e-12f);
    // A finite block scale bounds every |m| of its block, so the quotient
    // m / decode needs no guard for infinite operands (a NaN m stays NaN
    // either way); a row with an infinite scale takes the guarded division.
    const bool finite = __builtin_amdgcn_ballot_w64(!(decode < INFINITY)) == 0;
    const float gv[4] = {in.v.x, in.v.y, in.v.z, in.v.w};
    uint32_t cn = 0, qn = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float u2 = normalized(gv[e], rf, cf[e]);
      if (!DIV1) u2 = div_by(u2, divisor, rdiv);
      const float prev = static_cast<float>(static_cast<int8_t>(in.q4 >> (8 * e)));
      const float cval = static_cast<float>(static_cast<int8_t>(in.c4 >> (8 * e)));
      const float m = moment_of(u2, prev, in.s_old, p);
      const float delta = m * step_size;
      const float target = cval - delta;
      const float lower = floorf(target);
      const float uu = static_cast<float>(scramble_tail(head ^ static_cast<uint32_t>(e))) * (1.0f / 4294967296.0f);
      const float frac = target - lower;
      float rounded = lower + (uu < frac ? 1.0f : 0.0f);
      rounded = fminf(127.0f, fmaxf(-127.0f, rounded));
      float x;
      if (finite) {
        const float q0 = m * in.rdec;
        x = fmaf(fmaf(-q0, decode, m), in.rdec, q0);
      } else {
        x = div_by(m, decode, in.rdec);
      }
      // clamp(rint(x)) == rint(clamp(x)) for integer bounds; adding 1.5 * 2^23
      // rounds to the nearest integer, ties to even, into the low byte
      const float q = fminf(127.0f, fmaxf(-127.0f, x)) + 12582912.0f;
      cn |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(rounded))) << (8 * e);
      qn |= (__float_as_uint(q) & 0xFFu) << (8 * e);
    }
    // sign bits: a coordinate >= 0 has bit 7 of its byte clear; the
    // multiply gathers bits 7, 15, 23, 31 into bits 28..31
    const uint32_t nib = ((~cn & 0x80808080u) * 0x00204081u) >> 28;
    // the other half of the packed byte comes from the neighbouring lane
    const uint32_t other = static_cast<uint32_t>(__shfl_xor(static_cast<int>(nib), 1));
    if (on) {
      const uint32_t rowb = static_cast<uint32_t>(i) * static_cast<uint32_t>(cols);
      __builtin_amdgcn_raw_buffer_store_b32(cn, rc8, vq, rowb, 0);
      __builtin_amdgcn_raw_buffer_store_b32(qn, rq, vq, rowb, 0);
      if ((lane & 1) == 0)
        __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(nib | (other << 4)), rpk, vpk, rowb >> 3, 0);
      // the block's new scale into place: every lane of the block read the
      // old one before this row's arithmetic
      if ((lane & (gsize - 1)) == gsize - 1)
        __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(in.s16), rso, 2 * vblk,
                                              2 * static_cast<uint32_t>(i) * row_blocks, 0);
    }
    flips += __popc(((in.old >> shift_nib) ^ nib) & 0xFu);
  };
  if (divisor == 1.0f)
    sweep(EF_{}, fwd_d, [&](int i, const RowIn& in) { final_row(T_{}, i, in); });
  else
    sweep(EF_{}, fwd_d, [&](int i, const RowIn& in) { final_row(F_{}, i, in); });
  // flip total: one 64-bit atomic per workgroup adds its flips (shifted
  // by 10 bits) and one arrival; the workgroup that completes the arrivals
  // holds the total.  Integer sums, so the result does not depend on order.
  flips = block_sum(flips, ired);
  if (threadIdx.x == 0) {
    const uint64_t mine = (static_cast<uint64_t>(on ? flips : 0) << 10) | 1u;
    const uint64_t now = __hip_atomic_fetch_add(reinterpret_cast<uint64_t*>(w.sync + kSyncFlips), mine,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    if ((now & 1023u) == gridDim.x && flips_out)
      *flips_out = ld_agent(w.sync + kSyncError) ? int64_t{-1} : static_cast<int64_t>(now >> 10);
  }
}

}  // namespace fused

// -- plan ------------------------------------------------------------------------
constexpr int kSegments = 13;

struct Layout {
  size_t off[kSegments];
  size_t total;
};

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static Layout layout(int64_t rows, int64_t cols, int64_t block_size, Work* w) {
  const int64_t nchunks = (cols + kColChunk - 1) / kColChunk;
  const int64_t nstrips = (rows + kStrip - 1) / kStrip;
  // the row path's stats pass writes one strip per usq workgroup of a chunk
  const int64_t row_strips = nchunks <= kUsqGroups ? kUsqGroups / nchunks : 0;
  const int64_t count = rows * cols;
  const int64_t blocks = (count + block_size - 1) / block_size;
  const size_t sizes[kSegments] = {
      sizeof(double) * static_cast<size_t>((nstrips > row_strips ? nstrips : row_strips) * cols),
      sizeof(double) * kRowsGroups,
      sizeof(double) * static_cast<size_t>(nchunks > 1 ? nchunks * rows : 1),
      sizeof(float) * static_cast<size_t>(rows),
      sizeof(float) * static_cast<size_t>(rows),
      sizeof(float) * static_cast<size_t>(cols),
      sizeof(float) * static_cast<size_t>(cols),
      sizeof(double) * kUsqGroups,
      sizeof(double) * kMomentGroups,
      sizeof(float) * 4,
      sizeof(uint16_t) * static_cast<size_t>(blocks),
      sizeof(int64_t) * kFinalGroups,
      sizeof(float) * static_cast<size_t>(blocks),
  };
  // the scalars block first: both step paths keep it at offset 0
  Layout l{};
  size_t at = 0;
  constexpr int order[kSegments] = {9, 0, 1, 2, 3, 4, 5, 6, 7, 8, 10, 11, 12};
  for (int k = 0; k < kSegments; ++k) {
    const int i = order[k];
    l.off[i] = at;
    at += align_up(sizes[i]);
  }
  l.total = at;
  if (w) {
    w->nchunks = nchunks;
    w->nstrips = nstrips;
  }
  return l;
}

// Layout of the one-launch step's workspace; cgs / wpc from fused_plan.
struct FusedLayout {
  size_t scalars, sync, colpart, rowpart, col_factor, clamp, usq, msq, s_new, s_rcp, total;
};

static FusedLayout fused_layout(int64_t rows, int64_t cols, int64_t block_size, int cgs, int wpc) {
  const int64_t nwg = static_cast<int64_t>(cgs) * wpc;
  const int64_t blocks = (rows * cols + block_size - 1) / block_size;
  FusedLayout l{};
  size_t at = 0;
  auto seg = [&](size_t& off, size_t bytes) {
    off = at;
    at += align_up(bytes);
  };
  seg(l.scalars, sizeof(float) * 4);
  seg(l.sync, sizeof(unsigned) * fused::kSyncWords);
  seg(l.colpart, sizeof(double) * static_cast<size_t>(nwg * fused::kTile));
  seg(l.rowpart, sizeof(double) * static_cast<size_t>(cgs * rows));
  seg(l.col_factor, sizeof(float) * static_cast<size_t>(cols));
  seg(l.clamp, sizeof(double) * static_cast<size_t>(wpc));
  seg(l.usq, sizeof(double) * static_cast<size_t>(nwg));
  seg(l.msq, sizeof(double) * static_cast<size_t>(nwg));
  seg(l.s_new, sizeof(uint16_t) * static_cast<size_t>(blocks));
  seg(l.s_rcp, sizeof(float) * static_cast<size_t>(blocks));
  l.total = at;
  return l;
}

}  // namespace step

// The one-launch step's grid for a shape on the current device: cgs column
// groups of 2048 columns, wpc workgroups (strips of rows) each, one
// workgroup per compute unit, lds_rows rows of each wave's strip in LDS.
// False when the shape takes the multi-launch path: columns not a multiple
// of 2048 (or more than 8 groups), block_size not a power of two in 8..256,
// more than kMaxRows rows per strip, or a device that cannot hold the grid.
struct FusedPlan {
  int cgs, wpc, lds_rows;
  size_t lds_bytes;
};

static bool fused_plan(int64_t rows, int64_t cols, int64_t block_size, FusedPlan* fp) {
  using namespace step::fused;
  if (rows <= 0 || cols <= 0 || cols % kTile != 0 || cols / kTile > 8) return false;
  if (block_size < 8 || block_size > 256 || (block_size & (block_size - 1)) != 0) return false;
  struct Dev {
    int cus = -1;  // workgroups of the step resident at once (kPerCU per compute unit)
    size_t static_lds = 0;
  };
  static Dev cache[64];
  static std::mutex lock;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  Dev d;
  {
    std::lock_guard<std::mutex> hold(lock);
    if (cache[dev].cus < 0) {
      Dev n;
      n.cus = 0;
      hipFuncAttributes attr{};
      int cus = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
          hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(fused_step_kernel)) == hipSuccess) {
        const size_t dyn = static_cast<size_t>(kLdsTotal) - attr.sharedSizeBytes;
        int per_cu = 0;
        if (attr.sharedSizeBytes < static_cast<size_t>(kLdsTotal) &&
            hipFuncSetAttribute(reinterpret_cast<const void*>(fused_step_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(dyn)) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fused_step_kernel, kThreads, dyn) == hipSuccess &&
            per_cu >= kPerCU) {
          n.cus = cus * kPerCU;
          n.static_lds = attr.sharedSizeBytes;
        }
      }
      (void)hipGetLastError();
      cache[dev] = n;
    }
    d = cache[dev];
  }
  if (d.cus <= 0) return false;
  const int cgs = static_cast<int>(cols / kTile);
  int64_t wpc = d.cus / cgs;
  if (wpc > rows) wpc = rows;
  if (wpc < 4) return false;  // a workgroup sums at most 512 columns after the first barrier
  if ((rows + wpc - 1) / wpc > kMaxRows || cgs * wpc > 1023) return false;
  if ((cols + cgs * wpc - 1) / (cgs * wpc) > kThreads) return false;
  const int64_t max_rows = (rows + wpc - 1) / wpc;
  int lds_rows = static_cast<int>((static_cast<size_t>(kLdsTotal) - d.static_lds) / (kThreads * 16));
  if (lds_rows > max_rows) lds_rows = static_cast<int>(max_rows);
  fp->cgs = cgs;
  fp->wpc = static_cast<int>(wpc);
  fp->lds_rows = lds_rows;
  fp->lds_bytes = static_cast<size_t>(lds_rows) * kThreads * 16;
  return true;
}

// Workgroups of final_row_kernel resident at once on the current device
// (compute units x workgroups per unit at its register use), cached per
// device; 0 when the runtime cannot say.
static int64_t resident_final_groups() {
  static int64_t cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step::final_row_kernel, step::kThreads, 0) !=
            hipSuccess)
      return 0;
    cache[dev] = static_cast<int64_t>(cus) * per_cu;
  }
  return cache[dev];
}

size_t coordinate_update_workspace(int64_t rows, int64_t cols, int64_t block_size) {
  if (rows <= 0 || cols <= 0 || block_size <= 0) return 0;
  size_t need = step::layout(rows, cols, block_size, nullptr).total;
  FusedPlan fp;
  if (fused_plan(rows, cols, block_size, &fp)) {
    const size_t f = step::fused_layout(rows, cols, block_size, fp.cgs, fp.wpc).total;
    if (f > need) need = f;
  }
  return need;
}

// Both paths keep the scalars block at the start of the workspace.
size_t coordinate_update_scalars_offset(int64_t, int64_t, int64_t) { return 0; }

int coordinate_update_one_launch(int64_t rows, int64_t cols, int64_t block_size) {
  FusedPlan fp;
  return fused_plan(rows, cols, block_size, &fp) ? 1 : 0;
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
  w.col_part = reinterpret_cast<double*>(base + l.off[0]);
  w.clamp_part = reinterpret_cast<double*>(base + l.off[1]);
  w.row_part = reinterpret_cast<double*>(base + l.off[2]);
  w.new_row = reinterpret_cast<float*>(base + l.off[3]);
  w.row_factor = reinterpret_cast<float*>(base + l.off[4]);
  w.new_col = reinterpret_cast<float*>(base + l.off[5]);
  w.col_factor = reinterpret_cast<float*>(base + l.off[6]);
  w.usq_part = reinterpret_cast<double*>(base + l.off[7]);
  w.msq_part = reinterpret_cast<double*>(base + l.off[8]);
  w.scalars = reinterpret_cast<float*>(base + l.off[9]);
  w.s_new = reinterpret_cast<uint16_t*>(base + l.off[10]);
  w.flips_part = reinterpret_cast<int64_t*>(base + l.off[11]);
  w.s_rcp = reinterpret_cast<float*>(base + l.off[12]);

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
  const bool pow2 = (int64_t{1} << shift) == block_size;
  p.block_shift = pow2 ? shift : -1;
  p.seed_part = seed_hash(seed);
  p.step = step_;
  p.step_device = step_device;
  p.enabled = update_enabled;
  p.vec = (cols % 8 == 0) && pow2 && block_size >= 8 && (reinterpret_cast<uintptr_t>(g) & 15) == 0 &&
          (reinterpret_cast<uintptr_t>(coord) & 7) == 0 && (reinterpret_cast<uintptr_t>(moment_q) & 7) == 0;
  p.small = p.count < (int64_t{1} << 32) && p.blocks * p.block_size < (int64_t{1} << 32);
  p.bpr = (p.small && cols % block_size == 0) ? static_cast<uint32_t>(cols / block_size) : 0u;
  // the usq pass guesses the momentum only where the guess usually holds:
  // the clip divisor is 1 once the second-moment EMA has warmed up (rms(U)
  // falls towards 1), not in the first tens of steps from a fresh state
  p.spec = p.vec && cols % 256 == 0 && block_size >= 4 && block_size <= 256 &&
           (reinterpret_cast<uintptr_t>(moment_q) & 3) == 0 && step_device == nullptr && step_ >= 64;

  FusedPlan fp;
  if (p.vec && (reinterpret_cast<uintptr_t>(coord) & 3) == 0 && (reinterpret_cast<uintptr_t>(moment_q) & 3) == 0 &&
      fused_plan(rows, cols, block_size, &fp)) {
    const FusedLayout fl = fused_layout(rows, cols, block_size, fp.cgs, fp.wpc);
    if (workspace_bytes < fl.total) return QSTE_E_WORKSPACE;
    fused::FWork fw{};
    fw.sync = reinterpret_cast<unsigned*>(base + fl.sync);
    fw.colpart = reinterpret_cast<double*>(base + fl.colpart);
    fw.rowpart = reinterpret_cast<double*>(base + fl.rowpart);
    fw.col_factor = reinterpret_cast<float*>(base + fl.col_factor);
    fw.clamp_part = reinterpret_cast<double*>(base + fl.clamp);
    fw.usq_part = reinterpret_cast<double*>(base + fl.usq);
    fw.msq_part = reinterpret_cast<double*>(base + fl.msq);
    fw.s_new = reinterpret_cast<uint16_t*>(base + fl.s_new);
    fw.s_rcp = reinterpret_cast<float*>(base + fl.s_rcp);
    fw.scalars = reinterpret_cast<float*>(base + fl.scalars);
    fw.wpc = fp.wpc;
    fw.cgs = fp.cgs;
    fw.lds_rows = fp.lds_rows;
    fused::sync_clear_kernel<<<1, 256, 0, stream>>>(fw.sync);
    int rc0 = static_cast<int>(hipGetLastError());
    if (rc0) return rc0;
    fused::fused_step_kernel<<<fp.cgs * fp.wpc, fused::kThreads, fp.lds_bytes, stream>>>(
        g, coord, packed, moment_q, moment_scale, row_v, col_v, p, fw, flips_out);
    return static_cast<int>(hipGetLastError());
  }

  // row path: whole 256-column slots, momentum blocks inside one slot, and
  // at least one usq workgroup per chunk
  const bool row_path = p.vec && cols % 256 == 0 && block_size <= 256 && w.nchunks <= kUsqGroups;
  const unsigned row_groups = static_cast<unsigned>(kUsqGroups / w.nchunks);
  w.parts = row_path ? static_cast<int64_t>(row_groups) * w.nchunks : kUsqGroups;

  int rc;
  if (row_path) {
    w.nstrips = row_groups;
    stats_row_kernel<<<dim3(row_groups, static_cast<unsigned>(w.nchunks)), kThreads, 0, stream>>>(g, row_v, p, w);
  } else {
    stats_kernel<<<dim3(static_cast<unsigned>(w.nchunks), static_cast<unsigned>(w.nstrips)), kThreads, 0, stream>>>(
        g, row_v, p, w);
  }
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  const int col_groups = ceil_div(cols, 16);
  colrow_kernel<<<col_groups + kRowsGroups, kThreads, 0, stream>>>(col_v, row_v, p, w, col_groups);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  if (row_path) {
    const dim3 grid(row_groups, static_cast<unsigned>(w.nchunks));
    elem_row_kernel<false><<<grid, kThreads, 0, stream>>>(g, moment_q, moment_scale, p, w);
    if ((rc = static_cast<int>(hipGetLastError()))) return rc;
    elem_row_kernel<true><<<grid, kThreads, 0, stream>>>(g, moment_q, moment_scale, p, w);
  } else {
    usq_kernel<<<kUsqGroups, kThreads, 0, stream>>>(g, moment_q, moment_scale, p, w);
    if ((rc = static_cast<int>(hipGetLastError()))) return rc;
    moment_kernel<<<kMomentGroups, kThreads, 0, stream>>>(g, moment_q, moment_scale, p, w);
  }
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  const int64_t fchunks = (cols + kFinalChunk - 1) / kFinalChunk;
  const bool final_rows = row_path && fchunks <= kFinalGroups;
  // as many workgroups as the device holds at once (one round, no tail),
  // at most kFinalGroups in all
  const int64_t fit = resident_final_groups();
  const int64_t per_chunk = (fit > 0 ? (fit < kFinalGroups ? fit : kFinalGroups) : kFinalGroups) / fchunks;
  const unsigned final_groups = static_cast<unsigned>(per_chunk > 0 ? per_chunk : 1);
  w.fparts = final_rows ? static_cast<int64_t>(final_groups) * fchunks : kFinalGroups;
  if (final_rows)
    final_row_kernel<<<dim3(final_groups, static_cast<unsigned>(fchunks)), kThreads, 0, stream>>>(
        g, coord, packed, moment_q, moment_scale, p, w);
  else if (p.vec)
    final_vec_kernel<<<kFinalGroups, kThreads, 0, stream>>>(g, coord, packed, moment_q, moment_scale, p, w);
  else
    final_kernel<<<kFinalGroups, kThreads, 0, stream>>>(g, coord, packed, moment_q, moment_scale, p, w);
  if ((rc = static_cast<int>(hipGetLastError()))) return rc;
  finish_kernel<<<ceil_div(p.blocks, kThreads) < 1024 ? ceil_div(p.blocks, kThreads) : 1024, kThreads, 0,
                  stream>>>(moment_scale, flips_out, p, w);
  return static_cast<int>(hipGetLastError());
}

// -- the step without a caller workspace ------------------------------------------
// For callers that cannot allocate (code under graph capture, serving loops,
// harnesses that forbid hipMalloc): the workspace is a file-scope device
// array of kStaticScratchBytes, one copy per GPU, that lives until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol); each device's address comes
// from hipGetSymbolAddress, looked up once per device with that device
// current and kept.  Every call on a GPU shares that GPU's array, so calls
// that overlap on one GPU (different streams, or threads) race on it.  No
// kernel of the step reads a workspace byte it did not write earlier in the
// same call, so nothing has to be cleared between calls.
constexpr size_t kStaticScratchBytes = size_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_lock;
void* scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, or NULL with *rc set.
void* device_scratch(int* rc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = QSTE_E_SHAPE;
    return nullptr;
  }
  std::lock_guard<std::mutex> hold(scratch_lock);
  if (scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      *rc = e != hipSuccess ? static_cast<int>(e) : static_cast<int>(hipErrorInvalidSymbol);
      return nullptr;
    }
    scratch_ptr[dev] = ptr;
  }
  *rc = 0;
  return scratch_ptr[dev];
}
}  // namespace

size_t coordinate_update_static_limit() { return kStaticScratchBytes; }

int launch_coordinate_update_static(const float* g, int8_t* coord, uint8_t* packed, int8_t* moment_q,
                                    uint16_t* moment_scale, uint16_t* row_v, uint16_t* col_v, int64_t rows,
                                    int64_t cols, double beta1, double beta2, double update_clip,
                                    double coordinate_lr, int64_t block_size, int64_t seed, int64_t step_,
                                    const int64_t* step_device, int64_t* flips_out,
                                    const uint8_t* update_enabled, hipStream_t stream) {
  const size_t need = coordinate_update_workspace(rows, cols, block_size);
  if (need > kStaticScratchBytes) return QSTE_E_SCRATCH;
  int rc = 0;
  void* ptr = device_scratch(&rc);
  if (ptr == nullptr) return rc;
  return launch_coordinate_update(g, coord, packed, moment_q, moment_scale, row_v, col_v, rows, cols, beta1, beta2,
                                  update_clip, coordinate_lr, block_size, seed, step_, step_device, flips_out,
                                  update_enabled, ptr, kStaticScratchBytes, stream);
}

}  // namespace qste
