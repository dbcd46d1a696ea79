// Measurement probes (no counterpart in the reference): a plain streaming
// read, the floor any kernel that reads the same bytes once can reach, and
// the shader clock as a wave sees it.  bench.py and device_profile() use
// them; they compute nothing the operators need.
#include "common.hpp"

namespace qste {
namespace probe {

constexpr int kThreads = 256;
constexpr int kDepth = 8;  // 16-byte loads in flight per thread

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Workgroup b reads [b * per, (b + 1) * per) of the buffer, kDepth loads of
// 16 bytes per thread at a time; lanes read consecutive 16 bytes.  The
// bytes are xor-folded into one word per thread, stored only when it equals
// a value the data cannot produce by chance, so the loads are not removed.
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                               int64_t per, uint32_t* __restrict__ sink) {
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * per;
  const int64_t end = begin + per < n16 ? begin + per : n16;
  uint32_t acc = 0;
  for (int64_t i = begin + threadIdx.x; i < end; i += static_cast<int64_t>(kThreads) * kDepth) {
    u32x4 v[kDepth];
#pragma unroll
    for (int k = 0; k < kDepth; ++k) {
      const int64_t j = i + static_cast<int64_t>(k) * kThreads;
      v[k] = j < end ? src[j] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < kDepth; ++k) acc ^= (v[k].x ^ v[k].y) ^ (v[k].z ^ v[k].w);
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x * kThreads + threadIdx.x] = acc;
}

// One wave: the shader-clock counter (s_memtime) and the 100 MHz real-time
// counter (s_memrealtime) before and after a dependent integer loop.
__global__ void clock_probe_kernel(int64_t* __restrict__ out, int64_t spins) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  uint32_t v = threadIdx.x;
  for (int64_t i = 0; i < spins; ++i) v = v * 1664525u + 1013904223u;
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    out[0] = static_cast<int64_t>(c1 - c0);
    out[1] = static_cast<int64_t>(r1 - r0);
    out[2] = v == 0x12345678u ? 1 : 0;  // keeps the loop
  }
}

}  // namespace probe

int launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t groups, hipStream_t stream) {
  if (bytes <= 0) return 0;
  if (!src || !sink || groups <= 0 || (reinterpret_cast<uintptr_t>(src) & 15) || bytes % 16) return QSTE_E_SHAPE;
  const int64_t n16 = bytes / 16;
  const int64_t per = (n16 + groups - 1) / groups;
  probe::stream_read_kernel<<<static_cast<unsigned>(groups), probe::kThreads, 0, stream>>>(
      static_cast<const probe::u32x4*>(src), n16, per, sink);
  return static_cast<int>(hipGetLastError());
}

int device_info(int64_t* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  const hipDeviceAttribute_t attrs[4] = {hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeClockRate,
                                         hipDeviceAttributeMemoryClockRate,
                                         hipDeviceAttributeMaxSharedMemoryPerMultiprocessor};
  for (int i = 0; i < 4; ++i) {
    int v = 0;
    e = hipDeviceGetAttribute(&v, attrs[i], dev);
    if (e != hipSuccess) return static_cast<int>(e);
    out[i] = v;
  }
  return 0;
}

int launch_clock_probe(int64_t* out, int64_t spins, hipStream_t stream) {
  if (!out || spins <= 0) return QSTE_E_SHAPE;
  probe::clock_probe_kernel<<<1, 64, 0, stream>>>(out, spins);
  return static_cast<int>(hipGetLastError());
}

}  // namespace qste
