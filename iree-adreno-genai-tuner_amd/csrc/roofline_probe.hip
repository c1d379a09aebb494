// Measured-roofline probes (the MI355X counterpart of the reference's gemm/roofline.py:27-70,
// which measures FMA and streaming-read peaks of its device): a 16-byte streaming read over a
// buffer, and an empty kernel that measures the launch floor of a given grid.
#include "q4_common.h"

namespace q4 {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Each thread issues all of its kLoads 16-byte loads up front (consecutive threads read
// consecutive 16-byte words, so every load instruction of a wave covers 1 KB contiguously), then
// folds them; the single store is predicated on a value that never occurs, which keeps the loads
// live without writing anything.
template <int kLoads>
__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ buf, int64_t n16, float* sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kLoads + threadIdx.x;
  u32x4 v[kLoads];
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
    const int64_t i = base + u * 256;
    v[u] = i < n16 ? __builtin_nontemporal_load(buf + i) : u32x4{0, 0, 0, 0};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < kLoads; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == 0x9E3779B9u && threadIdx.x == 0x3FF) sink[0] = __builtin_bit_cast(float, acc);
}

__global__ void empty_kernel() {}

// One wave that sleeps until `ticks` of the constant-rate real-time counter (s_memrealtime) have
// passed since it started, or until `max_iter` sleeps, whichever comes first: a bounded stretch of
// device time that lets the host queue a timed region before the device reaches it.
__global__ void wait_kernel(uint64_t ticks, uint64_t max_iter) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (uint64_t i = 0; i < max_iter; ++i) {
    if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(32);
  }
}

}  // namespace
}  // namespace q4

using namespace q4;

extern "C" int q4_probe_read(const void* buf, int64_t bytes, float* sink, int loads_per_thread, void* stream) {
  if (!buf || !sink) return Q4_ERR_NULL;
  if (bytes <= 0 || bytes % 16) return Q4_ERR_SHAPE;
  if (!aligned(buf, 16)) return Q4_ERR_ALIGN;
  const int64_t n16 = bytes / 16;
  auto grid_for = [&](int L) { return dim3(static_cast<unsigned>((n16 + 256LL * L - 1) / (256LL * L))); };
  const hipStream_t s = as_stream(stream);
  const u32x4* b = static_cast<const u32x4*>(buf);
  switch (loads_per_thread) {
    case 1: hipLaunchKernelGGL(read_kernel<1>, grid_for(1), dim3(256), 0, s, b, n16, sink); break;
    case 2: hipLaunchKernelGGL(read_kernel<2>, grid_for(2), dim3(256), 0, s, b, n16, sink); break;
    case 4: hipLaunchKernelGGL(read_kernel<4>, grid_for(4), dim3(256), 0, s, b, n16, sink); break;
    case 8: hipLaunchKernelGGL(read_kernel<8>, grid_for(8), dim3(256), 0, s, b, n16, sink); break;
    default: return Q4_ERR_SHAPE;
  }
  return launch_status();
}

extern "C" int q4_probe_empty(int grid, int block, void* stream) {
  if (grid <= 0 || block <= 0 || block > 1024) return Q4_ERR_SHAPE;
  hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(block), 0, as_stream(stream));
  return launch_status();
}

extern "C" int q4_probe_wait(int64_t microseconds, void* stream) {
  if (microseconds < 0 || microseconds > 1000 * 1000) return Q4_ERR_RANGE;
  int dev = 0, khz = 0;
  Q4_CHECK_HIP(hipGetDevice(&dev));
  Q4_CHECK_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  if (khz <= 0) return Q4_ERR_UNSUPPORTED;
  const uint64_t ticks = static_cast<uint64_t>(microseconds) * static_cast<uint64_t>(khz) / 1000;
  // s_sleep 32 lasts about 32 * 64 shader clocks (0.85 us at 2.4 GHz), so the sleep cap lets the
  // counter end the loop at any clock down to ~1.4 GHz and ends it by itself within ~7x the request
  // even at a quarter of 2.4 GHz
  const uint64_t max_iter = static_cast<uint64_t>(microseconds) * 2 + 64;
  hipLaunchKernelGGL(wait_kernel, dim3(1), dim3(64), 0, as_stream(stream), ticks, max_iter);
  return launch_status();
}
