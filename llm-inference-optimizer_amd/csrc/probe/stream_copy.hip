// Measurement helper, not part of the kernel ABI: a plain 16-byte-per-lane
// streaming copy.  bench.py uses it (libmi355_probe.so) to measure the
// device's achievable HBM copy bandwidth and to calibrate the FETCH_SIZE /
// WRITE_SIZE counters against a kernel whose traffic is known exactly
// (read `bytes`, write `bytes`).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int kBlock = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kBlock) void stream_copy(const u32x4* __restrict__ src,
                                                      u32x4* __restrict__ dst, int64_t n) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * kBlock * kUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kBlock * kUnroll + threadIdx.x; base < n;
       base += step) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j)
      if (base + j * kBlock < n) v[j] = src[base + j * kBlock];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j)
      if (base + j * kBlock < n) dst[base + j * kBlock] = v[j];
  }
}
}  // namespace

// Copies `bytes` (a multiple of 16; both pointers 16-byte aligned) on
// `stream`.  Returns 0, -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_copy(const void* src, void* dst,
                                                                      int64_t bytes, int max_blocks,
                                                                      void* stream) {
  if (bytes < 0 || (bytes & 15) || ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15))
    return -1;
  if (bytes == 0) return 0;
  const int64_t n = bytes / 16;
  int64_t grid = (n + kBlock * kUnroll - 1) / (kBlock * kUnroll);
  if (max_blocks > 0 && grid > max_blocks) grid = max_blocks;
  hipLaunchKernelGGL(stream_copy, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                     static_cast<u32x4*>(dst), n);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
