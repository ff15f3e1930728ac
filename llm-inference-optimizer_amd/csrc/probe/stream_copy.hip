// Measurement helper, not part of the kernel ABI: a plain streaming copy in
// the shape that measured fastest on MI355X (one 16-byte packet per lane,
// 256-lane workgroups, one workgroup per 4 KiB, buffer descriptors per
// workgroup, non-temporal loads and stores).  bench.py uses it
// (libmi355_probe.so) to report the device's achievable HBM copy bandwidth,
// and rocprofv3 runs use it to calibrate FETCH_SIZE / WRITE_SIZE against a
// kernel whose traffic is known exactly (read `bytes`, write `bytes`).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void stream_copy(const char* __restrict__ src, char* __restrict__ dst,
                                                      int64_t bytes) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBlock * 16;
  const int64_t left = bytes - first;
  const uint32_t nb = left < kBlock * 16 ? static_cast<uint32_t>(left) : static_cast<uint32_t>(kBlock * 16);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(src) + first, 0, nb, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(dst + first, 0, nb, 0x00020000);
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, threadIdx.x * 16u, 0, 2);
  __builtin_amdgcn_raw_buffer_store_b128(v, rd, threadIdx.x * 16u, 0, 2);
}
}  // namespace

// Copies `bytes` (a multiple of 16; both pointers 16-byte aligned) on
// `stream`.  `max_blocks` is unused (kept for the binding's signature).
// Returns 0, -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_copy(const void* src, void* dst,
                                                                      int64_t bytes, int max_blocks,
                                                                      void* stream) {
  (void)max_blocks;
  if (bytes < 0 || (bytes & 15) || ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15))
    return -1;
  if (bytes == 0) return 0;
  const int64_t grid = (bytes + kBlock * 16 - 1) / (kBlock * 16);
  if (grid > 0x7fffffff) return -1;
  hipLaunchKernelGGL(stream_copy, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const char*>(src), static_cast<char*>(dst), bytes);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
