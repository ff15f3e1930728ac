// Measurement helpers, not part of the kernel ABI: a plain streaming copy in
// the shape that measured fastest on MI355X (one 16-byte packet per lane,
// 256-lane workgroups, one workgroup per 4 KiB, buffer descriptors per
// workgroup, non-temporal loads and stores), and the same stream with two
// inputs and one output (out = a + b as 32-bit integers), the access mix of
// SiLU-and-mul without its arithmetic, and an empty kernel (the fixed cost of
// a launch, eager and as a hipGraph node).  bench.py uses them
// (libmi355_probe.so) to report the device's achievable HBM bandwidth for
// each access mix, at 1 GiB and at the byte counts of the benchmarked
// kernels; rocprofv3 runs use the copy to calibrate FETCH_SIZE / WRITE_SIZE
// against a kernel whose traffic is known exactly (read `bytes`, write
// `bytes`).
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

__global__ __launch_bounds__(kBlock) void stream_add2(const char* __restrict__ a, const char* __restrict__ b,
                                                      char* __restrict__ dst, int64_t bytes) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBlock * 16;
  const int64_t left = bytes - first;
  const uint32_t nb = left < kBlock * 16 ? static_cast<uint32_t>(left) : static_cast<uint32_t>(kBlock * 16);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(a) + first, 0, nb, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(b) + first, 0, nb, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(dst + first, 0, nb, 0x00020000);
  const u32x4 va = __builtin_amdgcn_raw_buffer_load_b128(ra, threadIdx.x * 16u, 0, 2);
  const u32x4 vb = __builtin_amdgcn_raw_buffer_load_b128(rb, threadIdx.x * 16u, 0, 2);
  __builtin_amdgcn_raw_buffer_store_b128(va + vb, rd, threadIdx.x * 16u, 0, 2);
}

__global__ __launch_bounds__(64) void empty_kernel() {}
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

// dst = a + b (32-bit integer lanes) over `bytes` of each (a multiple of 16;
// all pointers 16-byte aligned) on `stream`: reads 2 * bytes, writes bytes.
// Returns 0, -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_add2(const void* a, const void* b, void* dst,
                                                                      int64_t bytes, void* stream) {
  if (bytes < 0 || (bytes & 15) ||
      ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(dst)) & 15))
    return -1;
  if (bytes == 0) return 0;
  const int64_t grid = (bytes + kBlock * 16 - 1) / (kBlock * 16);
  if (grid > 0x7fffffff) return -1;
  hipLaunchKernelGGL(stream_add2, dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const char*>(a), static_cast<const char*>(b),
                     static_cast<char*>(dst), bytes);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// One workgroup of one wave that does nothing, on `stream`.  Returns 0 or -3
// on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_empty(void* stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream));
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
