// Measurement variant, not part of the kernel ABI: SiLU-and-mul (fp16 in and
// out) on a persistent grid, against the library's one-shot grid of
// silu_mul_chunks.  Workgroup w of G owns the contiguous packets
// [npk * w / G, npk * (w + 1) / G) -- every workgroup within one packet of
// the same share, so no round of workgroups finishes early and leaves the
// CUs idle at the end of the launch -- and walks them B * U packets at a
// time (lane t: packets t + j * B of each step, 1 KiB per wave-wide load),
// issuing the next step's loads before the current step's arithmetic and
// stores.  Same arithmetic and rounding as silu_mul_chunks (silu_mul_f32,
// one rounding), same non-temporal buffer accesses.
#include "../common.h"

namespace {

using mi355::F16;

template <int B, int U>
__global__ __launch_bounds__(B) void silu_mul_persist(const void* __restrict__ gate, const void* __restrict__ up,
                                                      void* __restrict__ out, int64_t npk) {
  constexpr int W = mi355::pack_width<F16>::value;
  const int64_t g = gridDim.x;
  const int64_t lo = npk * blockIdx.x / g, hi = npk * (blockIdx.x + 1) / g;
  const uint32_t count = static_cast<uint32_t>(hi - lo);  // packets of this workgroup
  const mi355::rsrc_t rg = mi355::make_rsrc(static_cast<const char*>(gate) + lo * 16, count * 16u);
  const mi355::rsrc_t ru = mi355::make_rsrc(static_cast<const char*>(up) + lo * 16, count * 16u);
  const mi355::rsrc_t ro = mi355::make_rsrc(static_cast<char*>(out) + lo * 16, count * 16u);

  mi355::Packet<F16> gv[U], uv[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t off = (threadIdx.x + j * B) * 16u;
    gv[j].raw = mi355::buf_load16(rg, off);
    uv[j].raw = mi355::buf_load16(ru, off);
  }
  for (uint32_t base = 0; base < count; base += B * U) {
    mi355::Packet<F16> gn[U], un[U];
    const uint32_t next = base + B * U;
#pragma unroll
    for (int j = 0; j < U; ++j) {  // past `count` the loads read zeros without traffic
      const uint32_t off = (next + threadIdx.x + j * B) * 16u;
      gn[j].raw = mi355::buf_load16(rg, next < count ? off : mi355::kOob);
      un[j].raw = mi355::buf_load16(ru, next < count ? off : mi355::kOob);
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      float gf[W], uf[W], o[W];
      gv[j].unpack(gf);
      uv[j].unpack(uf);
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = mi355::silu_mul_f32(gf[e], uf[e]);
      mi355::buf_store_chunk<F16, W>(ro, (base + threadIdx.x + j * B) * 16u, o);
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      gv[j] = gn[j];
      uv[j] = un[j];
    }
  }
}

template <int B, int U>
int launch_persist(const void* gate, const void* up, void* out, int64_t npk, int grid, hipStream_t s) {
  hipLaunchKernelGGL((silu_mul_persist<B, U>), dim3(grid), dim3(B), 0, s, gate, up, out, npk);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace

// out = silu(gate) * up over `numel` fp16 elements (a multiple of 8; all
// pointers 16-byte aligned) on a persistent grid of `grid` workgroups of
// `block` lanes (256 or 512) moving `unroll` packets per lane per step (1, 2
// or 4).  Each workgroup's share must stay under 2^27 packets.  Returns 0,
// -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_silu_persist(const void* gate, const void* up,
                                                                               void* out, int64_t numel, int grid,
                                                                               int block, int unroll, void* stream) {
  if (numel <= 0 || (numel & 7) || grid < 1 ||
      ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(out)) & 15))
    return -1;
  const int64_t npk = numel / 8;
  if (npk / grid + 1 >= (int64_t{1} << 27)) return -1;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (block == 512 && unroll == 1) return launch_persist<512, 1>(gate, up, out, npk, grid, s);
  if (block == 512 && unroll == 2) return launch_persist<512, 2>(gate, up, out, npk, grid, s);
  if (block == 512 && unroll == 4) return launch_persist<512, 4>(gate, up, out, npk, grid, s);
  if (block == 256 && unroll == 1) return launch_persist<256, 1>(gate, up, out, npk, grid, s);
  if (block == 256 && unroll == 2) return launch_persist<256, 2>(gate, up, out, npk, grid, s);
  if (block == 256 && unroll == 4) return launch_persist<256, 4>(gate, up, out, npk, grid, s);
  return -1;
}
