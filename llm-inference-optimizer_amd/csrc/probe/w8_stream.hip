// Measurement helpers for the int8 weight-streaming (decode) kernels, not part
// of the kernel ABI.  Each probe moves exactly the bytes a decode GEMV reads,
// with no MFMA, no reduction and no epilogue (every loaded dword is folded
// into one XOR that guards a store the data never trigger, so no load can be
// dropped), to split a kernel's time into its weight stream and the rest:
//
//   read_stream  a read-only stream of `bytes` in the copy probe's shape (one
//                16-byte packet per lane, 256 lanes, one workgroup per 4 KiB,
//                non-temporal): the device's read floor for that many bytes.
//   w8_stream    the weights of an [n, k] int8 matrix read with a decode
//                kernel's launch shape: one workgroup per `rpw` consecutive
//                weight rows, `waves` waves splitting the K range into
//                contiguous pieces, U pieces in flight per wave (all U issued,
//                then all consumed).  Load layouts: one weight row x 1 KiB per
//                load instruction (layout 1), or 8-row groups read through
//                one of the lane layouts WL below, optionally with the x
//                operand's loads in one of the x lane layouts XL.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr uint32_t kOob = 0xfffffff0u;  // past every descriptor: reads 0, no traffic
constexpr uint32_t kMagic = 0x9e3779b9u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 ld_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}
__device__ __forceinline__ u32x4 ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t fold(u32x4 v) { return (v.x ^ v.y) ^ (v.z ^ v.w); }

__global__ __launch_bounds__(256) void read_stream(const char* __restrict__ src, int64_t bytes,
                                                   uint32_t* __restrict__ sink) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 * 16;
  const int64_t left = bytes - first;
  const uint32_t nb = left < 256 * 16 ? static_cast<uint32_t>(left) : 256u * 16u;
  const u32x4 v = ld_nt(rsrc(src + first, nb), threadIdx.x * 16u);
  const uint32_t h = fold(v);
  if (h == kMagic) sink[threadIdx.x] = h;
}

struct StreamParams {
  const int8_t* q;
  int n, k;
  int64_t qs;
  const uint16_t* x;  // [rows, xs] (layout 0 with X only)
  int rows;
  int64_t xs;
  int rpw;  // weight rows per workgroup
  uint32_t* sink;  // >= 1024 dwords
};

// Weight lane layouts of one 1 KiB load instruction (8 weight rows x 128
// bytes, or 4 rows x 256 bytes for WL 3), relative to the 8-row group and the
// 128-column block s:
//   WL 0  lane l: row l % 8, bytes 64 ((l / 8) % 2) + 16 (l / 16)   (w8a16_skinny)
//   WL 2  lane l: row l / 8, bytes 16 (l % 8)                        (lanes in row order)
//   WL 3  rows 4 (s % 2) + (l % 16) / 4, bytes 256 (s / 2) + 16 (l % 4) + 64 (l / 16)
//   WL 4  lane l: row (l % 16) / 2, bytes 16 (l % 2) + 32 (l / 16)   (pairs of lanes on 32 bytes)
// x lane layouts of the two 16-byte loads per block (8 x rows x 128 columns
// of 16-bit x), XL:
//   1  lane l: x row l % 8, byte 2 (64 ((l / 8) % 2) + 16 (l / 16)) and +16  (w8a16_skinny)
//   2  load a: x row l / 16, bytes 16 (l % 16); load b: rows 4 + l / 16
//   3  x rows 2 (s % 4) and 2 (s % 4) + 1, 1 KiB each at byte 1024 (s / 4) + 16 l
//   4  lane l: x row (l % 16) / 2, columns 16 (l % 2) + 32 (l / 16) .. + 8 and + 8 .. + 16
//      (the k of WL 4's bytes)
//   5  x rows 4 (s % 2) + (l % 16) / 4, columns 256 (s / 2) + 16 (l % 4) + 64 (l / 16)
//      .. + 8 and + 8 .. + 16 (the decode kernel's x loads beside WL 3)
// STAGGER rotates each wave's walk over its blocks by the workgroup index.
template <int G, int U, int WL, int XL>
__global__ __launch_bounds__(1024) void w8_stream_mfma_layout(const StreamParams p, int stagger) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwave = blockDim.x >> 6;
  const int n0 = blockIdx.x * p.rpw;
  const int nrows = p.n - n0 < p.rpw ? p.n - n0 : p.rpw;
  const auto rq = rsrc(p.q + static_cast<int64_t>(n0) * p.qs, static_cast<uint32_t>((nrows - 1) * p.qs + p.k));
  __amdgpu_buffer_rsrc_t rx = rq;
  if constexpr (XL != 0) rx = rsrc(p.x, static_cast<uint32_t>(((p.rows - 1) * p.xs + p.k) * 2));
  const int nblk = (p.k + 127) >> 7;
  const int s0 = (nblk * wave) / nwave, s1 = (nblk * (wave + 1)) / nwave;
  const int len = s1 - s0;
  const int rot = stagger && len > 0 ? static_cast<int>(blockIdx.x % static_cast<unsigned>(len)) : 0;
  // weight lane -> (row within the group, byte within the block) for block s
  auto wpos = [&](int s, int& row, int& off) {
    if constexpr (WL == 0) {
      row = lane & 7;
      off = 128 * s + ((lane >> 3) & 1) * 64 + (lane >> 4) * 16;
    } else if constexpr (WL == 2) {
      row = lane >> 3;
      off = 128 * s + 16 * (lane & 7);
    } else if constexpr (WL == 4) {
      row = (lane & 15) >> 1;
      off = 128 * s + 16 * (lane & 1) + 32 * (lane >> 4);
    } else {
      row = 4 * (s & 1) + ((lane & 15) >> 2);
      off = 256 * (s >> 1) + 16 * (lane & 3) + 64 * (lane >> 4);
    }
  };
  uint32_t h = 0;
  for (int i = 0; i < len; i += U) {
    u32x4 w[U][G], xa[U][2];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const bool in = i + j < len;
      int s = s0 + (i + j + rot) % (len > 0 ? len : 1);
      int row, off;
      wpos(s, row, off);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const bool live = in && 8 * g + row < nrows && off < p.k;
        w[j][g] = ld_nt(rq, live ? static_cast<uint32_t>((8 * g + row) * p.qs + off) : kOob);
      }
      if constexpr (XL == 1) {
        const int xr = lane & 7;
        const int c = 128 * s + ((lane >> 3) & 1) * 64 + (lane >> 4) * 16;
        const bool live = in && xr < p.rows && c < p.k;
        const uint32_t o = static_cast<uint32_t>((xr * p.xs + c) * 2);
        xa[j][0] = ld(rx, live ? o : kOob);
        xa[j][1] = ld(rx, live ? o + 16u : kOob);
      } else if constexpr (XL == 2) {
        const int xr = lane >> 4;
        const int c = 128 * s + 8 * (lane & 15);
        const bool la = in && xr < p.rows && c < p.k, lb = in && xr + 4 < p.rows && c < p.k;
        xa[j][0] = ld(rx, la ? static_cast<uint32_t>((xr * p.xs + c) * 2) : kOob);
        xa[j][1] = ld(rx, lb ? static_cast<uint32_t>(((xr + 4) * p.xs + c) * 2) : kOob);
      } else if constexpr (XL == 4) {
        const int xr = (lane & 15) >> 1;
        const int c = 128 * s + 16 * (lane & 1) + 32 * (lane >> 4);
        const bool live = in && xr < p.rows && c < p.k;
        const uint32_t o = static_cast<uint32_t>((xr * p.xs + c) * 2);
        xa[j][0] = ld(rx, live ? o : kOob);
        xa[j][1] = ld(rx, live ? o + 16u : kOob);
      } else if constexpr (XL == 5) {
        const int xr = 4 * (s & 1) + ((lane & 15) >> 2);
        const int c = 256 * (s >> 1) + 16 * (lane & 3) + 64 * (lane >> 4);
        const bool live = in && xr < p.rows && c < p.k;
        const uint32_t o = static_cast<uint32_t>((xr * p.xs + c) * 2);
        xa[j][0] = ld(rx, live ? o : kOob);
        xa[j][1] = ld(rx, live ? o + 16u : kOob);
      } else if constexpr (XL == 3) {
        const int xr = 2 * (s & 3);
        const int c = 512 * (s >> 2) + 8 * lane;
        const bool la = in && xr < p.rows && c < p.k, lb = in && xr + 1 < p.rows && c < p.k;
        xa[j][0] = ld(rx, la ? static_cast<uint32_t>((xr * p.xs + c) * 2) : kOob);
        xa[j][1] = ld(rx, lb ? static_cast<uint32_t>(((xr + 1) * p.xs + c) * 2) : kOob);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) h ^= fold(w[j][g]);
      if constexpr (XL != 0) h ^= fold(xa[j][0]) ^ fold(xa[j][1]);
    }
  }
  if (h == kMagic) p.sink[threadIdx.x] = h;
}

template <int U>
__global__ __launch_bounds__(1024) void w8_stream_row_layout(const StreamParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwave = blockDim.x >> 6;
  const int n0 = blockIdx.x * p.rpw;
  const int nrows = p.n - n0 < p.rpw ? p.n - n0 : p.rpw;
  const auto rq = rsrc(p.q + static_cast<int64_t>(n0) * p.qs, static_cast<uint32_t>((nrows - 1) * p.qs + p.k));
  const int nch = (p.k + 1023) >> 10;
  const int items = nrows * nch;
  const int i0 = (items * wave) / nwave, i1 = (items * (wave + 1)) / nwave;
  uint32_t h = 0;
  for (int i = i0; i < i1; i += U) {
    u32x4 w[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int it = i + j;
      const int r = it / nch, c = 1024 * (it % nch) + 16 * lane;
      const bool live = it < i1 && c < p.k;
      w[j] = ld_nt(rq, live ? static_cast<uint32_t>(r * p.qs + c) : kOob);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < U; ++j) h ^= fold(w[j]);
  }
  if (h == kMagic) p.sink[threadIdx.x] = h;
}

template <int G, int WL, int XL>
const void* mfma_layout_kernel(int u) {
  switch (u) {
    case 1: return reinterpret_cast<const void*>(w8_stream_mfma_layout<G, 1, WL, XL>);
    case 2: return reinterpret_cast<const void*>(w8_stream_mfma_layout<G, 2, WL, XL>);
    case 4: return reinterpret_cast<const void*>(w8_stream_mfma_layout<G, 4, WL, XL>);
    case 8: return G <= 1 ? reinterpret_cast<const void*>(w8_stream_mfma_layout<(G <= 1 ? G : 1), 8, WL, XL>) : nullptr;
    default: return nullptr;
  }
}

template <int WL, int XL>
const void* mfma_layout_kernel_g(int g, int u) {
  if (g == 1) return mfma_layout_kernel<1, WL, XL>(u);
  if (g == 2) return mfma_layout_kernel<2, WL, XL>(u);
  if (g == 4) return mfma_layout_kernel<4, WL, XL>(u);
  return nullptr;
}

template <int WL>
const void* mfma_layout_kernel_x(int xl, int g, int u) {
  switch (xl) {
    case 0: return mfma_layout_kernel_g<WL, 0>(g, u);
    case 1: return mfma_layout_kernel_g<WL, 1>(g, u);
    case 2: return mfma_layout_kernel_g<WL, 2>(g, u);
    case 3: return mfma_layout_kernel_g<WL, 3>(g, u);
    case 4: return mfma_layout_kernel_g<WL, 4>(g, u);
    case 5: return mfma_layout_kernel_g<WL, 5>(g, u);
    default: return nullptr;
  }
}

}  // namespace

// Reads `bytes` (a multiple of 16, src 16-byte aligned) on `stream`; `sink`
// holds at least 256 dwords and is written only if the data fold to a magic
// value.  Returns 0, -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_read(const void* src, int64_t bytes, void* sink,
                                                                      void* stream) {
  if (bytes <= 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(src) & 15) || !sink) return -1;
  const int64_t grid = (bytes + 4095) / 4096;
  if (grid > 0x7fffffff) return -1;
  hipLaunchKernelGGL(read_stream, dim3(static_cast<unsigned>(grid)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const char*>(src), bytes, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Streams the int8 weights q [n, qs] (k columns, q and qs 16-byte aligned)
// with `waves` waves per workgroup over ceil(n / rpw) workgroups, U pieces in
// flight per wave.  layout 1: one row x 1 KiB per load (G 1, no x); layout
// 0, 2, 3 or 4: the weight lane layouts WL above (G 8-row groups per piece),
// with x [rows <= 8, xs] of 16-bit values loaded in x layout xl (1-5) when x is
// not NULL; stagger != 0 rotates each wave's walk by the workgroup index.
// `sink` holds at least 1024 dwords.  Returns 0, -1 on bad arguments, -3 on a
// launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_w8_stream(
    const void* q, int n, int k, int64_t qs, const void* x, int rows, int64_t xs, int rpw, int waves, int g, int u,
    int layout, int xl, int stagger, void* sink, void* stream) {
  if (!q || !sink || n < 1 || k < 16 || (k & 15) || qs < k || (qs & 15) || (reinterpret_cast<uintptr_t>(q) & 15) ||
      waves < 1 || waves > 16 || rpw < 1)
    return -1;
  if (static_cast<int64_t>(rpw) * qs >= (int64_t{1} << 31)) return -1;
  const void* kern = nullptr;
  if (layout != 1) {
    if (rpw > 8 * g || (x && (rows < 1 || rows > 8 || xs < k || (xs & 7) || (reinterpret_cast<uintptr_t>(x) & 15))))
      return -1;
    if (!x) xl = 0;
    else if (xl < 1 || xl > 5) return -1;
    if (layout == 0) kern = mfma_layout_kernel_x<0>(xl, g, u);
    else if (layout == 2) kern = mfma_layout_kernel_x<2>(xl, g, u);
    else if (layout == 3) kern = mfma_layout_kernel_x<3>(xl, g, u);
    else if (layout == 4) kern = mfma_layout_kernel_x<4>(xl, g, u);
  } else if (g == 1 && !x) {
    if (u == 1) kern = reinterpret_cast<const void*>(w8_stream_row_layout<1>);
    else if (u == 2) kern = reinterpret_cast<const void*>(w8_stream_row_layout<2>);
    else if (u == 4) kern = reinterpret_cast<const void*>(w8_stream_row_layout<4>);
    else if (u == 8) kern = reinterpret_cast<const void*>(w8_stream_row_layout<8>);
  }
  if (!kern) return -1;
  StreamParams p{static_cast<const int8_t*>(q), n, k, qs, static_cast<const uint16_t*>(x), rows, xs, rpw,
                 static_cast<uint32_t*>(sink)};
  int st = stagger;
  void* args[] = {&p, &st};
  void* args_row[] = {&p};
  const unsigned grid = static_cast<unsigned>((n + rpw - 1) / rpw);
  if (hipLaunchKernel(kern, dim3(grid), dim3(64 * waves), layout == 1 ? args_row : args, 0,
                      static_cast<hipStream_t>(stream)) != hipSuccess)
    return -3;
  return 0;
}
