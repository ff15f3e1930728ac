// RMSNorm kernels for gfx950.
//
// Semantics follow the reference's Triton kernel
// (src/kernels/fused_rmsnorm_triton.py:35-49): per row, the sum of squares is
// accumulated in fp32 and divided by the true n, rstd = 1 / sqrt(var + eps),
// and y = (x * rstd) * w is computed in fp32 and rounded once to y's type.
//
// Three kernels, chosen by the host launcher:
//   rmsnorm_wave_rows   one wave64 per row, n <= 64 * VPL * W.  The row lives in
//                       VGPRs (read from HBM exactly once), the sum of squares
//                       is reduced with DPP + permlane swaps (no LDS), and the
//                       wave's slice of the weight is loaded once into VGPRs
//                       and reused for every row the wave visits.
//   rmsnorm_block_rows  one workgroup per row for wider rows; same scheme, the
//                       per-wave partial sums meet in LDS (double-buffered so
//                       a row costs one barrier).
//   rmsnorm_generic     any n, alignment or dtype mix: scalar loads, two passes
//                       over the row (the second pass re-reads x through L2).
// All three stride over rows (grid-stride), so the launcher can cap the grid at
// what the device holds resident.
#pragma once

#include "common.h"

namespace mi355 {

// rstd exactly as the reference orders it: (sum / n) + eps, sqrt, reciprocal,
// each rounded to fp32 (correctly rounded sqrt and division).
__device__ __forceinline__ float rms_rstd(float sumsq, int n, float eps) {
  const float var = sumsq / static_cast<float>(n);
  return 1.0f / __builtin_sqrtf(var + eps);
}

template <typename TX, typename TW, typename TY, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_wave_rows(const void* __restrict__ x,
                                                         const void* __restrict__ w,
                                                         void* __restrict__ y, int64_t rows, int n,
                                                         int64_t xs, int64_t ys, float eps) {
  constexpr int W = pack_width<TX>::value;
  using XB = typename TX::bits;
  using WB = typename TW::bits;
  using YB = typename TY::bits;
  const int lane = threadIdx.x & 63;
  const int waves_per_block = blockDim.x >> 6;
  const int nvec = n / W;

  Chunk<TW, W> wv[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nvec) wv[k].load(static_cast<const WB*>(w) + static_cast<int64_t>(v) * W);
  }

  const int64_t step = static_cast<int64_t>(gridDim.x) * waves_per_block;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * waves_per_block + (threadIdx.x >> 6); r < rows;
       r += step) {
    const XB* xr = static_cast<const XB*>(x) + r * xs;
    Packet<TX> xv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + 64 * k;
      xv[k].raw = (v < nvec) ? *reinterpret_cast<const u32x4*>(xr + static_cast<int64_t>(v) * W)
                             : u32x4{0u, 0u, 0u, 0u};
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      float f[W];
      xv[k].unpack(f);
#pragma unroll
      for (int e = 0; e < W; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
    }
    const float rstd = rms_rstd(wave_allreduce_sum(ss), n, eps);

    YB* yr = static_cast<YB*>(y) + r * ys;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + 64 * k;
      if (v < nvec) {
        float f[W], o[W];
        xv[k].unpack(f);
#pragma unroll
        for (int e = 0; e < W; ++e) o[e] = (f[e] * rstd) * wv[k].get(e);
        store_chunk<TY, W>(yr + static_cast<int64_t>(v) * W, o);
      }
    }
  }
}

template <typename TX, typename TW, typename TY, int VPL, int BLOCK>
__global__ __launch_bounds__(BLOCK) void rmsnorm_block_rows(const void* __restrict__ x,
                                                            const void* __restrict__ w,
                                                            void* __restrict__ y, int64_t rows, int n,
                                                            int64_t xs, int64_t ys, float eps) {
  constexpr int W = pack_width<TX>::value;
  constexpr int NWAVE = BLOCK / 64;
  using XB = typename TX::bits;
  using WB = typename TW::bits;
  using YB = typename TY::bits;
  __shared__ float partial[2][NWAVE];
  const int tid = threadIdx.x;
  const int nvec = n / W;

  Chunk<TW, W> wv[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = tid + BLOCK * k;
    if (v < nvec) wv[k].load(static_cast<const WB*>(w) + static_cast<int64_t>(v) * W);
  }

  int buf = 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const XB* xr = static_cast<const XB*>(x) + r * xs;
    Packet<TX> xv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = tid + BLOCK * k;
      xv[k].raw = (v < nvec) ? *reinterpret_cast<const u32x4*>(xr + static_cast<int64_t>(v) * W)
                             : u32x4{0u, 0u, 0u, 0u};
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      float f[W];
      xv[k].unpack(f);
#pragma unroll
      for (int e = 0; e < W; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
    }
    ss = wave_allreduce_sum(ss);
    if ((tid & 63) == 0) partial[buf][tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NWAVE; ++i) tot += partial[buf][i];
    buf ^= 1;  // the next row writes the other buffer; this row's barrier orders the reuse
    const float rstd = rms_rstd(tot, n, eps);

    YB* yr = static_cast<YB*>(y) + r * ys;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = tid + BLOCK * k;
      if (v < nvec) {
        float f[W], o[W];
        xv[k].unpack(f);
#pragma unroll
        for (int e = 0; e < W; ++e) o[e] = (f[e] * rstd) * wv[k].get(e);
        store_chunk<TY, W>(yr + static_cast<int64_t>(v) * W, o);
      }
    }
  }
}

template <typename TX, typename TW, typename TY>
__global__ __launch_bounds__(256) void rmsnorm_generic(const void* __restrict__ x,
                                                       const void* __restrict__ w,
                                                       void* __restrict__ y, int64_t rows, int n,
                                                       int64_t xs, int64_t ys, float eps) {
  __shared__ float partial[2][4];
  const int tid = threadIdx.x;
  int buf = 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t xo = r * xs;
    float ss = 0.0f;
    for (int j = tid; j < n; j += 256) {
      const float f = load_elem<TX>(x, xo + j);
      ss = __builtin_fmaf(f, f, ss);
    }
    ss = wave_allreduce_sum(ss);
    if ((tid & 63) == 0) partial[buf][tid >> 6] = ss;
    __syncthreads();
    const float tot = (partial[buf][0] + partial[buf][1]) + (partial[buf][2] + partial[buf][3]);
    buf ^= 1;
    const float rstd = rms_rstd(tot, n, eps);
    const int64_t yo = r * ys;
    for (int j = tid; j < n; j += 256) {
      const float f = load_elem<TX>(x, xo + j);
      store_elem<TY>(y, yo + j, (f * rstd) * load_elem<TW>(w, j));
    }
  }
}

}  // namespace mi355
