// RMSNorm kernels for gfx950.
//
// Semantics follow the reference's Triton kernel
// (src/kernels/fused_rmsnorm_triton.py:35-49): per row, the sum of squares is
// accumulated in fp32 and divided by the true n, rstd = 1 / sqrt(var + eps),
// and y = (x * rstd) * w is computed in fp32 and rounded once to y's type.
//
// Three kernels, chosen by the host launcher:
//   rmsnorm_wave_rows   one wave64 per row, n <= 64 * VPL * W.  The row lives in
//                       VGPRs (read from HBM exactly once) and the sum of
//                       squares is reduced with DPP + permlane swaps (no LDS).
//                       Each lane's slice of the weight is loaded into VGPRs
//                       together with the row (an L2 hit after the first
//                       wave) and reused for every row the wave visits.
//   rmsnorm_block_rows  one workgroup per row for wider rows; same scheme, the
//                       per-wave partial sums meet in LDS (double-buffered so
//                       a row costs one barrier).
//   rmsnorm_generic     any n, alignment or dtype mix: scalar loads, two passes
//                       over the row (the second pass re-reads x through L2).
// Rows and the weight are read through buffer descriptors that span exactly
// one row, so the packets past n need no lane branches, with the non-temporal
// hint on x and y.  All three kernels stride over rows; the launcher normally
// gives one wave (or workgroup) per row, which measured faster on MI355X than
// a persistent grid.
#pragma once

#include "common.h"

namespace mi355 {

// rstd exactly as the reference orders it: (sum / n) + eps, sqrt, reciprocal,
// each rounded to fp32 (correctly rounded sqrt and division).
__device__ __forceinline__ float rms_rstd(float sumsq, int n, float eps) {
  const float var = sumsq / static_cast<float>(n);
  return 1.0f / __builtin_sqrtf(var + eps);
}

// Per-lane work shared by the wave and workgroup kernels: load VPL packets of
// row r (packet index p = slot + k * STRIDE) through buffer descriptors sized
// to the row, so packets past n read 0 and their stores drop.
template <typename TX, typename TW, int VPL, int STRIDE>
struct RowSlice {
  static constexpr int W = pack_width<TX>::value;
  static constexpr uint32_t WB = W * sizeof(typename TW::bits);  // weight bytes per packet
  Packet<TX> xv[VPL];

  __device__ __forceinline__ void load_x(rsrc_t rx, int slot) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) xv[k].raw = buf_load16(rx, static_cast<uint32_t>(slot + k * STRIDE) * 16u);
  }
  __device__ __forceinline__ float sumsq() const {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      float f[W];
      xv[k].unpack(f);
#pragma unroll
      for (int e = 0; e < W; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
    }
    return ss;
  }
  template <typename TY>
  __device__ __forceinline__ void store_y(rsrc_t ry, int slot, float rstd, BufChunk<TW, W> (&wv)[VPL]) {
    constexpr uint32_t YB = W * sizeof(typename TY::bits);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      reg_barrier(xv[k].raw);  // re-widen x here instead of keeping fp32 copies from sumsq()
#pragma unroll
      for (int d = 0; d < BufChunk<TW, W>::DW; ++d) reg_barrier(wv[k].raw[d]);
      float f[W], o[W];
      xv[k].unpack(f);
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = (f[e] * rstd) * wv[k].get(e);
      buf_store_chunk<TY, W>(ry, static_cast<uint32_t>(slot + k * STRIDE) * YB, o);
    }
  }
};

// One wave64 per row.  The grid is normally one-shot (a wave per row); the
// row loop only repeats when the launcher caps the grid.
template <typename TX, typename TW, typename TY, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_wave_rows(const void* __restrict__ x,
                                                         const void* __restrict__ w,
                                                         void* __restrict__ y, int64_t rows, int n,
                                                         int64_t xs, int64_t ys, float eps) {
  using S = RowSlice<TX, TW, VPL, 64>;
  using WC = BufChunk<TW, S::W>;
  const int lane = threadIdx.x & 63;
  const int waves_per_block = blockDim.x >> 6;
  const uint32_t xbytes = static_cast<uint32_t>(n) * sizeof(typename TX::bits);
  const uint32_t ybytes = static_cast<uint32_t>(n) * sizeof(typename TY::bits);
  const uint32_t wbytes = static_cast<uint32_t>(n) * sizeof(typename TW::bits);
  const rsrc_t rw = make_rsrc(w, wbytes);
  WC wv[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) wv[k].load(rw, static_cast<uint32_t>(lane + 64 * k) * S::WB);

  // The wave's index in its workgroup is wave-uniform; readfirstlane says so,
  // which keeps the row's buffer descriptor in SGPRs (no waterfall loop).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t step = static_cast<int64_t>(gridDim.x) * waves_per_block;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * waves_per_block + wave; r < rows; r += step) {
    S row;
    row.load_x(make_rsrc(static_cast<const typename TX::bits*>(x) + r * xs, xbytes), lane);
    const float rstd = rms_rstd(wave_allreduce_sum(row.sumsq()), n, eps);
    row.template store_y<TY>(make_rsrc(static_cast<typename TY::bits*>(y) + r * ys, ybytes), lane, rstd, wv);
  }
}

// One workgroup per row, blockDim.x = 64 * (waves per row) <= 1024 threads;
// lane t of the workgroup holds packets t + k * blockDim.x, k < VPL.  Used
// for rows wider than one wave holds and, with VPL small, to spread a row over
// several waves (fewer VGPRs and finer-grained work per wave).  Per-wave
// partial sums meet in LDS, double-buffered so a row costs one barrier.
template <typename TX, typename TW, typename TY, int VPL>
__global__ __launch_bounds__(1024) void rmsnorm_block_rows(const void* __restrict__ x,
                                                           const void* __restrict__ w,
                                                           void* __restrict__ y, int64_t rows, int n,
                                                           int64_t xs, int64_t ys, float eps) {
  constexpr int W = pack_width<TX>::value;
  constexpr uint32_t WB = W * sizeof(typename TW::bits);
  constexpr uint32_t YB = W * sizeof(typename TY::bits);
  __shared__ float partial[2][16];
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int nwave = nthreads >> 6;
  const uint32_t xbytes = static_cast<uint32_t>(n) * sizeof(typename TX::bits);
  const uint32_t ybytes = static_cast<uint32_t>(n) * sizeof(typename TY::bits);

  BufChunk<TW, W> wv[VPL];
  const rsrc_t rw = make_rsrc(w, static_cast<uint32_t>(n) * sizeof(typename TW::bits));
#pragma unroll
  for (int k = 0; k < VPL; ++k) wv[k].load(rw, static_cast<uint32_t>(tid + nthreads * k) * WB);

  int buf = 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const rsrc_t rx = make_rsrc(static_cast<const typename TX::bits*>(x) + r * xs, xbytes);
    Packet<TX> xv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) xv[k].raw = buf_load16(rx, static_cast<uint32_t>(tid + nthreads * k) * 16u);
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
    for (int i = 0; i < nwave; ++i) tot += partial[buf][i];
    buf ^= 1;  // the next row writes the other buffer; this row's barrier orders the reuse
    const float rstd = rms_rstd(tot, n, eps);

    const rsrc_t ry = make_rsrc(static_cast<typename TY::bits*>(y) + r * ys, ybytes);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      reg_barrier(xv[k].raw);
      float f[W], o[W];
      xv[k].unpack(f);
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = (f[e] * rstd) * wv[k].get(e);
      buf_store_chunk<TY, W>(ry, static_cast<uint32_t>(tid + nthreads * k) * YB, o);
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
