// RMSNorm kernels for gfx950, optionally fused with the residual add that
// precedes the norm in a decoder layer.
//
// Semantics follow the reference's Triton kernel
// (src/kernels/fused_rmsnorm_triton.py:35-49): per row, the sum of squares is
// accumulated in fp32 and divided by the true n, rstd = 1 / sqrt(var + eps),
// and y = (x * rstd) * w is computed in fp32 and rounded once to y's type.
// With ADD, the normalised row is h = x + residual, rounded to x's type as the
// unfused `residual + hidden_states` of an HF decoder layer rounds it; h is
// also written out (the next residual), and y = RMSNorm(h).  The add uses the
// same row partition and reduction order, so the fused result is bit-identical
// to the add followed by the plain kernel.
//
// Three kernels, chosen by the host launcher:
//   rmsnorm_wave_rows   one wave64 per row, n <= 64 * VPL * W.  The row lives in
//                       VGPRs (read from HBM exactly once) and the sum of
//                       squares is reduced with DPP + permlane swaps (no LDS).
//                       Each lane's slice of the weight is loaded into VGPRs
//                       together with the row (an L2 hit after the first
//                       wave) and reused for every row the wave visits.
//   rmsnorm_block_rows  one workgroup per row, for rows wider than a wave holds
//                       comfortably; the per-wave partial sums meet in LDS
//                       (double-buffered so a row costs one barrier).
//   rmsnorm_generic     any n, alignment or dtype mix: scalar loads, two passes
//                       over the row (the second pass re-reads the row through
//                       L2).
// Rows and the weight are read through buffer descriptors that span exactly
// one row, so the packets past n need no lane branches, with the non-temporal
// hint on x, residual and the outputs.  All kernels stride over rows; the
// launcher normally gives one wave (or workgroup) per row, which measured
// faster on MI355X than a persistent grid.
#pragma once

#include "common.h"

namespace mi355 {

// Threads per workgroup of the wave-per-row kernel above the decode sizes
// (below them, 64: one wave per workgroup, so a few rows spread over CUs).
constexpr int kRmsWaveBlock = 256;

// Whether the workgroup-per-row kernel keeps the fp32 widening of a lane's
// `packets` row packets (and weight) live from the sum-of-squares pass to the
// scaling pass, instead of re-widening the packed 16-bit form there (fewer
// conversions, more VGPRs): measured on MI355X, 1% faster at 16384 x 3584
// bf16 (39.24 vs 39.62 us, 46 vs 37 VGPRs), for at most 4 packets (8 would
// hold 64 fp32 values a lane and spill).  The wave-per-row kernel re-widens:
// keeping fp32 there gains nothing.
template <int packets>
constexpr bool kKeepF32Block = packets <= 4;

// Kernel parameters, passed by value.  r / ro / rs / ros are used with ADD only.
struct RmsParams {
  const void* x;   // [rows, xs]
  const void* r;   // residual [rows, rs]
  const void* w;   // [n]
  void* y;         // [rows, ys]
  void* ro;        // residual out (h = x + r) [rows, ros]
  int64_t rows;
  int n;
  int64_t xs, rs, ys, ros;  // row strides, in elements
  float eps;
};

// rstd exactly as the reference orders it: (sum / n) + eps, sqrt, reciprocal,
// each rounded to fp32 (correctly rounded sqrt and division).
__device__ __forceinline__ float rms_rstd(float sumsq, int n, float eps) {
  const float var = sumsq / static_cast<float>(n);
  return 1.0f / __builtin_sqrtf(var + eps);
}

// One lane's share of a row: VPL packets with packet index slot + k * stride,
// through buffer descriptors sized to the row, so packets past n read 0 and
// their stores drop.  A row past the last one gets descriptors of 0 bytes:
// every access reads 0 or drops, so a kernel that holds several rows at once
// needs no branch for a ragged last group.
template <typename TX, typename TW, int VPL>
struct RowSlice {
  static constexpr int W = pack_width<TX>::value;
  static constexpr uint32_t WB = W * sizeof(typename TW::bits);  // weight bytes per packet
  Packet<TX> xv[VPL];
  Packet<TX> rv[VPL];  // residual packets (ADD only; dead otherwise)

  __device__ __forceinline__ void load_x(rsrc_t rx, int slot, int stride) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) xv[k].raw = buf_load16(rx, static_cast<uint32_t>(slot + k * stride) * 16u);
  }
  __device__ __forceinline__ void load_residual(rsrc_t rr, int slot, int stride) {
#pragma unroll
    for (int k = 0; k < VPL; ++k) rv[k].raw = buf_load16(rr, static_cast<uint32_t>(slot + k * stride) * 16u);
  }
  // xv <- round(xv + residual), the row the norm then runs on.
  __device__ __forceinline__ void add_residual() {
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      float a[W], b[W];
      xv[k].unpack(a);
      rv[k].unpack(b);
#pragma unroll
      for (int e = 0; e < W; ++e) a[e] += b[e];
      xv[k].pack(a);
    }
  }
  __device__ __forceinline__ void store_row(rsrc_t ro, int slot, int stride) const {
#pragma unroll
    for (int k = 0; k < VPL; ++k) buf_store16(ro, static_cast<uint32_t>(slot + k * stride) * 16u, xv[k].raw);
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
  template <typename TY, bool KEEP_F32>
  __device__ __forceinline__ void store_y(rsrc_t ry, int slot, int stride, float rstd,
                                          BufChunk<TW, W> (&wv)[VPL]) {
    constexpr uint32_t YB = W * sizeof(typename TY::bits);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      if constexpr (!KEEP_F32) {
        reg_barrier(xv[k].raw);  // re-widen x here instead of keeping fp32 copies from sumsq()
#pragma unroll
        for (int d = 0; d < BufChunk<TW, W>::DW; ++d) reg_barrier(wv[k].raw[d]);
      }
      float f[W], o[W];
      xv[k].unpack(f);
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = (f[e] * rstd) * wv[k].get(e);
      buf_store_chunk<TY, W>(ry, static_cast<uint32_t>(slot + k * stride) * YB, o);
    }
  }
};

// Byte extent of row r of a matrix of n-element rows: the whole row, or 0
// past the last row.
template <typename T>
__device__ __forceinline__ uint32_t row_bytes(const RmsParams& p, int64_t r) {
  return r < p.rows ? static_cast<uint32_t>(p.n) * sizeof(typename T::bits) : 0u;
}

// The R rows r0 .. r0 + R - 1 of one iteration: every load of every row is
// issued before the first wait, then (ADD) each row becomes h = x + residual,
// stored as the new residual.
template <typename TX, typename TW, int VPL, int R, bool ADD>
__device__ __forceinline__ void load_rows(RowSlice<TX, TW, VPL> (&row)[R], const RmsParams& p, int64_t r0,
                                          int slot, int stride) {
  using XB = typename TX::bits;
#pragma unroll
  for (int i = 0; i < R; ++i)
    row[i].load_x(make_rsrc(static_cast<const XB*>(p.x) + (r0 + i) * p.xs, row_bytes<TX>(p, r0 + i)), slot, stride);
  if constexpr (ADD) {
#pragma unroll
    for (int i = 0; i < R; ++i)
      row[i].load_residual(make_rsrc(static_cast<const XB*>(p.r) + (r0 + i) * p.rs, row_bytes<TX>(p, r0 + i)), slot,
                           stride);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      row[i].add_residual();
      row[i].store_row(make_rsrc(static_cast<XB*>(p.ro) + (r0 + i) * p.ros, row_bytes<TX>(p, r0 + i)), slot,
                       stride);
    }
  }
}

// One wave64 per R rows (R consecutive rows per wave, all loaded before the
// first reduction).  The grid is normally one-shot; the row loop only repeats
// when a grid is capped.  Each lane loads its weight packets lane + 64 k,
// k < VPL, once (an L2 hit after the first wave) and reuses them for every
// row it visits.
template <typename TX, typename TW, typename TY, int VPL, int R, bool ADD>
__global__ __launch_bounds__(kRmsWaveBlock) void rmsnorm_wave_rows(const RmsParams p) {
  using S = RowSlice<TX, TW, VPL>;
  const int lane = threadIdx.x & 63;
  const int waves_per_block = blockDim.x >> 6;

  BufChunk<TW, S::W> wv[VPL];
  const rsrc_t rw = make_rsrc(p.w, static_cast<uint32_t>(p.n) * sizeof(typename TW::bits));
#pragma unroll
  for (int k = 0; k < VPL; ++k) wv[k].load(rw, static_cast<uint32_t>(lane + 64 * k) * S::WB);

  // The wave's index in its workgroup is wave-uniform; readfirstlane says so,
  // which keeps the row's buffer descriptors in SGPRs (no waterfall loop).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t step = static_cast<int64_t>(gridDim.x) * waves_per_block * R;
  for (int64_t r0 = (static_cast<int64_t>(blockIdx.x) * waves_per_block + wave) * R; r0 < p.rows; r0 += step) {
    S row[R];
    load_rows<TX, TW, VPL, R, ADD>(row, p, r0, lane, 64);
    float ss[R];
#pragma unroll
    for (int i = 0; i < R; ++i) ss[i] = row[i].sumsq();
#pragma unroll
    for (int i = 0; i < R; ++i) ss[i] = wave_allreduce_sum(ss[i]);
#pragma unroll
    for (int i = 0; i < R; ++i)
      row[i].template store_y<TY, false>(
          make_rsrc(static_cast<typename TY::bits*>(p.y) + (r0 + i) * p.ys, row_bytes<TY>(p, r0 + i)), lane, 64,
          rms_rstd(ss[i], p.n, p.eps), wv);
  }
}

// One workgroup per R rows, blockDim.x = 64 * (waves per row) <= 1024
// threads; lane t of the workgroup holds packets t + k * blockDim.x, k < VPL,
// of each of its rows.  Used for rows wider than one wave holds comfortably:
// spreading a row over several waves keeps VGPRs low and the work per wave
// fine-grained.  Per-wave partial sums meet in LDS, double-buffered so an
// iteration (R rows) costs one barrier.
template <typename TX, typename TW, typename TY, int VPL, int R, bool ADD>
__global__ __launch_bounds__(1024) void rmsnorm_block_rows(const RmsParams p) {
  using S = RowSlice<TX, TW, VPL>;
  __shared__ float partial[2][R][16];
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int nwave = nthreads >> 6;

  BufChunk<TW, S::W> wv[VPL];
  const rsrc_t rw = make_rsrc(p.w, static_cast<uint32_t>(p.n) * sizeof(typename TW::bits));
#pragma unroll
  for (int k = 0; k < VPL; ++k) wv[k].load(rw, static_cast<uint32_t>(tid + nthreads * k) * S::WB);

  int buf = 0;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * R; r0 < p.rows; r0 += static_cast<int64_t>(gridDim.x) * R) {
    S row[R];
    load_rows<TX, TW, VPL, R, ADD>(row, p, r0, tid, nthreads);
    float ss[R];
#pragma unroll
    for (int i = 0; i < R; ++i) ss[i] = row[i].sumsq();
#pragma unroll
    for (int i = 0; i < R; ++i) ss[i] = wave_allreduce_sum(ss[i]);
    if ((tid & 63) == 0) {
#pragma unroll
      for (int i = 0; i < R; ++i) partial[buf][i][tid >> 6] = ss[i];
    }
    __syncthreads();
    float tot[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      tot[i] = 0.0f;
      for (int j = 0; j < nwave; ++j) tot[i] += partial[buf][i][j];
    }
    buf ^= 1;  // the next iteration writes the other buffer; this one's barrier orders the reuse
#pragma unroll
    for (int i = 0; i < R; ++i)
      row[i].template store_y<TY, kKeepF32Block<VPL * R>>(
          make_rsrc(static_cast<typename TY::bits*>(p.y) + (r0 + i) * p.ys, row_bytes<TY>(p, r0 + i)), tid,
          nthreads, rms_rstd(tot[i], p.n, p.eps), wv);
  }
}

// Scalar fallback, 256 threads per row.  Pass 1 forms the row (with ADD:
// h = round(x + r), written to ro) and its sum of squares; pass 2 re-reads
// the row -- from ro with ADD, since ro may alias r or x -- and writes y.
// Each element is written and re-read by the same thread, with the
// workgroup barrier (a workgroup-scope release/acquire) in between.
template <typename TX, typename TW, typename TY, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_generic(const RmsParams p) {
  __shared__ float partial[2][4];
  const int tid = threadIdx.x;
  int buf = 0;
  for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
    const int64_t xo = r * p.xs;
    const int64_t ho = r * p.ros;
    float ss = 0.0f;
    for (int j = tid; j < p.n; j += 256) {
      float f = load_elem<TX>(p.x, xo + j);
      if constexpr (ADD) {
        f = quantize<TX>(f + load_elem<TX>(p.r, r * p.rs + j));
        store_elem<TX>(p.ro, ho + j, f);
      }
      ss = __builtin_fmaf(f, f, ss);
    }
    ss = wave_allreduce_sum(ss);
    if ((tid & 63) == 0) partial[buf][tid >> 6] = ss;
    __syncthreads();
    const float tot = (partial[buf][0] + partial[buf][1]) + (partial[buf][2] + partial[buf][3]);
    buf ^= 1;
    const float rstd = rms_rstd(tot, p.n, p.eps);
    const int64_t yo = r * p.ys;
    for (int j = tid; j < p.n; j += 256) {
      const float f = ADD ? load_elem<TX>(p.ro, ho + j) : load_elem<TX>(p.x, xo + j);
      store_elem<TY>(p.y, yo + j, (f * rstd) * load_elem<TW>(p.w, j));
    }
  }
}

}  // namespace mi355
