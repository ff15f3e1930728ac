// 16-bit linear (nn.Linear's forward with fp16 / bf16 weights) for gfx950,
// plus its launcher:
//
//   out[m, n] = round(acc + bias[n]),  acc = sum_k x[m, k] * w[n, k]   (fp32)
//
// It serves the down projection of FusedMLP: the reference's FusedMLP runs
// `down_proj(fused_silu_mul(gate, up))` (src/engine/fused_norm_activation_
// patch.py:60-64), an nn.Linear that torch sends to hipBLASLt.  At decode
// batch sizes that call reads the whole [n, k] weight matrix for a handful of
// rows, so it is weight streaming, and hipBLASLt runs it far below HBM
// bandwidth (about 21 us for the 27.5 MB down projection of Qwen2.5-1.5B at
// 1 to 8 rows on MI355X).
//
// Three kernels, picked by the launcher:
//   w8a16_stream      rows <= 16 (decode; w8a16_stream.h with one 16-bit
//                     matrix), and 17 - 64 where the small tiled shapes do not
//                     pay: lane-coalesced weight streaming, every weight byte
//                     read once per call, MFMA (v_mfma_f32_16x16x32_*).
//   tiled_gemm        more rows, and 17 - 64 on wide outputs: the LDS-tiled
//                     MFMA GEMM of tiled_gemm.h with the weights as a 16-bit B
//                     operand and the bias in its epilogue (EPI_LINEAR).
//   linear16_generic  any k, stride or alignment the two above cannot take:
//                     one wave per (output feature, 4 rows of x), fp32 fma.
// Under the C ABI's limits (row strides < 2^22 elements) the buffer
// descriptors of the first two always span their inputs.
#include "common.h"
#include "tiled_gemm.h"
#include "w8a16_stream.h"

namespace mi355 {
namespace {

struct L16Params {
  const void* x;       // [rows, xs] of T
  const void* w;       // [n, ws] of T
  const void* bias;    // [n] of bdt, or null
  void* out;           // [rows, os] of TO
  int rows, k, n;
  int64_t xs, ws, os;  // row strides in elements
  int bdt;             // dtype code of the bias (< 0: no bias)
};

// The epilogue shared by the kernels: the bias in fp32, one rounding.
template <typename TO>
__device__ __forceinline__ void l16_store(const L16Params& p, int64_t m, int n, float acc) {
  const float v = p.bdt >= 0 ? acc + load_dyn(p.bias, n, p.bdt) : acc;
  store_elem<TO>(p.out, m * p.os + n, v);
}

// ----------------------------------------------------------------- generic

constexpr int kGenRows = 4;  // rows of x per wave

template <typename T, typename TO>
__global__ __launch_bounds__(256) void linear16_generic(const L16Params p) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t mblocks = (p.rows + kGenRows - 1) / kGenRows;
  if (gw >= static_cast<int64_t>(p.n) * mblocks) return;
  const int n = static_cast<int>(gw % p.n);
  const int64_t m0 = (gw / p.n) * kGenRows;
  const int64_t wrow = static_cast<int64_t>(n) * p.ws;
  float acc[kGenRows] = {};
  for (int c = lane; c < p.k; c += 64) {
    const float wv = load_elem<T>(p.w, wrow + c);
#pragma unroll
    for (int i = 0; i < kGenRows; ++i) {
      if (m0 + i < p.rows) acc[i] = __builtin_fmaf(load_elem<T>(p.x, (m0 + i) * p.xs + c), wv, acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kGenRows; ++i) {
    const float s = wave_allreduce_sum(acc[i]);
    if (lane == 0 && m0 + i < p.rows) l16_store<TO>(p, m0 + i, n, s);
  }
}

// ---------------------------------------------------------------- launchers

template <typename K>
int launch_l16(K kernel, dim3 grid, dim3 block, size_t lds, const L16Params& p, hipStream_t s) {
  void* args[] = {const_cast<L16Params*>(&p)};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, args, lds, s),
                    "linear16 launch");
}

// ------------------------------------------------------------------- tiled

// Buffer descriptors of the tiled GEMM span at most 256 rows of x and 256
// weight rows; both must stay below 2^31 bytes.
bool l16_tiled_fits(const L16Params& p) {
  return int64_t{256} * p.xs * 2 < (int64_t{1} << 31) && int64_t{256} * p.ws * 2 < (int64_t{1} << 31) &&
         static_cast<int64_t>((p.rows + 63) / 64) * ((p.n + 63) / 64) < (int64_t{1} << 31);
}

template <typename T, typename TO, int WGM, int WGN, int FM, int FN, int S, int RING = 0>
int l16_tiled_cfg(const L16Params& p, hipStream_t s) {
  using C = tiled::Cfg<T, tiled::B_16, TO, WGM, WGN, FM, FN, tiled::EPI_LINEAR, S>;
  static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
  tiled::Params tp{};
  tp.x = p.x;
  tp.b0 = p.w;
  tp.b1 = p.w;
  tp.bias = p.bias;
  tp.out = p.out;
  tp.rows = p.rows;
  tp.k = p.k;
  tp.n = p.n;
  tp.xs = p.xs;
  tp.bs = p.ws;
  tp.os = p.os;
  tp.sdt = MI355_F32;
  tp.bdt = p.bdt;
  tp.tiles_m = (p.rows + C::BM - 1) / C::BM;
  tp.tiles_n = (p.n + C::BN - 1) / C::BN;
  tp.group_m = tp.tiles_m < 4 ? tp.tiles_m : 4;
  void* args[] = {&tp};
  // all LDS is static (no dynamic shared memory)
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(tiled::tiled_gemm<T, tiled::B_16, TO, WGM, WGN, FM, FN,
                                                                                      tiled::EPI_LINEAR, S, RING>),
                                    dim3(static_cast<unsigned>(tp.tiles_m * tp.tiles_n)), dim3(C::BLOCK), args, 0, s),
                    "linear16 tiled launch");
}

// Tiled shapes (16-bit B, one matrix): 64 x 64 tiles on small grids, 128 x
// 128 (8 waves, 3 stages) otherwise.
template <typename T, typename TO>
int l16_tiled(const L16Params& p, hipStream_t s) {
  const int64_t t128 = static_cast<int64_t>((p.rows + 127) / 128) * ((p.n + 127) / 128);
  if (t128 < 128) return l16_tiled_cfg<T, TO, 2, 2, 1, 1, 4>(p, s);
  return l16_tiled_cfg<T, TO, 2, 4, 2, 1, 3>(p, s);
}

// Small tiled shapes: 32 x 64 (2 waves) or, for n > 10000, 32 x 128 (4 waves)
// up to 32 rows; 64 x 64 (4 waves) up to 64; 4 stages.  From a sweep over
// the Qwen2.5-1.5B / 7B down and o projections at 16 - 64 rows: at 17 - 32
// rows they lose to split-K weight streaming on these narrow outputs (1.5B
// down, 32 rows: 38.0 vs 22.3 us) unless the output has >= 128 tile
// columns; at 33 - 64 rows, where streaming re-reads the weights per 32-row
// tile, they win (7B down, 48 rows: 85.5 vs 101.6 us; 7B o 19.4 vs 22.6).
template <typename T, typename TO>
int l16_tiled_small(const L16Params& p, hipStream_t s) {
  if (p.rows <= 32) {
    if (p.n > 10000) return l16_tiled_cfg<T, TO, 1, 4, 1, 1, 4>(p, s);
    return l16_tiled_cfg<T, TO, 1, 2, 1, 1, 4>(p, s);
  }
  return l16_tiled_cfg<T, TO, 2, 2, 1, 1, 4>(p, s);
}

template <typename T, typename TO>
int l16_typed(const L16Params& p, hipStream_t s, int cus) {
  const bool vec = p.k % 8 == 0 && p.ws % 8 == 0 && p.xs % 8 == 0 && aligned16(p.x) && aligned16(p.w);
  if (!vec) {
    const int64_t waves = static_cast<int64_t>(p.n) * ((p.rows + kGenRows - 1) / kGenRows);
    return launch_l16(linear16_generic<T, TO>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, p, s);
  }
  // Up to 16 rows, and 17 - 64 where the small tiled shapes do not pay (fewer
  // than 128 tile columns): the weight-streaming kernel of w8a16_stream.h
  // with one 16-bit matrix (1.5B down, 32 rows 22.1 -> 14.4 us against the
  // skinny split-K kernel this launcher ran before, 64 rows 43.7 -> 22.2
  // against the small tiles; 7B down 51.9 -> 37.3 at 32 rows, 90.3 -> 78.8
  // at 64; 0.5B down 13.2 -> 7.9 at 32 rows).  Its x descriptor spans all
  // rows of x and each workgroup's weight descriptor up to 16 weight rows.
  const int64_t tb = sizeof(typename T::bits);
  if (((p.rows < 64 ? p.rows : 64) - 1) * p.xs * tb + p.k * tb >= (int64_t{1} << 32) ||
      (15 * p.ws + p.k) * tb >= (int64_t{1} << 32) || !l16_tiled_fits(p)) {
    set_error("mi355_linear16_fwd: row strides (%lld, %lld) beyond the kernels' buffer descriptors",
              static_cast<long long>(p.xs), static_cast<long long>(p.ws));
    return MI355_ERR_UNSUPPORTED;
  }
  const W8Params w{p.x, p.w, nullptr, p.bias, p.out, p.rows, p.k, p.n, p.xs, p.ws, p.os, MI355_F32, p.bdt,
                   nullptr, nullptr};
  if (p.rows <= 64) {
    const int bn = (p.rows <= 32 && p.n > 10000) ? 128 : 64;
    if (p.rows <= 16 || (p.n + bn - 1) / bn < 128)
      return w8_stream_launch<T, TO, false, 2>(w, l16_stream_plan(p.rows, p.k, p.n, cus), s);
    return l16_tiled_small<T, TO>(p, s);
  }
  // More rows: the tiled GEMM.  (32-row skinny tiles with split K re-read
  // 16-bit weights per tile: at 96 - 256 rows of the Qwen2.5-1.5B / 7B down
  // and o projections they measured 1.7 - 4.0x slower than the tiled GEMM
  // even on small grids, e.g. 7B down, 256 rows 350.9 vs 87.8 us.)
  return l16_tiled<T, TO>(p, s);
}

}  // namespace

int linear16_launch(const void* x, const void* w, const void* bias, void* out, int rows, int k, int n, int64_t xs,
                    int64_t ws, int64_t os, int dtype, int bias_dtype, int out_dtype, hipStream_t stream) {
  int cus = 0;
  const int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  const L16Params p{x, w, bias, out, rows, k, n, xs, ws, os, bias ? bias_dtype : -1};
  if (dtype == MI355_F16 && out_dtype == MI355_F16) return l16_typed<F16, F16>(p, stream, cus);
  if (dtype == MI355_F16 && out_dtype == MI355_F32) return l16_typed<F16, F32>(p, stream, cus);
  if (dtype == MI355_BF16 && out_dtype == MI355_BF16) return l16_typed<BF16, BF16>(p, stream, cus);
  if (dtype == MI355_BF16 && out_dtype == MI355_F32) return l16_typed<BF16, F32>(p, stream, cus);
  set_error("mi355_linear16_fwd: unsupported dtype pair (in=%d, out=%d)", dtype, out_dtype);
  return MI355_ERR_UNSUPPORTED;
}

}  // namespace mi355
