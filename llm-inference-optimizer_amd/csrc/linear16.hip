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
// Four kernels, picked by the launcher:
//   w8a16_stream      rows <= 16 (decode; w8a16_stream.h with one 16-bit
//                     matrix), and 17 - 64 where the small tiled shapes do not
//                     pay: lane-coalesced weight streaming, every weight byte
//                     read once per call, MFMA (v_mfma_f32_16x16x32_*).
//   linear16_skinny   inputs the stream kernel's descriptors cannot span, and
//                     larger ones whose tiled descriptors would pass 2^31
//                     bytes: every weight byte is read once per call with
//                     non-temporal loads and meets up to 32 rows of x on
//                     MFMA (the same instruction).
//   tiled_gemm        more rows: the LDS-tiled MFMA GEMM of tiled_gemm.h with
//                     the weights as a 16-bit B operand and the bias in its
//                     epilogue (EPI_LINEAR).
//   linear16_generic  any k, stride or alignment the two above cannot take:
//                     one wave per (output feature, 4 rows of x), fp32 fma.
//
// Skinny operand layout (the gate/up kernel's): the 16x16x32 MFMA B operand
// gives lane l column n = l % 16 and k-group l / 16 (8 consecutive k).  A B
// operand holds 8 weight rows x 64 columns: column n is weight row n % 8 over
// half h = n / 8 of a 64-column block, so lane l loads 16 bytes of weight row
// l % 8 at column 32 h + 8 (l / 16) and the 8 lanes of a row cover one
// 128-byte line.  The A operand stacks the (up to) 8 rows of an x tile twice
// with the same lane -> column map, so the product of x row a with weight
// row b over the block is D[a][b] + D[a + 8][b + 8].  D layout of the gfx950
// 16x16x32 MFMA: lane l holds rows 4 (l / 16) + j, j < 4, of column l % 16.
//
// Decomposition: a workgroup owns 8 G weight rows (blockIdx.y) and a tile of
// 8 MT rows of x (blockIdx.x) and splits the 64-column blocks of K between its
// waves (contiguous ranges); each wave keeps U blocks of loads in flight, and
// every x operand it loads feeds G weight groups.  Pieces past k address past
// the buffer descriptors (zeros, no traffic).  The per-wave partial sums meet
// in LDS in a fixed order, so a call's bits do not depend on scheduling.
#include "common.h"
#include "tiled_gemm.h"
#include "w8a16_stream.h"

namespace mi355 {
namespace {

constexpr int kMaxSplit = 16;  // waves per skinny workgroup

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

// ------------------------------------------------------------------ skinny

template <typename T, typename TO, int MT, int G, int U>
__global__ __launch_bounds__(64 * kMaxSplit) void linear16_skinny(const L16Params p) {
  using TB = typename T::bits;
  extern __shared__ float red[];  // [nwave][G][MT][4][64]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwave = blockDim.x >> 6;
  // x tiles vary fastest, so the workgroups sharing a weight group run
  // together and its re-reads (rows > 8 MT) hit L2.
  const int m0 = blockIdx.x * 8 * MT;
  const int n0 = blockIdx.y * 8 * G;
  const int nrows_w = p.n - n0 < 8 * G ? p.n - n0 : 8 * G;
  const int nrows_x = p.rows - m0 < 8 * MT ? p.rows - m0 : 8 * MT;

  // Descriptors end right after the last valid element, so weight rows past n
  // and x rows past the tile (offset >= rows * stride >= the extent) read 0.
  const rsrc_t rw = make_rsrc(static_cast<const TB*>(p.w) + static_cast<int64_t>(n0) * p.ws,
                              static_cast<uint32_t>(((nrows_w - 1) * p.ws + p.k) * sizeof(TB)));
  const rsrc_t rx = make_rsrc(static_cast<const TB*>(p.x) + static_cast<int64_t>(m0) * p.xs,
                              static_cast<uint32_t>(((nrows_x - 1) * p.xs + p.k) * sizeof(TB)));

  // Lane -> (row l % 8 of the operand, column 32 ((l / 8) % 2) + 8 (l / 16) of the block).
  const int r8 = lane & 7;
  const int col = ((lane >> 3) & 1) * 32 + (lane >> 4) * 8;
  uint32_t woff[G], xoff[MT];
#pragma unroll
  for (int g = 0; g < G; ++g) woff[g] = static_cast<uint32_t>(((8 * g + r8) * p.ws + col) * sizeof(TB));
#pragma unroll
  for (int t = 0; t < MT; ++t) xoff[t] = static_cast<uint32_t>(((8 * t + r8) * p.xs + col) * sizeof(TB));

  f32x4 acc[G][MT];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int nblk = (p.k + 63) >> 6;
  const int s_end = (nblk * (wave + 1)) / nwave;
  for (int s = (nblk * wave) / nwave; s < s_end; s += U) {
    u32x4 wv[U][G], xv[U][MT];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      // k is a multiple of 8, so a lane's 8-element piece is wholly inside or outside
      const bool live = s + j < s_end && 64 * (s + j) + col < p.k;
      const uint32_t c = 128u * static_cast<uint32_t>(s + j);
#pragma unroll
      for (int g = 0; g < G; ++g) wv[j][g] = buf_load16(rw, live ? woff[g] + c : kOob);
#pragma unroll
      for (int t = 0; t < MT; ++t) xv[j][t] = buf_load16_cached(rx, live ? xoff[t] + c : kOob);
    }
    // every load of the group ahead of its MFMAs: U blocks in flight per wave
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[g][t] = mfma16<T>(xv[j][t], wv[j][g], acc[g][t]);
      }
    }
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) red[(((wave * G + g) * MT + t) * 4 + j) * 64 + lane] = acc[g][t][j];
    }
  }
  __syncthreads();

  // Output (x row 8t + a, weight row 8g + b) = D[a][b] + D[a + 8][b + 8]:
  // register a % 4 of lanes 16 (a / 4) + b and 16 (a / 4) + 40 + b.
  for (int o = threadIdx.x; o < 64 * G * MT; o += blockDim.x) {
    const int b = o & 7, a = (o >> 3) & 7, gt = o >> 6;
    const int g = gt % G, t = gt / G;
    const int m = 8 * t + a, n = 8 * g + b;
    if (m >= nrows_x || n >= nrows_w) continue;
    const int l0 = 16 * (a >> 2) + b, j = a & 3;
    float sum = 0.f;
    for (int w = 0; w < nwave; ++w) {
      const float* r = red + (((w * G + g) * MT + t) * 4 + j) * 64;
      sum += r[l0] + r[l0 + 40];
    }
    l16_store<TO>(p, m0 + m, n0 + n, sum);
  }
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

// Skinny launch shape, fitted to a sweep of G x U x waves per workgroup on
// MI355X over the down, o and q projections of Qwen2.5-0.5B, 1.5B and 7B at
// 1, 8 and 32 rows (every pick within 1.06x of the best sampled shape):
//   G (weight-row groups per workgroup; each x operand feeds G B operands)
//     2 when that still leaves about 3/4 of a workgroup per CU (n / 16 >=
//     0.75 CUs: the 7B projections), else 1;
//   U (64-column blocks in flight per wave) 2 for one 8-row x tile, else 1
//     (more x operands per block);
//   waves per workgroup (the split of K) 16 / G for a single row (32 KiB of
//     weights in flight per workgroup), else 8; capped by the LDS for the
//     partial sums (<= 64 KiB) and the number of blocks, then evened out so
//     every wave gets the same number of blocks -- or, with no more
//     workgroups than CUs, rounded to a multiple of 4 so the CU's 4 SIMDs
//     carry equal loads.
template <typename T, typename TO, int MT, int G>
int l16_skinny_g(const L16Params& p, hipStream_t s, int cus) {
  const int groups = (p.n + 8 * G - 1) / (8 * G);
  const int nblk = (p.k + 63) / 64;
  const int tiles = (p.rows + 8 * MT - 1) / (8 * MT);
  const int64_t units = static_cast<int64_t>(groups) * tiles;
  int split = p.rows <= 1 ? 16 / G : 8;
  int u = MT == 1 ? 2 : 1;
  if (split > kMaxSplit) split = kMaxSplit;
  if (split > 64 / (G * MT)) split = 64 / (G * MT);  // partial sums: split * G * MT KiB <= 64 KiB
  if (split > nblk) split = nblk;
  if (split < 1) split = 1;
  int bpw = (nblk + split - 1) / split;
  if (units <= cus && split > 4) {
    split = ((split + 2) / 4) * 4;
    if (split > 64 / (G * MT)) split = (64 / (G * MT)) / 4 * 4;
    if (split > kMaxSplit) split = kMaxSplit;
    bpw = (nblk + split - 1) / split;
  } else {
    split = (nblk + bpw - 1) / bpw;  // even blocks per wave
  }
  if (u > bpw) u = bpw >= 2 ? 2 : 1;
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(groups));
  const dim3 block(64 * split);
  const size_t lds = static_cast<size_t>(split) * G * MT * 4 * 64 * sizeof(float);
  // register budget (128 VGPRs at 1024 threads): U (4 G + 4 MT) operand
  // dwords + 4 G MT accumulators <= 100
  constexpr int umax = (100 - 4 * G * MT) / (4 * G + 4 * MT);
  if (u >= 2 && umax >= 2) return launch_l16(linear16_skinny<T, TO, MT, G, (umax >= 2 ? 2 : 1)>, grid, block, lds, p, s);
  return launch_l16(linear16_skinny<T, TO, MT, G, 1>, grid, block, lds, p, s);
}

template <typename T, typename TO, int MT>
int l16_skinny_shape(const L16Params& p, hipStream_t s, int cus) {
  const int g = (p.n + 15) / 16 >= (3 * cus) / 4 ? 2 : 1;
  if (g >= 2) return l16_skinny_g<T, TO, MT, 2>(p, s, cus);
  return l16_skinny_g<T, TO, MT, 1>(p, s, cus);
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
  // Up to 16 rows, and 17 - 64 where the small tiled shapes below do not
  // pay: the weight-streaming kernel of w8a16_stream.h with one 16-bit
  // matrix, whose x descriptor spans all rows of x and each workgroup's
  // weight descriptor up to 16 weight rows (both under 2^32 bytes); else the
  // skinny kernel (1.5B down, 32 rows 22.1 -> 14.4 us on the stream kernel,
  // 64 rows 43.7 -> 22.2 against the small tiles; 7B down 51.9 -> 37.3 at
  // 32 rows, 90.3 -> 83.1 at 64; 0.5B down 13.2 -> 7.9 at 32 rows).
  const int64_t tb = sizeof(typename T::bits);
  const bool stream_fits = p.rows <= 64 && ((p.rows - 1) * p.xs + p.k) * tb < (int64_t{1} << 32) &&
                           (15 * p.ws + p.k) * tb < (int64_t{1} << 32);
  const W8Params w{p.x, p.w, nullptr, p.bias, p.out, p.rows, p.k, p.n, p.xs, p.ws, p.os, MI355_F32, p.bdt,
                   nullptr, nullptr};
  if (p.rows <= 16 && stream_fits)
    return w8_stream_launch<T, TO, false, 2>(w, l16_stream_plan(p.rows, p.k, p.n, cus), s);
  if (p.rows <= 8) return l16_skinny_shape<T, TO, 1>(p, s, cus);
  if (p.rows <= 16) return l16_skinny_shape<T, TO, 2>(p, s, cus);
  if (p.rows <= 64 && l16_tiled_fits(p)) {
    const int bn = (p.rows <= 32 && p.n > 10000) ? 128 : 64;
    if ((p.n + bn - 1) / bn >= 128 || (p.rows > 32 && !stream_fits)) return l16_tiled_small<T, TO>(p, s);
  }
  if (stream_fits) return w8_stream_launch<T, TO, false, 2>(w, l16_stream_plan(p.rows, p.k, p.n, cus), s);
  if (p.rows <= 24) return l16_skinny_shape<T, TO, 3>(p, s, cus);
  if (p.rows <= 32) return l16_skinny_shape<T, TO, 4>(p, s, cus);
  // More rows: the tiled GEMM wherever its descriptors fit.  (32-row skinny
  // tiles with split K re-read 16-bit weights per tile: at 96 - 256 rows of
  // the Qwen2.5-1.5B / 7B down and o projections 1.7 - 4.0x slower than the
  // tiled GEMM even on small grids, e.g. 7B down, 256 rows 350.9 vs 87.8 us.)
  if (!l16_tiled_fits(p)) return l16_skinny_shape<T, TO, 4>(p, s, cus);
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
