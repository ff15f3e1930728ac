// Gate/up projection fused with the SiLU-and-mul epilogue, plus its launcher:
//
//   out[m, n] = silu(g) * u,  g = sum_k x[m,k] * w_gate[n,k],  u = sum_k x[m,k] * w_up[n,k]
//
// g and u are fp32 MFMA accumulators that go straight into the activation;
// the result is rounded once to the output type.  This is the "fused
// activation with the up/gate projections" the reference plans
// (docs/architecture-cuda.md:94) for the MLP its FusedMLP runs as two GEMMs,
// a rounding of both to x's type and the SiLU-and-mul kernel
// (src/engine/fused_norm_activation_patch.py:60-64).
//
// At decode shapes (rows <= 32) the work is weight streaming: each weight
// element is read once per call (2 * n_out * k elements) and meets at most 32
// rows of x, so the kernel is bound by HBM bandwidth on the weights, not by
// MFMA.  Up to 32 rows the launcher runs the lane-coalesced weight-streaming
// kernel of w8a16_stream.h with 16-bit weights (from 17 rows where the small
// tiled shapes do not pay); the skinny kernel below serves more rows whose
// row strides (2^22 elements or more) the tiled kernel's buffer descriptors
// cannot span.
// More rows are a GEMM (MFMA-bound): they run the LDS-tiled kernel of
// tiled_gemm.h with both weight matrices as B operands and SiLU-and-mul in
// its epilogue.
//
// Operand layout.  The v_mfma_f32_16x16x32 B operand gives lane l column
// n = l % 16 and k-group l / 16 (8 consecutive k each).  Giving the 16
// columns to 16 weight rows would make each load instruction read 16 rows x
// 64 bytes, and half-line reads like that stream from HBM at about 70% of
// the rate of full 128-byte lines on MI355X.  Instead a B operand holds 8
// weight rows x 64 columns: column n is weight row n % 8 and half h = n / 8
// of a 64-column K block, so the 8 lanes of a row cover 128 contiguous
// bytes.  The A operand stacks the (up to) 8 rows of the x tile twice: A row
// i is x row i % 8 over half i / 8 of the same K block.  Then
//
//   D[i][n] = sum over the block's half of x[i % 8] * w[n % 8]  when i / 8 == n / 8
//
// and the product of x row a with weight row b over the block is
// D[a][b] + D[a + 8][b + 8]; the off-diagonal quarters of D are discarded.
// For up to 8 rows of x this costs no extra MFMA work (A rows 8..15 would
// otherwise be padding).  x loads use the same lane -> (row, column) map.
//
// Decomposition: a workgroup owns 8 * G weight rows (G MFMA B operands per
// matrix) and a tile of 8 * MT rows of x (blockIdx.y), and splits K between
// SPLITK waves (contiguous K ranges, so a workgroup reads whole weight
// rows).  Per 64-column K step a wave loads G B operands of w_gate, G of
// w_up and MT A operands of x, each one 16-byte load per lane, then issues
// 2 * G * MT MFMAs.  The loads of U steps are issued before their
// MFMAs.  Weight rows past n_out and x rows past the tile address past their
// buffer descriptor and read 0.  The SPLITK partial accumulators meet in
// LDS, where the two diagonal quarters are added (in a fixed order, so
// results do not depend on scheduling), then SiLU-and-mul and the store.
// D layout of the gfx950 16x16x32 MFMA: lane l holds rows 4 * (l / 16) + j,
// j < 4, of column l % 16.
#include "common.h"
#include "tiled_gemm.h"
#include "w8a16_stream.h"

// Launch shapes (split-K waves, weight row groups, K steps in flight per
// wave) were chosen by sweeping them on MI355X at Qwen2.5 decode shapes:
//   up to 8 rows of x, k <= 2048 and n_out < 16384: SPLITK 4, G 1 (the most
//     workgroups), U 6 (one load group per wave at k = 1536; U 4 for
//     k <= 1024);
//   otherwise SPLITK 4, G 2 (x read once per 16 weight rows), U 2.

namespace mi355 {
namespace {

struct GateUpParams {
  const void* x;       // [rows, xs]
  const void* wg;      // [n_out, ws]
  const void* wu;      // [n_out, ws]
  void* out;           // [rows, os]
  int rows;
  int k;               // multiple of 8
  int n_out;
  int64_t xs, ws, os;  // row strides in elements (xs, ws multiples of 8)
};

// Operands of N K-steps (64 columns each) of one wave.
template <int G, int MT, int N>
struct StepRegs {
  u32x4 bg[N][G], bu[N][G], a[N][MT];
};

// Issues the loads of N K-steps starting at step s (byte column 128 * s);
// steps at or past s_end address past the descriptors (no memory traffic,
// zeros).  woff / xoff: the lane's row and in-block column, in bytes.
template <int G, int MT, int N>
__device__ __forceinline__ void gu_load(StepRegs<G, MT, N>& r, rsrc_t rg, rsrc_t ru, rsrc_t rx,
                                        const uint32_t (&woff)[G], const uint32_t (&xoff)[MT], int s, int s_end) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const bool live = s + j < s_end;
    const uint32_t c = 128u * static_cast<uint32_t>(s + j);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      r.bg[j][g] = buf_load16(rg, live ? woff[g] + c : kOob);
      r.bu[j][g] = buf_load16(ru, live ? woff[g] + c : kOob);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) r.a[j][t] = buf_load16_cached(rx, live ? xoff[t] + c : kOob);
  }
}

template <typename T, int G, int MT, int N>
__device__ __forceinline__ void gu_mfma(const StepRegs<G, MT, N>& r, f32x4 (&accg)[G][MT], f32x4 (&accu)[G][MT]) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        accg[g][t] = mfma16<T>(r.a[j][t], r.bg[j][g], accg[g][t]);
        accu[g][t] = mfma16<T>(r.a[j][t], r.bu[j][g], accu[g][t]);
      }
    }
  }
}

template <typename T, typename TO, int MT, int SPLITK, int G, int U>
__global__ __launch_bounds__(64 * SPLITK) void gate_up_silu_skinny(const GateUpParams p) {
  using TB = typename T::bits;
  __shared__ float red[SPLITK][G][MT][2][4][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 8 * G;
  const int m0 = blockIdx.y * 8 * MT;
  const int nrows_w = p.n_out - n0 < 8 * G ? p.n_out - n0 : 8 * G;
  const int nrows_x = p.rows - m0 < 8 * MT ? p.rows - m0 : 8 * MT;

  // Descriptors end right after the last valid element, so weight rows past
  // n_out and x rows past the tile (offset >= rows * stride >= the extent,
  // since strides >= k) read as 0.
  const rsrc_t rg = make_rsrc(static_cast<const TB*>(p.wg) + static_cast<int64_t>(n0) * p.ws,
                              static_cast<uint32_t>(((nrows_w - 1) * p.ws + p.k) * sizeof(TB)));
  const rsrc_t ru = make_rsrc(static_cast<const TB*>(p.wu) + static_cast<int64_t>(n0) * p.ws,
                              static_cast<uint32_t>(((nrows_w - 1) * p.ws + p.k) * sizeof(TB)));
  const rsrc_t rx = make_rsrc(static_cast<const TB*>(p.x) + static_cast<int64_t>(m0) * p.xs,
                              static_cast<uint32_t>(((nrows_x - 1) * p.xs + p.k) * sizeof(TB)));

  // Lane -> (row r = l % 8 of the operand, half h = (l / 8) % 2, k-group kg = l / 16):
  // 16-byte piece at column 32 * h + 8 * kg of each 64-column block.
  const int r8 = lane & 7;
  const int colb = (((lane >> 3) & 1) * 32 + (lane >> 4) * 8) * static_cast<int>(sizeof(TB));
  uint32_t woff[G], xoff[MT];
#pragma unroll
  for (int g = 0; g < G; ++g) woff[g] = static_cast<uint32_t>((8 * g + r8) * p.ws * sizeof(TB) + colb);
#pragma unroll
  for (int t = 0; t < MT; ++t) xoff[t] = static_cast<uint32_t>((8 * t + r8) * p.xs * sizeof(TB) + colb);

  f32x4 accg[G][MT], accu[G][MT];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      accg[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      accu[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  const int kfull = p.k >> 6;  // whole 64-column steps
  const int s_end = (kfull * (wave + 1)) / SPLITK;
  // Every load of a group is issued before its MFMAs (sched_barrier keeps the
  // scheduler from interleaving them), so a wave keeps U steps in flight.
  for (int s = (kfull * wave) / SPLITK; s < s_end; s += U) {
    StepRegs<G, MT, U> cur;
    gu_load<G, MT, U>(cur, rg, ru, rx, woff, xoff, s, s_end);
    __builtin_amdgcn_sched_barrier(0);
    gu_mfma<T, G, MT, U>(cur, accg, accu);
  }
  if ((p.k & 63) != 0 && wave == SPLITK - 1) {
    // Partial last block: 16-byte pieces at or past k read 0.
    const bool live = kfull * 64 + (((lane >> 3) & 1) * 32 + (lane >> 4) * 8) < p.k;
    const uint32_t c = 128u * static_cast<uint32_t>(kfull);
    StepRegs<G, MT, 1> tail;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      tail.bg[0][g] = buf_load16(rg, live ? woff[g] + c : kOob);
      tail.bu[0][g] = buf_load16(ru, live ? woff[g] + c : kOob);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) tail.a[0][t] = buf_load16_cached(rx, live ? xoff[t] + c : kOob);
    gu_mfma<T, G, MT, 1>(tail, accg, accu);
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        red[wave][g][t][0][j][lane] = accg[g][t][j];
        red[wave][g][t][1][j][lane] = accu[g][t][j];
      }
    }
  }
  __syncthreads();

  // Output (x row 8t + a, weight row 8g + b) = D[a][b] + D[a + 8][b + 8]:
  // register a % 4 of lanes 16 * (a / 4) + b and 16 * (a / 4) + 40 + b.
  for (int o = threadIdx.x; o < 64 * G * MT; o += 64 * SPLITK) {
    const int b = o & 7, a = (o >> 3) & 7, gt = o >> 6;
    const int g = gt % G, t = gt / G;
    const int m = 8 * t + a, n = 8 * g + b;
    if (m >= nrows_x || n >= nrows_w) continue;
    const int l0 = 16 * (a >> 2) + b, j = a & 3;
    float gs = 0.f, us = 0.f;
#pragma unroll
    for (int w = 0; w < SPLITK; ++w) {
      gs += red[w][g][t][0][j][l0] + red[w][g][t][0][j][l0 + 40];
      us += red[w][g][t][1][j][l0] + red[w][g][t][1][j][l0 + 40];
    }
    store_elem<TO>(p.out, static_cast<int64_t>(m0 + m) * p.os + n0 + n, silu_mul_f32(gs, us));
  }
}

template <typename T, typename TO, int MT, int SPLITK, int G, int U>
int gate_up_launch_tiles(const GateUpParams& p, hipStream_t s) {
  void* args[] = {const_cast<GateUpParams*>(&p)};
  const dim3 grid(static_cast<unsigned>((p.n_out + 8 * G - 1) / (8 * G)),
                  static_cast<unsigned>((p.rows + 8 * MT - 1) / (8 * MT)));
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(gate_up_silu_skinny<T, TO, MT, SPLITK, G, U>),
                                    grid, dim3(64 * SPLITK), args, 0, s),
                    "gate_up_silu launch");
}

template <typename T, typename TO, int MT>
int gate_up_shape(const GateUpParams& p, hipStream_t s) {
  if (MT == 1 && p.k <= 2048 && p.n_out < 16384) {
    if (p.k <= 1024) return gate_up_launch_tiles<T, TO, 1, 4, 1, 4>(p, s);
    return gate_up_launch_tiles<T, TO, 1, 4, 1, 6>(p, s);
  }
  return gate_up_launch_tiles<T, TO, MT, 4, 2, 2>(p, s);
}

// m-blocks per group of the tiled GEMM's tile order inside each XCD's range
// (m fastest within a group).
constexpr int kGuGroupM = 4;

template <typename T, typename TO, int WGM, int WGN, int FM, int FN, int S, int RING = 0, int XR = 0>
int gate_up_tiled_cfg(const GateUpParams& p, hipStream_t s) {
  using C = tiled::Cfg<T, tiled::B_16, TO, WGM, WGN, FM, FN, tiled::EPI_SILU, S>;
  static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
  // a tile count that is not a multiple of 8: the instantiation with
  // contiguous tile ranges per XCD for any count (XR = 1; 1.5B at 384 rows
  // 34.7 -> 29.7 us, at 1400 rows 92.5 -> 87.3 us, 7B at 1792 rows 435.8 ->
  // 412.3 us)
  if constexpr (XR == 0) {
    const int64_t ntiles = static_cast<int64_t>((p.rows + C::BM - 1) / C::BM) * ((p.n_out + C::BN - 1) / C::BN);
    if (ntiles % 8 != 0) return gate_up_tiled_cfg<T, TO, WGM, WGN, FM, FN, S, RING, 1>(p, s);
  }
  tiled::Params tp{};
  tp.x = p.x;
  tp.b0 = p.wg;
  tp.b1 = p.wu;
  tp.out = p.out;
  tp.rows = p.rows;
  tp.k = p.k;
  tp.n = p.n_out;
  tp.xs = p.xs;
  tp.bs = p.ws;
  tp.os = p.os;
  tp.sdt = MI355_F32;
  tp.bdt = -1;
  tp.tiles_m = (p.rows + C::BM - 1) / C::BM;
  tp.tiles_n = (p.n_out + C::BN - 1) / C::BN;
  tp.group_m = tp.tiles_m < kGuGroupM ? tp.tiles_m : kGuGroupM;
  void* args[] = {&tp};
  // all LDS is static (no dynamic shared memory)
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(tiled::tiled_gemm<T, tiled::B_16, TO, WGM, WGN, FM, FN,
                                                                                      tiled::EPI_SILU, S, RING, 0, XR>),
                                    dim3(static_cast<unsigned>(tp.tiles_m * tp.tiles_n)), dim3(C::BLOCK), args, 0, s),
                    "gate_up_silu tiled launch");
}

// Tiled launch shapes from sweeps on MI355X (Qwen2.5-1.5B and 7B MLPs at
// 16 - 64, 128 and 384 - 4096 rows): up to 32 rows 32 x 64 output tiles (2
// waves) or, for n_out > 10000, 32 x 128 (4 waves); up to 64 rows 64 x 64 (4
// waves; n_out > 10000 keeps the next shape); up to 128 rows 128 x 64 (4
// waves, 4 stages) or, for n_out > 10000, 128 x 128 (8 waves, 3 stages); more
// rows by the round count below (1.5B, 256 rows 37.9 -> 27.8 us, 384 rows
// 48.1 -> 35.0 us, 768 rows 58.1 -> 48.7 us, 4096 rows 251 -> 233 us; 7B, 256
// rows 118 -> 97 us, 2048 rows 518 -> 469 us).
// The small shapes run 4 stages.  Descriptors span at most 256 rows of x and
// 128 weight rows, each below 2^31 bytes.
template <typename T, typename TO>
int gate_up_tiled(const GateUpParams& p, hipStream_t s) {
  const bool wide = p.n_out > 10000;
  if (p.rows <= 32) {
    if (wide) return gate_up_tiled_cfg<T, TO, 1, 4, 1, 1, 4>(p, s);  // 32 x 128, 4 waves
    return gate_up_tiled_cfg<T, TO, 1, 2, 1, 1, 4>(p, s);            // 32 x 64, 2 waves
  }
  if (p.rows <= 64 && !wide) return gate_up_tiled_cfg<T, TO, 2, 2, 1, 1, 4>(p, s);  // 64 x 64, 4 waves
  if (p.rows <= 128) {
    if (p.n_out <= 10000) return gate_up_tiled_cfg<T, TO, 2, 2, 2, 1, 4>(p, s);
    return gate_up_tiled_cfg<T, TO, 2, 4, 2, 1, 3>(p, s);
  }
  // More rows: the plan with the fewest weighted rounds of workgroups over
  // the CUs, in units of one round of 256 x 64 tiles (8 waves, 3 stages).
  // One shape for the whole output: 256 x 64; 128 x 64 (4 waves, the
  // sub-step ring at 2 stages: 64 KiB of LDS, two workgroups per CU, each
  // with its own barriers), 1.05 a round; 256 x 128 (8 waves of 128 x 32,
  // the sub-step ring at 2 stages), which moves two thirds of 256 x 64's
  // operand bytes per MFMA through the DMA and three quarters through LDS
  // reads, 1.72 a round for twice the work.  Or a column split: whole rounds
  // of 256 x 128 tiles over the leading columns, then the remaining columns
  // in one round of the smallest tile that covers them in one -- 64 x 64 (4
  // waves, 0.8), 128 x 64 (4 waves, 4 stages, 1.0), 128 x 64 on the ring
  // (two per CU, 1.05) or 256 x 64 (1.0) -- so a last, thinly filled round
  // of large tiles becomes a full round of small ones (1.5B, 1024 rows
  // 80.5 -> 64.6 us).  The whole rounds are counted in tiles, not in
  // 128-column blocks per round: with 6 row blocks, 3 rounds on 256 CUs hold
  // 128 column blocks, where 3 x 42 blocks of whole columns per round left 4
  // CUs idle each round and the rest too wide for one round of small tiles
  // (7B, 1536 rows: 368 -> 355 us).  The split is two launches of one kernel on column
  // ranges: every output element sums its k products in the same order
  // either way.  Weights are the measured per-round times at Qwen2.5-1.5B
  // and 7B shapes; ties keep the single launch, then 256 x 64.
  int cus = 0;
  const int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  const auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  const auto rounds = [&](int rows, int cols, int bm, int bn, int per_cu) {
    return static_cast<double>(cdiv(cdiv(rows, bm) * cdiv(cols, bn), static_cast<int64_t>(cus) * per_cu));
  };
  const double c64 = rounds(p.rows, p.n_out, 256, 64, 1), c_small = 1.05 * rounds(p.rows, p.n_out, 128, 64, 2),
               c128 = 1.72 * rounds(p.rows, p.n_out, 256, 128, 1);
  const double single = c64 < c_small ? (c64 < c128 ? c64 : c128) : (c_small < c128 ? c_small : c128);

  // 256 x 128 tiles (a ragged tile count gets XCD ranges, as every launch
  // does: 1.5B at 768 rows, 210 tiles, 49.0 -> 46.3 us; at 1536 rows, 420
  // tiles, 93.6 -> 90.5 us)
  const auto big_tiles = [&](const GateUpParams& q) { return gate_up_tiled_cfg<T, TO, 2, 4, 4, 1, 2, 1>(q, s); };
  // whole rounds of 256 x 128 tiles, and the 128-column blocks that fill
  // them (a round need not end at a column boundary: the head launch's
  // tiles fill its rounds in order)
  const int64_t tiles_m = cdiv(p.rows, 256);
  const int64_t full = cdiv(p.n_out, 128) * tiles_m / cus;
  const int lead = static_cast<int>(full * cus / tiles_m * 128);  // columns in whole rounds
  if (full >= 1 && lead > 0 && lead < p.n_out) {
    const int rest = p.n_out - lead;
    const auto one_round = [&](int bm, int bn, int per_cu) { return rounds(p.rows, rest, bm, bn, per_cu) <= 1.0; };
    int shape = 0;
    double rest_cost = 0.0;
    if (one_round(64, 64, 1)) shape = 1, rest_cost = 0.8;
    else if (one_round(128, 64, 1)) shape = 2, rest_cost = 1.0;
    else if (one_round(128, 64, 2)) shape = 3, rest_cost = 1.05;
    else if (one_round(256, 64, 1)) shape = 4, rest_cost = 1.0;
    if (shape != 0 && 1.72 * static_cast<double>(full) + rest_cost < single) {
      GateUpParams head = p, tail = p;
      head.n_out = lead;
      tail.n_out = rest;
      const int64_t wskip = static_cast<int64_t>(lead) * p.ws * static_cast<int64_t>(sizeof(typename T::bits));
      tail.wg = static_cast<const uint8_t*>(p.wg) + wskip;
      tail.wu = static_cast<const uint8_t*>(p.wu) + wskip;
      tail.out = static_cast<uint8_t*>(p.out) + static_cast<int64_t>(lead) * static_cast<int64_t>(sizeof(typename TO::bits));
      const int r = big_tiles(head);
      if (r != MI355_OK) return r;
      if (shape == 1) return gate_up_tiled_cfg<T, TO, 2, 2, 1, 1, 4>(tail, s);
      if (shape == 2) return gate_up_tiled_cfg<T, TO, 2, 2, 2, 1, 4>(tail, s);
      if (shape == 3) return gate_up_tiled_cfg<T, TO, 2, 2, 2, 1, 2, 1>(tail, s);
      return gate_up_tiled_cfg<T, TO, 4, 2, 2, 1, 3>(tail, s);
    }
  }
  if (c64 == single) return gate_up_tiled_cfg<T, TO, 4, 2, 2, 1, 3>(p, s);
  if (c_small == single) return gate_up_tiled_cfg<T, TO, 2, 2, 2, 1, 2, 1>(p, s);
  return big_tiles(p);
}

template <typename T, typename TO>
int gate_up_typed(const GateUpParams& p, hipStream_t s) {
  // Up to 16 rows: the lane-coalesced weight-streaming kernel of
  // w8a16_stream.h with 16-bit weights (its x descriptor must span under
  // 2^32 bytes; else the skinny kernel above with the fewest 8-row MFMA
  // tiles that cover the rows).  More rows take the tiled GEMM when its
  // descriptors fit -- from 17 rows its small tiles read each weight byte
  // once from HBM and x once per workgroup, where 3 or 4 skinny x tiles
  // re-load x per weight piece (1.5B, 32 rows 20.0 -> 15.5 us; 7B 66.7 ->
  // 53.8 us), as long as the output has >= 128 tile columns to spread over
  // the CUs -- else the stream kernel again with 6 or 8 x sets (0.5B, 32
  // rows 10.5 -> 9.0 us against 32-row skinny tiles), or 24- or 32-row
  // skinny tiles along grid y where its descriptors cannot span the inputs.
  const int64_t tb = sizeof(typename T::bits);
  const bool stream_fits = p.rows <= 32 && ((p.rows - 1) * p.xs + p.k) * tb < (int64_t{1} << 32) &&
                           (15 * p.ws + p.k) * tb < (int64_t{1} << 32);
  const W8Params w{p.x, p.wg, nullptr, nullptr, p.out, p.rows, p.k, p.n_out, p.xs, p.ws, p.os, MI355_F32, -1,
                   p.wu, nullptr};
  auto stream = [&]() {
    int cus = 0;
    const int st = compute_units(&cus);
    if (st != MI355_OK) return st;
    return w8_stream_launch<T, TO, true, 2>(w, gu16_stream_plan(p.rows, p.k, p.n_out, cus), s);
  };
  if (p.rows <= 16) {
    if (stream_fits) return stream();
    return p.rows <= 8 ? gate_up_shape<T, TO, 1>(p, s) : gate_up_shape<T, TO, 2>(p, s);
  }
  const bool tiled_fits = int64_t{256} * p.xs * tb < (int64_t{1} << 31) && int64_t{128} * p.ws * tb < (int64_t{1} << 31);
  const int bn = p.n_out > 10000 ? 128 : 64;
  if (tiled_fits && (p.rows > 32 || (p.n_out + bn - 1) / bn >= 128)) return gate_up_tiled<T, TO>(p, s);
  if (stream_fits) return stream();
  if (p.rows <= 24) return gate_up_shape<T, TO, 3>(p, s);
  return gate_up_shape<T, TO, 4>(p, s);
}

}  // namespace

int gate_up_silu_launch(const void* x, const void* wg, const void* wu, void* out, int rows, int k, int n_out,
                        int64_t xs, int64_t ws, int64_t os, int dtype, int out_dtype, hipStream_t stream) {
  const GateUpParams p{x, wg, wu, out, rows, k, n_out, xs, ws, os};
  if (dtype == MI355_F16 && out_dtype == MI355_F16) return gate_up_typed<F16, F16>(p, stream);
  if (dtype == MI355_F16 && out_dtype == MI355_F32) return gate_up_typed<F16, F32>(p, stream);
  if (dtype == MI355_BF16 && out_dtype == MI355_BF16) return gate_up_typed<BF16, BF16>(p, stream);
  if (dtype == MI355_BF16 && out_dtype == MI355_F32) return gate_up_typed<BF16, F32>(p, stream);
  set_error("mi355_gate_up_silu_fwd: unsupported dtype pair (in=%d, out=%d)", dtype, out_dtype);
  return MI355_ERR_UNSUPPORTED;
}

}  // namespace mi355
