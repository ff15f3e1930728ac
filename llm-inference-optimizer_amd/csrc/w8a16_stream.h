// The W8A16 decode kernel (up to 64 rows of x): int8 weight streaming with
// lane-coalesced loads, plus its launch plans.  Shared by the W8A16 linear and
// the int8 gate/up + SiLU-and-mul launchers (w8a16.hip) and, with 16-bit
// weights (template argument WB = 2, below), by the 16-bit gate/up +
// SiLU-and-mul launcher (gate_up_silu.hip) and the 16-bit linear
// (linear16.hip).
//
//   out[m, n] = round(acc * scale[n] + bias[n]),  acc = sum_k x[m, k] * q[n, k]
//   (DUAL: out[m, n] = round(silu(acc_g * scale_g[n]) * (acc_u * scale_u[n])))
//   (16-bit weights: no scales; out = round(acc + bias[n]), or the SiLU-and-mul
//   of the two sums when DUAL)
//
// Load layout.  The weights are read 4 rows x 256 bytes per load instruction:
// lane l reads 16 bytes of weight row 4 r + (l % 16) / 4 (4-row set r of the
// workgroup) at byte 16 (l % 4) + 64 (l / 16) of a 256-byte chunk of K, so
// every quad of lanes reads 64 contiguous bytes and each row's 256 bytes come
// from 16 lanes.  (The 8 rows x 128 bytes of w8a16_skinny's layout, with
// consecutive lanes on different rows, streams the same bytes about 10%
// slower on MI355X, and its x loads cost twice as much; see the weight-stream
// probe in csrc/probe/w8_stream.hip.)
//
// MFMA mapping (v_mfma_f32_16x16x32_{f16,bf16}: A lane l holds A[l % 16][8 (l
// / 16) + e], B lane l holds B[8 (l / 16) + e][l % 16], e < 8; D lane l holds
// D[4 (l / 16) + j][l % 16], j < 4).  A lane's 16 int8 weights are widened
// into two B operands (bytes 0-7, 8-15), so B column c = l % 16 is weight row
// 4 r + c / 4 over the k-subset
//   S(c % 4) = {16 (c % 4) + 64 g + e : g < 4, e < 8}   (+ 8 for the second),
// and A row i = 4 m' + q is x row m' of a 4-row x set over S(q): lane l loads
// x[(l % 16) / 4][16 (l % 4) + 64 (l / 16) .. + 16] (two 16-byte loads).
// Then D[4 m' + q][4 r' + q] = sum over S(q) of x[m'] * w[r'], the products
// with i % 4 != c % 4 are discarded, and
//   acc(x row m', weight row r') = sum_q D[4 m' + q][4 r' + q],
// which lane 16 m' + 4 r' + q holds in its register q: each lane keeps its own
// register l % 4 and a quad sum (two DPP adds, one fixed order) finishes it.
// An x tile of up to 64 rows takes MT4 = stream_x_sets(rows) A sets
// (ceil(rows / 4) up to 16 rows, then 6, 8, 12 or 16), so the MFMA work is
// up to four times the minimum -- far below what the weight stream leaves
// idle.
//
// Decomposition.  A workgroup owns rpw <= 4 R4 consecutive weight rows and all
// rows of x; its waves split the 256-byte chunks of K into contiguous ranges
// and keep U chunks of loads in flight (issued together, then consumed).  The
// per-wave sums meet in LDS and are added in wave order, so a call's bits do
// not depend on scheduling.  Weight rows past the workgroup's share and x rows
// past `rows` lie past their buffer descriptors (zeros, no traffic); pieces
// past k are redirected past the descriptors, so any k that is a multiple of
// 16 needs no remainder loop.
#pragma once

#include "common.h"

namespace mi355 {

struct W8Params {
  const void* x;       // [rows, xs] of T
  const void* q;       // [n, qs] int8 (gate weights for the dual kernels)
  const void* scale;   // [n] of sdt
  const void* bias;    // [n] of bdt, or null
  void* out;           // [rows, os] of TO
  int rows, k, n;
  int64_t xs, qs, os;  // row strides in elements
  int sdt, bdt;        // dtype codes of scale and bias (bdt < 0: no bias)
  const void* q2;      // dual kernels: [n, qs] int8 up weights
  const void* scale2;  // dual kernels: [n] of sdt
};

// The epilogue shared by all kernels: scale once, then the bias, one rounding.
template <typename TO>
__device__ __forceinline__ void w8_store(const W8Params& p, int64_t m, int n, float acc) {
  const float sc = load_dyn(p.scale, n, p.sdt);
  const float v = p.bdt >= 0 ? __builtin_fmaf(acc, sc, load_dyn(p.bias, n, p.bdt)) : acc * sc;
  store_elem<TO>(p.out, m * p.os + n, v);
}

// The dual (gate/up) epilogue: both projections scaled once, SiLU-and-mul in
// fp32, one rounding.
template <typename TO>
__device__ __forceinline__ void w8_store_silu(const W8Params& p, int64_t m, int n, float acc_g, float acc_u) {
  const float g = acc_g * load_dyn(p.scale, n, p.sdt);
  const float u = acc_u * load_dyn(p.scale2, n, p.sdt);
  store_elem<TO>(p.out, m * p.os + n, silu_mul_f32(g, u));
}

// 16 int8 weights (one 16-byte load) -> the B operands of two MFMAs.
template <typename T>
__device__ __forceinline__ void widen_i8x16(u32x4 w, u32x4& b0, u32x4& b1) {
  const u32x2 p0 = widen_i8x4<T>(w.x), p1 = widen_i8x4<T>(w.y);
  const u32x2 p2 = widen_i8x4<T>(w.z), p3 = widen_i8x4<T>(w.w);
  b0 = u32x4{p0.x, p0.y, p1.x, p1.y};
  b1 = u32x4{p2.x, p2.y, p3.x, p3.y};
}

// Launch shape of w8a16_stream.
struct StreamPlan {
  int rpw;    // weight rows per workgroup (<= 4 R4)
  int r4;     // 4-row weight sets per workgroup (R4: 1, 2 or 4)
  int waves;  // waves per workgroup (the split of K)
  int u;      // 256-byte chunks in flight per wave (1 or 2)
};

// WB: bytes per weight element -- 1 (int8 weights with per-row scales, the
// W8A16 linear and the int8 gate/up + SiLU-and-mul) or 2 (weights of x's
// 16-bit type, no scales: the 16-bit gate/up + SiLU-and-mul when DUAL, else
// the 16-bit linear, out = acc + bias).  A lane's 16-byte weight load is then
// 8 k, one B operand as loaded, a chunk of a weight row's 256 bytes is 128 k,
// and one 16-byte x load per 4-row x set matches it.
//
// Registers w8a16_stream<R4, MT4, U, DUAL, WB> keeps live per lane, as an
// estimate: 4 per 16x16 accumulator tile (NQ * R4 * MT4 of them), per chunk
// in flight 4 per weight set and 8 -- 4 with 16-bit weights -- per x set,
// and one load offset per weight set and per x set.
constexpr int stream_regs(int r4, int mt4, int u, bool dual, int wb) {
  const int nq = dual ? 2 : 1;
  return 4 * nq * r4 * mt4 + u * (4 * nq * r4 + (wb == 1 ? 8 : 4) * mt4) + r4 + mt4;
}

// Most threads per workgroup of that instantiation: 1024 (16 waves, 128
// VGPRs per lane) below 112 estimated registers, else 512 (8 waves, 256
// VGPRs), and 0 -- no such kernel -- above 224: the shapes at or above 112
// spilled 8 - 432 B per lane under the 128-register budget, those above 224
// spilled under 256 (hipcc -Rpass-analysis=kernel-resource-usage).
constexpr int stream_max_threads(int r4, int mt4, int u, bool dual, int wb) {
  const int e = stream_regs(r4, mt4, u, dual, wb);
  return e > 224 ? 0 : (e >= 112 ? 512 : 1024);
}

// 4-row x sets (MT4) for `rows` of x: ceil(rows / 4) up to 16 rows, then 6
// (17 - 24 rows), 8 (25 - 32), 12 (33 - 48) or 16 (49 - 64); x rows past
// `rows` read zeros.
constexpr int stream_x_sets(int rows) {
  return rows <= 16 ? (rows + 3) / 4 : (rows <= 24 ? 6 : (rows <= 32 ? 8 : (rows <= 48 ? 12 : 16)));
}

template <typename T, typename TO, int R4, int MT4, int U, bool DUAL, int WB = 1>
__global__ __launch_bounds__(stream_max_threads(R4, MT4, U, DUAL, WB)) void w8a16_stream(const W8Params p,
                                                                                          const int rpw) {
  using TB = typename T::bits;
  constexpr int NQ = DUAL ? 2 : 1;
  constexpr bool W16 = WB == 2;
  constexpr int KC = 256 / WB;  // k per 256-byte chunk of a weight row
  static_assert(WB == 1 || WB == 2, "int8 or 16-bit weights");
  extern __shared__ float red[];  // [nwave][NQ][R4][MT4][16]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwave = blockDim.x >> 6;
  const int n0 = blockIdx.x * rpw;
  const int nrows_w = p.n - n0 < rpw ? p.n - n0 : rpw;

  // Descriptors end right after the last valid element: weight rows past the
  // workgroup's share and x rows past `rows` (offset >= rows * stride >= the
  // extent) read 0.
  rsrc_t rq[NQ];
  rq[0] = make_rsrc(static_cast<const int8_t*>(p.q) + static_cast<int64_t>(n0) * p.qs * WB,
                    static_cast<uint32_t>(((nrows_w - 1) * p.qs + p.k) * WB));
  if constexpr (DUAL)
    rq[1] = make_rsrc(static_cast<const int8_t*>(p.q2) + static_cast<int64_t>(n0) * p.qs * WB,
                      static_cast<uint32_t>(((nrows_w - 1) * p.qs + p.k) * WB));
  const rsrc_t rx = make_rsrc(p.x, static_cast<uint32_t>(((p.rows - 1) * p.xs + p.k) * sizeof(TB)));

  const int quad = lane & 3, set_row = (lane & 15) >> 2, kg = lane >> 4;
  // the lane's 16 bytes of a weight row's 256-byte chunk: 16 k (int8) or 8 k
  const int piece = (16 * quad + 64 * kg) >> (WB - 1);
  uint32_t qoff[R4], xoff[MT4];
#pragma unroll
  for (int r = 0; r < R4; ++r) qoff[r] = static_cast<uint32_t>(((4 * r + set_row) * p.qs + piece) * WB);
#pragma unroll
  for (int t = 0; t < MT4; ++t) xoff[t] = static_cast<uint32_t>(((4 * t + set_row) * p.xs + piece) * sizeof(TB));

  // Scales (and bias) of the outputs this thread stores, loaded now so their
  // latency hides behind the weight stream instead of following it.
  constexpr int NOUT = 16 * R4 * MT4;
  constexpr int OPT = (NOUT + 63) / 64;  // outputs per thread with one wave
  float osc[OPT][NQ], obias[OPT];
#pragma unroll
  for (int i = 0; i < OPT; ++i) {
    if constexpr (W16 && DUAL) break;  // no scales, no bias
    const int o = threadIdx.x + i * blockDim.x;
    const int nn = 4 * ((o >> 4) % R4) + (o & 3);
    const bool mine = o < NOUT && nn < nrows_w;
    if constexpr (!W16) {
      osc[i][0] = mine ? load_dyn(p.scale, n0 + nn, p.sdt) : 0.f;
      if constexpr (DUAL) osc[i][NQ - 1] = mine ? load_dyn(p.scale2, n0 + nn, p.sdt) : 0.f;
    }
    obias[i] = mine && !DUAL && p.bdt >= 0 ? load_dyn(p.bias, n0 + nn, p.bdt) : 0.f;
  }

  f32x4 acc[NQ][R4][MT4];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int r = 0; r < R4; ++r) {
#pragma unroll
      for (int t = 0; t < MT4; ++t) acc[qi][r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  const int nchunk = (p.k + KC - 1) >> (W16 ? 7 : 8);
  const int c0 = (nchunk * wave) / nwave, c1 = (nchunk * (wave + 1)) / nwave;
  for (int c = c0; c < c1; c += U) {
    u32x4 wq[U][NQ][R4], xa[U][MT4][2];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const bool live = c + j < c1 && KC * (c + j) + piece < p.k;
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
        for (int r = 0; r < R4; ++r) wq[j][qi][r] = buf_load16(rq[qi], live ? qoff[r] + 256u * (c + j) : kOob);
      }
#pragma unroll
      for (int t = 0; t < MT4; ++t) {
        const uint32_t o = xoff[t] + KC * sizeof(TB) * (c + j);
        xa[j][t][0] = buf_load16_cached(rx, live ? o : kOob);
        if constexpr (!W16) xa[j][t][1] = buf_load16_cached(rx, live ? o + 16u : kOob);
      }
    }
    // every load of the group ahead of its MFMAs: U chunks in flight per wave
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
        for (int r = 0; r < R4; ++r) {
          if constexpr (W16) {
#pragma unroll
            for (int t = 0; t < MT4; ++t) acc[qi][r][t] = mfma16<T>(xa[j][t][0], wq[j][qi][r], acc[qi][r][t]);
          } else {
            u32x4 b0, b1;
            widen_i8x16<T>(wq[j][qi][r], b0, b1);
#pragma unroll
            for (int t = 0; t < MT4; ++t) {
              acc[qi][r][t] = mfma16<T>(xa[j][t][0], b0, acc[qi][r][t]);
              acc[qi][r][t] = mfma16<T>(xa[j][t][1], b1, acc[qi][r][t]);
            }
          }
        }
      }
    }
  }

  // Each lane keeps its diagonal register (l % 4), a quad sum adds the four
  // k-subsets, and lane 16 m' + 4 r' (quad 0) writes acc(x row m', weight row
  // r') of each set to slot 4 m' + r'.
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int r = 0; r < R4; ++r) {
#pragma unroll
      for (int t = 0; t < MT4; ++t) {
        const f32x4 a = acc[qi][r][t];
        float v = quad == 0 ? a.x : (quad == 1 ? a.y : (quad == 2 ? a.z : a.w));
        v += dpp_f32<0xb1>(v);  // quad_perm [1,0,3,2]
        v += dpp_f32<0x4e>(v);  // quad_perm [2,3,0,1]
        if (quad == 0) red[(((wave * NQ + qi) * R4 + r) * MT4 + t) * 16 + (lane >> 2)] = v;
      }
    }
  }
  __syncthreads();

  // Output (x row 4 t + m', weight row 4 r + r') = sum over waves, in order;
  // then the epilogue of w8_store / w8_store_silu with the preloaded scales
  // (16-bit weights: no scales; the single matrix adds the bias in fp32).
#pragma unroll
  for (int i = 0; i < OPT; ++i) {
    const int o = threadIdx.x + i * blockDim.x;
    if (o >= NOUT) break;
    const int slot = o & 15, rt = o >> 4;
    const int r = rt % R4, t = rt / R4;
    const int m = 4 * t + (slot >> 2), nn = 4 * r + (slot & 3);
    if (m >= p.rows || nn >= nrows_w) continue;
    float sum[NQ];
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      sum[qi] = 0.f;
      for (int w = 0; w < nwave; ++w) sum[qi] += red[(((w * NQ + qi) * R4 + r) * MT4 + t) * 16 + slot];
    }
    const int64_t off = static_cast<int64_t>(m) * p.os + n0 + nn;
    if constexpr (W16 && DUAL) {
      store_elem<TO>(p.out, off, silu_mul_f32(sum[0], sum[NQ - 1]));
    } else if constexpr (W16) {
      store_elem<TO>(p.out, off, p.bdt >= 0 ? sum[0] + obias[i] : sum[0]);
    } else if constexpr (DUAL) {
      store_elem<TO>(p.out, off, silu_mul_f32(sum[0] * osc[i][0], sum[NQ - 1] * osc[i][NQ - 1]));
    } else {
      store_elem<TO>(p.out, off, p.bdt >= 0 ? __builtin_fmaf(sum[0], osc[i][0], obias[i]) : sum[0] * osc[i][0]);
    }
  }
}

// Rows per workgroup of a plan of 16-row workgroups, spread evenly over the
// CUs: the fewest rounds of 16 rows per CU, then as few rows per workgroup as
// fill those rounds (8 - 16 where n >= 8 CUs).  Qwen2.5-14B, n 5120: 10 rows
// (512 workgroups, two per CU, where 16 rows leave 320: the down projection
// with 8 rows of x 22.19 -> 17.79 us, the 16-bit one 32.96 -> 25.41); 7B,
// n 3584: 14 (256), n 18944: 15 (1263) (bench.py --only stream-sweep-bal).
inline int balanced_rows16(int n, int cus) {
  const int64_t per_round = 16 * static_cast<int64_t>(cus);
  const int64_t rounds = (n + per_round - 1) / per_round;
  return static_cast<int>((n + rounds * cus - 1) / (rounds * cus));
}

// Launch plan for `rows` <= 64 rows of x (48 when dual) against [n, k] int8
// weights (two matrices when dual), fitted to a graph-timed sweep of rows per workgroup x
// waves x chunks in flight on MI355X over the Qwen2.5-0.5B, 1.5B and 7B
// decode projections and MLPs at 1, 4 and 8 rows (bench.py --only
// w8-stream-sweep; every pick within 1.08x of the best sampled shape, 1.02x
// on geometric average, the best one at the 1.5B gate/up and down and the 7B
// projections with 8 rows):
//   rows per workgroup: 8 (two 4-row sets); narrow outputs (n <= 2048, or
//     fewer 8-row workgroups than CUs) as few as give every CU a workgroup,
//     4 to 8; 16 (the class of balanced_rows16) at k >= 3072 with more than
//     4 rows of x (k >= 2048 beyond 16 rows of int8 weights), or with 2 - 4
//     (4 with 16-bit weights) where that leaves every CU a workgroup (one
//     matrix of int8 weights: 1 - 4 rows, at 1 row 4 per CU) or k >= 8192,
//     since every
//     workgroup re-reads a long x (half the x re-reads of 8); the dual
//     kernel 4 with one row of x (or with up to 4 below k = 3072 or on
//     narrow outputs, or with more where 8-row workgroups would number under
//     4 per CU), else 8 (16 as above with more than 4 rows);
//   waves per workgroup: the dual kernel 3 (half the chunks, two in flight
//     each, with 2 - 4 rows below k = 3072; 2 with more than 4 rows of x and
//     8-row workgroups -- 1 beyond 16 rows --, 8 with 2 - 4 rows at k >= 3072
//     on outputs that are not narrow, 8 with one row at k >= 2048, 1 with
//     16-row workgroups where they number at least 4 per CU, else 2); else
//     about 14 per CU with up to 4 rows of x, 12 (one workgroup per CU) or
//     10 with more, 7 for 16-row workgroups (6 with more than 8 rows of x,
//     12 with up to 4 and more workgroups than CUs); at least 2 (but for
//     the dual kernel's 1) and at most 16 waves (8 where stream_max_threads
//     gives 512 threads), no more than 256-column chunks, and a multiple of
//     4 above 8 when there is at most one workgroup per CU, so the CU's 4
//     SIMDs carry equal loads (14 waves: 1.06x the time of 12; 8 in place
//     of 7);
//   1 chunk in flight per wave (the CU's waves keep enough bytes in flight;
//     the dual kernel's 2 - 4 rows below k = 3072 as above).
// 9 - 16 rows of x (three or four x sets; bench.py --only stream-sweep16 and
// stream-sweep16-wide, 9, 12 and 16 rows): 8 weight rows per workgroup,
// about 8 waves per CU with one workgroup per CU, else 5 (1.5B down, 16 rows
// 8.69 us against 12.47 us for w8a16_skinny), 16 rows at k >= 3072 as above
// (7B down, 16 rows 20.5 - 21.7 us against 27.0 for 8-row workgroups; 7B
// gate/up 20.6 vs 22.9 us for w8a16_skinny, its dual form 33.4 vs 36.2).
// 17 - 32 rows (6 or 8 x sets; bench.py --only stream-sweep32, 20, 24 and
// 32 rows, where the launchers' small tiled shapes do not pay): the same,
// with 7 waves per CU for 16-row workgroups and at most 8 weight rows per
// workgroup for the dual kernel (1.5B down, 32 rows 12.95 us against 20.59
// for w8a16_skinny; 7B down 30.1 vs 44.4; 0.5B down 7.29 vs 12.63).
// 33 - 64 rows (12 or 16 x sets, one matrix; bench.py --only stream-sweep64):
// the same, with as many 4-row weight sets as the registers of that many x
// sets allow (16-bit weights: 2, int8 weights: 2 up to 48 rows, then 1), and
// 7 waves per CU with more workgroups than CUs, at least 4 per workgroup
// (7B down, 64 rows of 16-bit weights: 4 waves 78.9 us, 3 waves 83.4).
// 1 - 4 rows on deep rows (bench.py --only stream-sweep-m4, the 7B
// projections and MLP at 1 - 4 rows): 16-row workgroups (7B gate/up, 3 / 4
// rows 12.72 / 12.74 us against 14.34 / 14.87 with 8 rows; 7B down, 4 rows
// 13.61 vs 15.34; with 16-bit weights from 4 rows, 21.77 vs 22.98), and the
// dual kernel on 8-row workgroups of 8 waves (7B, 3 / 4 rows 22.33 / 22.82
// us against 23.85 / 25.27 on 4-row workgroups of 3); with one row of x the
// 8-row (dual: 4-row) workgroups stay ahead (7B down 12.51 vs 12.92 us) but
// where 16-row ones still fill the CUs (7B gate/up, 12.59 vs 13.18), and so
// they do at k = 3584 where 16-row workgroups leave CUs idle (7B q/o, 2 / 3
// rows 4.48 / 4.65 us against 4.79 / 4.82).
// `wb` is the weight element size the plan is for (k counts bytes).
inline StreamPlan w8_stream_plan(int rows, int k, int n, bool dual, int cus, int wb = 1) {
  const bool two_sets = rows > 4;  // x rows in two (or more) 4-row sets
  const bool four_sets = rows > 8;  // three or more sets
  // 16-row workgroups for one matrix on deep rows (k >= 3072 bytes), where
  // every 8-row workgroup re-reads a long x: with more than 4 rows of x, and
  // with 2 - 4 (4 with 16-bit weights, whose x is half as many bytes per
  // weight byte) at k >= 8192 or where 16-row workgroups still give every CU
  // one -- there with one row of x of int8 weights too
  // (beyond 16 rows of x, with 4 or more times its bytes re-read per 8-row
  // workgroup, from k = 2048 for int8 weights: 3B gate/up, 32 rows 19.68 ->
  // 13.72 us, 20 rows 12.11 -> 11.11)
  const int deep_k = rows > 16 && wb == 1 ? 2048 : 3072;
  // (with one row of x, 4 per CU: the 14B projections, 320 - 864 of them,
  // run 1.4 - 4% faster on 8-row workgroups; the 7B gate/up has 1184)
  const bool deep16 = k >= deep_k && (two_sets || (rows >= 2 * wb && k >= 8192) ||
                                      ((wb == 1 || rows >= 4) && (n + 15) / 16 >= (rows == 1 ? 4 : 1) * cus));
  const bool narrow = n <= 2048 || (n + 7) / 8 < cus;
  // the dual kernel at 2 - 4 rows where one matrix would take 16-row workgroups
  const bool deep_dual = dual && rows >= 2 && !two_sets && deep16 && !narrow;
  const int nchunk = (k + 255) / 256;
  StreamPlan sp{8, 2, 1, 1};
  bool wg16 = false;  // the 16-row class (balanced_rows16)
  if (narrow) {
    sp.rpw = (n + cus - 1) / cus;
    sp.rpw = sp.rpw < 4 ? 4 : (sp.rpw > 8 ? 8 : sp.rpw);
  } else if (dual ? two_sets && rows <= 16 && k >= 3072 : deep16) {
    wg16 = true;
    sp.rpw = balanced_rows16(n, cus);
  }
  // the dual kernel's 8-row workgroups with more than 4 rows of x only where
  // they number at least 4 per CU (0.5B MLP, 608 of them: 4-row workgroups
  // 5 - 10% faster at 6 - 32 rows)
  if (dual && !wg16) sp.rpw = (two_sets && (n + 7) / 8 >= 4 * cus) || deep_dual ? 8 : 4;
  sp.r4 = sp.rpw <= 4 ? 1 : (sp.rpw <= 8 ? 2 : 4);
  // fewer 4-row weight sets where this many x sets leave no registers for more
  while (sp.r4 > 1 && stream_max_threads(sp.r4, stream_x_sets(rows), sp.u, dual, wb) == 0) {
    sp.r4 /= 2;
    if (sp.rpw > 4 * sp.r4) sp.rpw = 4 * sp.r4;
  }
  const int64_t wgs = (n + sp.rpw - 1) / sp.rpw;
  int64_t waves;
  int min_waves = 2;
  if (dual && rows >= 2 && !two_sets && !deep_dual && !wg16 && !narrow && nchunk >= 2) {
    // 2 - 4 rows below k = 3072: every chunk of a wave in flight at once, two
    // per wave (0.5B MLP, 4 rows 4.16 us against 4.66 with 3 waves of one;
    // 3B, 2 rows 9.20 vs 9.39; bench.py --only stream-sweep-dual4)
    sp.u = 2;
    waves = (nchunk + 1) / 2;
    min_waves = 1;
  } else if (dual) {
    // 8-row workgroups with 6 or 8 x sets: one wave (1.5B MLP, 24 rows 13.77
    // us against 15.50 with two; 3B, 32 rows 21.29 vs 25.68), and so any
    // workgroup with 12 x sets (0.5B, 48 rows 11.43 vs 13.20); the 16-row
    // class one where its workgroups number at least 4 per CU, else two (7B
    // MLP, 1263 of them, 16 rows 33.17 us against 39.60 with two; 14B, 988,
    // 35.33 vs 38.15 with one)
    const bool one_wave = (wg16 && wgs >= 4 * static_cast<int64_t>(cus)) || (sp.rpw == 8 && rows > 16) ||
                          rows > 32;
    // (one row of x: 8 waves from k = 2048, 14B MLP 22.61 us against 24.96
    // with 3; 3B 8.99 vs 9.42)
    waves = one_wave ? 1 : (two_sets ? 2 : (deep_dual || (rows == 1 && k >= 2048) ? 8 : 3));
    min_waves = one_wave ? 1 : 2;
  } else {
    // (the 16-row class with one x set and more workgroups than CUs: 12 per
    // CU, its waves carrying few bytes each -- 14B down, 1 row 14.12 us
    // against 15.71 with 7 per CU; bench.py --only stream-sweep-smallm)
    const int per_cu = wg16 && sp.r4 == 4 ? (four_sets && rows <= 16 ? 6 : (two_sets || wgs <= cus ? 7 : 12))
                                    : (four_sets ? (wgs <= cus ? 8 : (rows > 32 ? 7 : 5))
                                                 : (two_sets ? (wgs <= cus ? 12 : 10) : 14));
    waves = (static_cast<int64_t>(per_cu) * cus + wgs / 2) / wgs;
    // beyond 32 rows with more workgroups than CUs a multiple of 4, at least
    // 4 (14B o, 48 rows 26.79 us against 29.34 with 3; the 16-bit 14B down,
    // 64 rows 85.83 vs 88.61; bench.py --only stream-sweep-14b-wide; 1.5B o,
    // 64 rows 8.03 vs 10.70 with 5)
    if (rows > 32 && wgs > cus) waves = waves < 4 ? 4 : waves / 4 * 4;
  }
  const int max_waves = stream_max_threads(sp.r4, stream_x_sets(rows), sp.u, dual, wb) / 64;
  if (waves > max_waves) waves = max_waves;
  if (waves > nchunk) waves = nchunk;
  if (waves < min_waves) waves = nchunk < min_waves ? nchunk : min_waves;
  if (wgs <= cus && waves > 8) waves = waves / 4 * 4;
  // one workgroup per CU: 8 waves, not 7, so each SIMD carries two (7B down
  // with 14-row workgroups, 8 rows of x: 15.28 us against 15.53 with 6)
  if (wgs <= cus && waves == 7 && max_waves >= 8 && nchunk >= 8) waves = 8;
  sp.waves = static_cast<int>(waves);
  return sp;
}

// Launch plan of the 16-bit gate/up + SiLU-and-mul (WB = 2) for `rows` <= 32
// rows of x against two [n, k] weight matrices, from a graph-timed sweep of
// rows per workgroup x waves x chunks in flight on MI355X over the
// Qwen2.5-0.5B, 1.5B and 7B MLPs at 1, 4 and 8 rows (bench.py --only
// gu16-stream-sweep): up to k = 2048, 4 weight rows per workgroup, 2 waves,
// 2 chunks in flight (the most workgroups; 1.5B, 8 rows 11.17 us against
// 12.59 us for gate_up_silu_skinny); deeper (7B), 4 rows and 8 waves with 2
// chunks in flight up to 4 rows of x (39.84 vs 42.77 us), 16 rows and 8
// waves with one chunk beyond, where every workgroup re-reads the long x
// (42.07 vs 44.48 us); 9 - 16 rows (bench.py --only stream-sweep16 and
// stream-sweep16-wide), one chunk in flight, below k = 2048 8 rows per
// workgroup and 2 waves (1.5B, 16 rows 13.44 vs 15.73 us) or 4 rows where
// 8-row workgroups would number under 4 per CU (0.5B, 10 / 12 rows 6.00 /
// 5.92 us against 6.62 / 6.50; bench.py --only stream-sweep-dualn), from
// k = 2048 the 16-row class and about 6 waves per CU (7B, 16 rows one wave,
// 46.1 vs 50.3 us for 8 rows and 8 waves; 3B, 16 rows two, 18.43 vs 20.06).
inline StreamPlan gu16_stream_plan(int rows, int k, int n, int cus) {
  StreamPlan sp{16, 4, 8, 1};
  if (rows > 16) {
    // 17 - 32 rows: 0.5B, 32 rows 9.04 us vs 10.52 for skinny tiles; one
    // wave from k = 2048 (14B, 24 / 32 rows 58.94 / 69.05 us against 68.94 /
    // 78.49 with two; bench.py --only stream-sweep-14b-wide)
    sp = StreamPlan{8, 2, k >= 2048 ? 1 : 2, 1};
  } else if (rows > 8) {
    if (k < 2048) {
      // 4-row workgroups where 8-row ones would number under 4 per CU
      sp = (n + 7) / 8 < 4 * cus ? StreamPlan{4, 1, 2, 1} : StreamPlan{8, 2, 2, 1};
    } else {
      // the 16-row class with about 6 waves per CU (3B, 16 rows: 2 waves;
      // 14B: 2, 48.03 us at 12 rows against 51.47 with one; 7B: 1)
      sp = StreamPlan{16, 4, 1, 1};
      if (n >= 8 * cus) sp.rpw = balanced_rows16(n, cus);
      const int64_t wgs = (n + sp.rpw - 1) / sp.rpw;
      const int64_t w = (6 * static_cast<int64_t>(cus) + wgs / 2) / wgs;
      sp.waves = static_cast<int>(w < 1 ? 1 : (w > 8 ? 8 : w));
    }
  } else if (k <= 2048) {
    sp = StreamPlan{4, 1, 2, 2};
  } else if (rows <= 4) {
    sp = StreamPlan{4, 1, 8, 2};
  } else if (n >= 8 * cus) {
    sp.rpw = balanced_rows16(n, cus);  // 14B, 8 rows: 14 rows 44.03 us against 46.84 with 16
  }
  if (sp.rpw <= 8 && sp.r4 == 4) sp.r4 = 2;
  const int nchunk = (k + 127) / 128;  // no more waves than 128-column chunks
  if (sp.waves > nchunk) sp.waves = nchunk;
  const int max_waves = stream_max_threads(sp.r4, stream_x_sets(rows), sp.u, true, 2) / 64;
  if (sp.waves > max_waves) sp.waves = max_waves;
  return sp;
}

// Launch plan of the 16-bit linear (WB = 2, one matrix) for `rows` <= 64
// rows of x against [n, k] weights, from graph-timed sweeps over the
// Qwen2.5-0.5B, 1.5B and 7B MLP down projections at 1 - 64 rows (bench.py
// --only l16-stream-sweep, stream-sweep32, stream-sweep64): the int8
// kernel's plan for the same
// bytes per weight row (2 k), except
//   - narrow outputs (its plan's 4 - 8 rows per workgroup) with up to 8 rows
//     of x: 2 chunks in flight, about 12 waves per CU with one x set, 8 with
//     two (1.5B down, 1 row 6.36 us against 6.72 with one chunk; 0.5B down,
//     8 rows 4.71 vs 5.04);
//   - 16-row workgroups with more than 8 rows of x: about 7 waves per CU,
//     as with fewer rows (7B down, 16 rows: 8 waves 27.7 us, 7 waves 29.2).
// linear16_skinny, which served these rows before, took 10.27 / 14.75 us
// at the 1.5B down with 8 / 16 rows (now 7.76 / 9.94) and 27.37 / 35.41 us
// at the 7B down (now 23.42 / 27.7).
inline StreamPlan l16_stream_plan(int rows, int k, int n, int cus) {
  StreamPlan sp = w8_stream_plan(rows, 2 * k, n, false, cus, 2);
  const int64_t wgs = (n + sp.rpw - 1) / sp.rpw;
  int per_cu = 0;
  if (sp.rpw <= 8 && (n <= 2048 || (n + 7) / 8 < cus) && rows <= 8) {
    sp.u = 2;
    per_cu = rows <= 4 ? 12 : 8;
  } else if (sp.rpw > 8 && rows > 8) {
    per_cu = 7;
  }
  if (per_cu > 0) {
    int64_t waves = (static_cast<int64_t>(per_cu) * cus + wgs / 2) / wgs;
    const int nchunk = (k + 127) / 128;
    const int max_waves = stream_max_threads(sp.r4, stream_x_sets(rows), sp.u, false, 2) / 64;
    if (waves > max_waves) waves = max_waves;
    if (waves > nchunk) waves = nchunk;
    if (waves < 1) waves = 1;
    if (wgs <= cus && waves > 8) waves = waves / 4 * 4;
    if (wgs <= cus && waves == 7 && max_waves >= 8 && nchunk >= 8) waves = 8;  // as in w8_stream_plan
    sp.waves = static_cast<int>(waves);
  }
  return sp;
}

// Launches w8a16_stream with plan `sp` (rows <= 64, <= 48 when DUAL; k, qs
// multiples of 16 -- of 8 for 16-bit weights --, xs a multiple of 8, x and
// the weights 16-byte aligned: the callers check these).
template <typename T, typename TO, bool DUAL, int WB = 1>
int w8_stream_launch(const W8Params& p, const StreamPlan& sp, hipStream_t s) {
  constexpr int NQ = DUAL ? 2 : 1;
  const int mt4 = stream_x_sets(p.rows);  // 4-row x sets: 1 .. 4, 6, 8, 12, 16
  if (p.rows < 1 || p.rows > (DUAL ? 48 : 64) || (mt4 > 2 && sp.u > 1)) {
    set_error("w8a16 stream launch: %d rows of x (1 - %d; more than 8 take one chunk in flight, u %d)", p.rows,
              DUAL ? 48 : 64, sp.u);
    return MI355_ERR_UNSUPPORTED;
  }
  if ((sp.r4 != 1 && sp.r4 != 2 && sp.r4 != 4) || sp.rpw < 1 || sp.rpw > 4 * sp.r4) {
    set_error("w8a16 stream launch: %d weight rows per workgroup in %d 4-row sets (1, 2 or 4)", sp.rpw, sp.r4);
    return MI355_ERR_UNSUPPORTED;
  }
  const int max_threads = stream_max_threads(sp.r4, mt4, sp.u >= 2 ? 2 : 1, DUAL, WB);
  if (max_threads == 0) {
    set_error("w8a16 stream launch: no kernel for %d rows of x with %d weight rows per workgroup", p.rows, sp.rpw);
    return MI355_ERR_UNSUPPORTED;
  }
  if (sp.waves < 1 || 64 * sp.waves > max_threads) {
    set_error("w8a16 stream launch: %d waves per workgroup, this shape takes 1 - %d", sp.waves, max_threads / 64);
    return MI355_ERR_UNSUPPORTED;
  }
  const dim3 grid(static_cast<unsigned>((p.n + sp.rpw - 1) / sp.rpw));
  const dim3 block(64 * sp.waves);
  const size_t lds = static_cast<size_t>(sp.waves) * NQ * sp.r4 * mt4 * 16 * sizeof(float);
  void* args[] = {const_cast<W8Params*>(&p), const_cast<int*>(&sp.rpw)};
  const void* kern = nullptr;
#define MI355_W8S(R4, MT4, U) kern = reinterpret_cast<const void*>(w8a16_stream<T, TO, R4, MT4, U, DUAL, WB>)
#define MI355_W8S_U(R4, MT4) \
  if (sp.u >= 2) MI355_W8S(R4, MT4, 2); else MI355_W8S(R4, MT4, 1)
#define MI355_W8S_MT(R4) \
  if (mt4 == 1) { MI355_W8S_U(R4, 1); } else { MI355_W8S_U(R4, 2); }
  // three or four x sets: one chunk in flight
#define MI355_W8S_MT4(R4) \
  if (mt4 == 3) { MI355_W8S(R4, 3, 1); } else { MI355_W8S(R4, 4, 1); }
  // six or eight x sets: one chunk in flight, and only the shapes whose
  // registers fit (stream_max_threads > 0; the others were rejected above)
#define MI355_W8S_IF(R4, MT4) \
  if constexpr (stream_max_threads(R4, MT4, 1, DUAL, WB) > 0) MI355_W8S(R4, MT4, 1);
#define MI355_W8S_MT8(R4) \
  if (mt4 == 6) { MI355_W8S_IF(R4, 6) } else { MI355_W8S_IF(R4, 8) }
  // 12 or 16 x sets (33 - 64 rows; the dual kernel 12, with one 4-row weight
  // set: the shapes whose registers fit)
#define MI355_W8S_MT16(R4) \
  if (mt4 == 12) { MI355_W8S_IF(R4, 12) } else { MI355_W8S_IF(R4, 16) }
  if (mt4 <= 2) {
    if (sp.r4 == 4) { MI355_W8S_MT(4) } else if (sp.r4 == 2) { MI355_W8S_MT(2) } else { MI355_W8S_MT(1) }
  } else if (mt4 <= 4) {
    if (sp.r4 == 4) { MI355_W8S_MT4(4) } else if (sp.r4 == 2) { MI355_W8S_MT4(2) } else { MI355_W8S_MT4(1) }
  } else if (mt4 <= 8) {
    if (sp.r4 == 4) { MI355_W8S_MT8(4) } else if (sp.r4 == 2) { MI355_W8S_MT8(2) } else { MI355_W8S_MT8(1) }
  } else {
    if (sp.r4 == 4) { MI355_W8S_MT16(4) } else if (sp.r4 == 2) { MI355_W8S_MT16(2) } else { MI355_W8S_MT16(1) }
  }
#undef MI355_W8S_MT16
#undef MI355_W8S_MT8
#undef MI355_W8S_IF
#undef MI355_W8S_MT4
#undef MI355_W8S_MT
#undef MI355_W8S_U
#undef MI355_W8S
  if (!kern) {
    set_error("w8a16 stream launch: no kernel for %d rows of x with %d weight rows per workgroup", p.rows, sp.rpw);
    return MI355_ERR_UNSUPPORTED;
  }
  return hip_status(hipLaunchKernel(kern, grid, block, args, lds, s), "w8a16 stream launch");
}

}  // namespace mi355
