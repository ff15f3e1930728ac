// Weight-only int8 linear (W8A16), the int8 gate/up projections fused with
// SiLU-and-mul, and the int8 weight quantiser for gfx950, with their
// launchers.
//
//   out[m, n] = round(acc * scale[n] + bias[n]),  acc = sum_k x[m, k] * q[n, k]
//
// Semantics follow the reference's Triton kernel
// (src/kernels/w8a16_matmul_triton.py:64-86): the integer weights meet x in
// 16-bit floating point (every int8 is exact in fp16 and in bf16, and so is
// every product in the fp32 accumulator), the per-output-channel scale is
// applied once to the fp32 accumulator, then the bias (fp32), then one
// rounding to the output type.  Here scale and bias go through one fma.
//
// Four kernels, picked by the launcher:
//   w8a16_stream   rows <= 16 (decode; w8a16_stream.h), and 17 - 48 (49 -
//                  64 for one matrix of at most 8 MB) where the small tiled
//                  shapes do not pay (and the gate/up + SiLU-and-mul at 17 -
//                  24 rows with k <= 2048): weight streaming with
//                  lane-coalesced loads, every weight byte read once per call
//                  at HBM bandwidth, MFMA (v_mfma_f32_16x16x32_{f16,bf16}).
//   w8a16_skinny   9 - 32 rows of wide outputs with 2048 < k < 3072, x
//                  descriptors past 2^32 bytes, and a few 32-row tiles where
//                  the tiled grid would be small: weight streaming with up to
//                  32 rows of x per workgroup (MFMA, the same instruction).
//   tiled_gemm     more rows (prefill): the LDS-tiled MFMA GEMM of
//                  tiled_gemm.h with int8 weights kept int8 in LDS and widened
//                  after each LDS read, scale and bias in its epilogue.
//   w8a16_generic  any k, stride or alignment the three above cannot take:
//                  one wave per (output feature, 4 rows of x), fp32 fma.
//
// And the quantiser of QuantizedLinearInt8.from_linear
// (src/quantization/int8.py:45-50), one wave per weight row:
//   amax = max_k |w|,  scale = max(amax / 127, 1e-8),
//   q = clamp(rint(w / scale), -127, 127)   (IEEE fp32 division, ties to even)
// which is bit-identical to the reference's torch expression.
//
// Skinny operand layout.  The 16x16x32 MFMA's B operand gives lane l column
// n = l % 16 and k-group l / 16 (8 consecutive k).  Each lane loads 16 int8
// weights (one 16-byte load): weight row n % 8, columns 64 * (n / 8) +
// 16 * (l / 16) .. + 16 of a 128-column block, so the 8 lanes of a weight row
// cover 128 contiguous bytes (full cache lines).  The first 8 of the 16
// weights feed one MFMA and the last 8 a second one.  The A operand stacks
// the 8 rows of an x tile twice, row i = x row i % 8 over half i / 8 of the
// block, with the same lane -> column map, so
//   D[i][n] = sum over the block half of x[i % 8] * w[n % 8]  when i / 8 == n / 8
// and the product of x row a with weight row b is D[a][b] + D[a + 8][b + 8]
// (the off-diagonal quarters are discarded).  D layout of the gfx950
// 16x16x32 MFMA: lane l holds rows 4 * (l / 16) + j, j < 4, of column l % 16.
//
// Skinny decomposition: a workgroup owns 8 * G weight rows (blockIdx.y) and a
// tile of 8 * MT rows of x (blockIdx.x) and splits the 128-column blocks of K
// between its waves (contiguous ranges); each wave keeps U blocks of loads in
// flight, and every x operand it loads feeds G weight groups.  Blocks and
// 16-byte pieces past k address past the buffer descriptors (zeros, no
// traffic), so any k that is a multiple of 16 needs no remainder loop.  The
// per-wave partial sums meet in LDS in a fixed order.
#include "common.h"
#include "tiled_gemm.h"
#include "w8a16_stream.h"

namespace mi355 {
namespace {

constexpr int kMaxSplit = 16;  // waves per skinny workgroup

// ------------------------------------------------------------------ skinny

// DUAL: two int8 weight matrices (gate and up) against the same x, each with
// its scale, and SiLU-and-mul in the epilogue; x is loaded once for both.
template <typename T, typename TO, int MT, int G, int U, bool DUAL>
__global__ __launch_bounds__(64 * kMaxSplit) void w8a16_skinny(const W8Params p) {
  using TB = typename T::bits;
  constexpr int NQ = DUAL ? 2 : 1;  // weight matrices
  extern __shared__ float red[];    // [nwave][NQ][G][MT][4][64]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwave = blockDim.x >> 6;
  // x tiles vary fastest, so the workgroups sharing a weight group run
  // together and its re-reads (rows > 8 * MT) hit L2.
  const int m0 = blockIdx.x * 8 * MT;
  const int n0 = blockIdx.y * 8 * G;
  const int nrows_w = p.n - n0 < 8 * G ? p.n - n0 : 8 * G;
  const int nrows_x = p.rows - m0 < 8 * MT ? p.rows - m0 : 8 * MT;

  // Descriptors end right after the last valid element, so weight rows past n
  // and x rows past the tile (offset >= rows * stride >= the extent) read 0.
  rsrc_t rq[NQ];
  rq[0] = make_rsrc(static_cast<const int8_t*>(p.q) + static_cast<int64_t>(n0) * p.qs,
                    static_cast<uint32_t>((nrows_w - 1) * p.qs + p.k));
  if constexpr (DUAL)
    rq[1] = make_rsrc(static_cast<const int8_t*>(p.q2) + static_cast<int64_t>(n0) * p.qs,
                      static_cast<uint32_t>((nrows_w - 1) * p.qs + p.k));
  const rsrc_t rx = make_rsrc(static_cast<const TB*>(p.x) + static_cast<int64_t>(m0) * p.xs,
                              static_cast<uint32_t>(((nrows_x - 1) * p.xs + p.k) * sizeof(TB)));

  // Lane -> (row l % 8 of the operand, column 64 * ((l / 8) % 2) + 16 * (l / 16) of the block).
  const int r8 = lane & 7;
  const int col = ((lane >> 3) & 1) * 64 + (lane >> 4) * 16;
  uint32_t qoff[G], xoff[MT];
#pragma unroll
  for (int g = 0; g < G; ++g) qoff[g] = static_cast<uint32_t>((8 * g + r8) * p.qs + col);
#pragma unroll
  for (int t = 0; t < MT; ++t) xoff[t] = static_cast<uint32_t>(((8 * t + r8) * p.xs + col) * sizeof(TB));

  f32x4 acc[NQ][G][MT];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[qi][g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // The 128-column blocks of K, split over the waves.
  const int nblk = (p.k + 127) >> 7;
  const int s_begin = (nblk * wave) / nwave;
  const int s_end = (nblk * (wave + 1)) / nwave;
  // Block s into slot (wq, xa); blocks past the wave's range or past k load
  // zeros without touching memory.
  auto issue = [&](u32x4 (&wq)[NQ][G], u32x4 (&xa)[MT][2], int s) {
    const bool live = s < s_end && 128 * s + col < p.k;
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
      for (int g = 0; g < G; ++g) wq[qi][g] = buf_load16(rq[qi], live ? qoff[g] + 128u * s : kOob);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const uint32_t o = xoff[t] + 256u * s;
      xa[t][0] = buf_load16_cached(rx, live ? o : kOob);
      xa[t][1] = buf_load16_cached(rx, live ? o + 16u : kOob);
    }
  };
  auto consume = [&](const u32x4 (&wq)[NQ][G], const u32x4 (&xa)[MT][2]) {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        u32x4 b0, b1;
        widen_i8x16<T>(wq[qi][g], b0, b1);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[qi][g][t] = mfma16<T>(xa[t][0], b0, acc[qi][g][t]);
          acc[qi][g][t] = mfma16<T>(xa[t][1], b1, acc[qi][g][t]);
        }
      }
    }
  };
  u32x4 wq[U][NQ][G], xa[U][MT][2];
  // U blocks issued together, then consumed together.
  for (int s = s_begin; s < s_end; s += U) {
#pragma unroll
    for (int j = 0; j < U; ++j) issue(wq[j], xa[j], s + j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < U; ++j) consume(wq[j], xa[j]);
  }

#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          red[((((wave * NQ + qi) * G + g) * MT + t) * 4 + j) * 64 + lane] = acc[qi][g][t][j];
      }
    }
  }
  __syncthreads();

  // Output (x row 8t + a, weight row 8g + b) = D[a][b] + D[a + 8][b + 8]:
  // register a % 4 of lanes 16 * (a / 4) + b and 16 * (a / 4) + 40 + b.
  for (int o = threadIdx.x; o < 64 * G * MT; o += blockDim.x) {
    const int b = o & 7, a = (o >> 3) & 7, gt = o >> 6;
    const int g = gt % G, t = gt / G;
    const int m = 8 * t + a, n = 8 * g + b;
    if (m >= nrows_x || n >= nrows_w) continue;
    const int l0 = 16 * (a >> 2) + b, j = a & 3;
    float sum[NQ];
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      sum[qi] = 0.f;
      for (int w = 0; w < nwave; ++w) {
        const float* r = red + ((((w * NQ + qi) * G + g) * MT + t) * 4 + j) * 64;
        sum[qi] += r[l0] + r[l0 + 40];
      }
    }
    if constexpr (DUAL) w8_store_silu<TO>(p, m0 + m, n0 + n, sum[0], sum[NQ - 1]);
    else w8_store<TO>(p, m0 + m, n0 + n, sum[0]);
  }
}

// ----------------------------------------------------------------- generic

constexpr int kGenRows = 4;  // rows of x per wave

template <typename T, typename TO, bool DUAL>
__global__ __launch_bounds__(256) void w8a16_generic(const W8Params p) {
  constexpr int NQ = DUAL ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t mblocks = (p.rows + kGenRows - 1) / kGenRows;
  if (gw >= static_cast<int64_t>(p.n) * mblocks) return;
  const int n = static_cast<int>(gw % p.n);
  const int64_t m0 = (gw / p.n) * kGenRows;
  const int8_t* qrow[NQ];
  qrow[0] = static_cast<const int8_t*>(p.q) + static_cast<int64_t>(n) * p.qs;
  if constexpr (DUAL) qrow[1] = static_cast<const int8_t*>(p.q2) + static_cast<int64_t>(n) * p.qs;
  float acc[NQ][kGenRows] = {};
  for (int c = lane; c < p.k; c += 64) {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      const float qv = static_cast<float>(qrow[qi][c]);
#pragma unroll
      for (int i = 0; i < kGenRows; ++i) {
        if (m0 + i < p.rows) acc[qi][i] = __builtin_fmaf(load_elem<T>(p.x, (m0 + i) * p.xs + c), qv, acc[qi][i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kGenRows; ++i) {
    float s[NQ];
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) s[qi] = wave_allreduce_sum(acc[qi][i]);
    if (lane == 0 && m0 + i < p.rows) {
      if constexpr (DUAL) w8_store_silu<TO>(p, m0 + i, n, s[0], s[NQ - 1]);
      else w8_store<TO>(p, m0 + i, n, s[0]);
    }
  }
}

// --------------------------------------------------------------- quantiser

template <typename TW>
__global__ __launch_bounds__(256) void quantize_int8_rows(const void* __restrict__ w, int8_t* __restrict__ q,
                                                          float* __restrict__ scale, int64_t n, int k, int64_t ws,
                                                          int64_t qs) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= n) return;
  float amax = 0.f;
  for (int c = lane; c < k; c += 64) amax = __builtin_fmaxf(amax, __builtin_fabsf(load_elem<TW>(w, r * ws + c)));
  // max is exact and order-free; the symmetric butterfly leaves it in every lane
  amax = __builtin_fmaxf(amax, dpp_f32<0xb1>(amax));
  amax = __builtin_fmaxf(amax, dpp_f32<0x4e>(amax));
  amax = __builtin_fmaxf(amax, dpp_f32<0x141>(amax));
  amax = __builtin_fmaxf(amax, dpp_f32<0x140>(amax));
  {
    const uint32_t b = as_u32(amax);
    auto s = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const uint32_t lo = s[0], hi = s[1];
    amax = __builtin_fmaxf(as_f32(lo), as_f32(hi));
  }
  {
    const uint32_t b = as_u32(amax);
    auto s = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    const uint32_t lo = s[0], hi = s[1];
    amax = __builtin_fmaxf(as_f32(lo), as_f32(hi));
  }
  float sc = amax / 127.0f;  // IEEE division (HIP's default for fp32 '/')
  if (sc < 1e-8f) sc = 1e-8f;
  if (lane == 0) scale[r] = sc;
  for (int c = lane; c < k; c += 64) {
    float v = __builtin_rintf(load_elem<TW>(w, r * ws + c) / sc);
    v = __builtin_fminf(__builtin_fmaxf(v, -127.0f), 127.0f);
    q[r * qs + c] = static_cast<int8_t>(static_cast<int>(v));
  }
}

// ---------------------------------------------------------------- launchers

template <typename K>
int launch_w8(K kernel, dim3 grid, dim3 block, size_t lds, const W8Params& p, hipStream_t s) {
  void* args[] = {const_cast<W8Params*>(&p)};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, args, lds, s),
                    "w8a16 launch");
}

// Skinny launch shape (9 - 32 rows, and the 32-row tiles of small grids),
// fitted to a graph-timed sweep of G x waves x U on MI355X over the q/o, k/v,
// gate/up and down projections of Qwen2.5-0.5B, 1.5B and 7B:
//   G (weight-row groups per workgroup; each x operand feeds G B operands)
//     the largest of 4, 2, 1 with n / (8 G) >= 160 (<= 32 rows) or 48
//     (several 32-row tiles); the dual kernel at most 2, and 1 for MT >= 3 so
//     its 2 G MT accumulator tiles fit the register budget;
//   waves per workgroup (the split of K) so that about 1024 (<= 32 rows) or
//     1536 (several 32-row tiles) waves run in total, within the LDS for the
//     partial sums (<= 64 KiB), then evened out so every wave gets the same
//     number of 128-column blocks -- or, when there are no more workgroups
//     than CUs, rounded to a multiple of 4 so the CU's 4 SIMDs carry equal
//     loads;
//   U (blocks in flight per wave) = 2 for narrow outputs (n <= 1536) whose
//     waves own 2 or more blocks, else 1.
template <typename T, typename TO, int MT, int G, bool DUAL>
int w8_skinny_g(const W8Params& p, hipStream_t s, int cus) {
  constexpr int NQ = DUAL ? 2 : 1;
  const int groups = (p.n + 8 * G - 1) / (8 * G);
  const int nblk = (p.k + 127) / 128;
  const int tiles = (p.rows + 8 * MT - 1) / (8 * MT);
  const int64_t units = static_cast<int64_t>(groups) * tiles;
  const int64_t waves = (p.rows <= 32 ? 4 : 6) * static_cast<int64_t>(cus);
  int split = static_cast<int>((waves + units / 2) / units);
  if (split > kMaxSplit) split = kMaxSplit;
  if (split > 64 / (NQ * G * MT)) split = 64 / (NQ * G * MT);  // partial sums: split * NQ * G * MT KiB <= 64 KiB
  if (split > nblk) split = nblk;
  if (split < 1) split = 1;
  int bpw = (nblk + split - 1) / split;
  if (units <= cus && split > 4) {
    // one workgroup per CU: a multiple of 4 waves keeps the CU's 4 SIMDs evenly loaded
    split = ((split + 2) / 4) * 4;
    if (split > 64 / (NQ * G * MT)) split = (64 / (NQ * G * MT)) / 4 * 4;
    if (split > kMaxSplit) split = kMaxSplit;
    bpw = (nblk + split - 1) / split;
  } else {
    split = (nblk + bpw - 1) / bpw;  // even blocks per wave
  }
  const int u = (p.n <= 1536 && bpw >= 2) ? 2 : 1;
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(groups));
  const dim3 block(64 * split);
  const size_t lds = static_cast<size_t>(split) * NQ * G * MT * 4 * 64 * sizeof(float);
  // register budget (128 VGPRs at 1024 threads): U * (4 NQ G + 8 MT) operand
  // dwords + 4 NQ G MT accumulators <= 100
  constexpr int umax = (100 - 4 * NQ * G * MT) / (4 * NQ * G + 8 * MT);
  if (u >= 2 && umax >= 2)
    return launch_w8(w8a16_skinny<T, TO, MT, G, (umax >= 2 ? 2 : 1), DUAL>, grid, block, lds, p, s);
  return launch_w8(w8a16_skinny<T, TO, MT, G, 1, DUAL>, grid, block, lds, p, s);
}

template <typename T, typename TO, int MT, bool DUAL>
int w8_skinny_shape(const W8Params& p, hipStream_t s, int cus) {
  const int min_groups = p.rows <= 32 ? 160 : 48;
  int g = 1;
  if ((p.n + 31) / 32 >= min_groups) g = 4;
  else if ((p.n + 15) / 16 >= min_groups) g = 2;
  constexpr int gmax = !DUAL ? 4 : (MT >= 3 ? 1 : 2);
  if constexpr (gmax >= 4) {
    if (g >= 4) return w8_skinny_g<T, TO, MT, (gmax >= 4 ? 4 : 1), DUAL>(p, s, cus);
  }
  if constexpr (gmax >= 2) {
    if (g >= 2) return w8_skinny_g<T, TO, MT, 2, DUAL>(p, s, cus);
  }
  return w8_skinny_g<T, TO, MT, 1, DUAL>(p, s, cus);
}

// ------------------------------------------------------------------- tiled

// Buffer descriptors of the tiled GEMM span at most 256 rows of x and 256
// weight rows; both must stay below 2^31 bytes.
bool tiled_fits(const W8Params& p, bool) {
  return int64_t{256} * p.xs * 2 < (int64_t{1} << 31) && int64_t{256} * p.qs < (int64_t{1} << 31) &&
         static_cast<int64_t>((p.rows + 63) / 64) * ((p.n + 63) / 64) < (int64_t{1} << 31);
}

// m-blocks per group of the tiled GEMM's tile order inside each XCD's range
// (m fastest within a group).
constexpr int kW8GroupM = 4;

template <typename T, typename TO, int WGM, int WGN, int FM, int FN, int S, int EPI = tiled::EPI_W8, int RING = 0,
          int WPE = 0, int XR = 0>
int w8_tiled_cfg(const W8Params& p, hipStream_t s) {
  using C = tiled::Cfg<T, tiled::B_I8, TO, WGM, WGN, FM, FN, EPI, S>;
  static_assert(C::LDS <= 160 * 1024, "LDS per workgroup");
  // A tile count that is not a multiple of 8 takes the instantiation that
  // gives the XCDs contiguous tile ranges for any count (XR = 1; the
  // multiples of 8 keep the other, whose code predates it).  Prefill row
  // counts are mostly not powers of two: 1.5B gate/up at 1400 rows (770
  // tiles of 128 x 128) 66.1 -> 58.3 us, 2900 rows 112.0 -> 103.8 us, 7B
  // gate/up at 1100 rows 179.2 -> 174.9 us; the narrow outputs even.
  if constexpr (XR == 0) {
    const int64_t ntiles = static_cast<int64_t>((p.rows + C::BM - 1) / C::BM) * ((p.n + C::BN - 1) / C::BN);
    if (ntiles % 8 != 0) return w8_tiled_cfg<T, TO, WGM, WGN, FM, FN, S, EPI, RING, WPE, 1>(p, s);
  }
  tiled::Params tp{};
  tp.x = p.x;
  tp.b0 = p.q;
  tp.b1 = EPI == tiled::EPI_SILU_W8 ? p.q2 : p.q;
  tp.scale = p.scale;
  tp.scale1 = p.scale2;
  tp.bias = p.bias;
  tp.out = p.out;
  tp.rows = p.rows;
  tp.k = p.k;
  tp.n = p.n;
  tp.xs = p.xs;
  tp.bs = p.qs;
  tp.os = p.os;
  tp.sdt = p.sdt;
  tp.bdt = p.bdt;
  tp.tiles_m = (p.rows + C::BM - 1) / C::BM;
  tp.tiles_n = (p.n + C::BN - 1) / C::BN;
  tp.group_m = tp.tiles_m < kW8GroupM ? tp.tiles_m : kW8GroupM;
  void* args[] = {&tp};
  // all LDS is static (no dynamic shared memory)
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(tiled::tiled_gemm<T, tiled::B_I8, TO, WGM, WGN, FM, FN,
                                                                                      EPI, S, RING, WPE, XR>),
                                    dim3(static_cast<unsigned>(tp.tiles_m * tp.tiles_n)), dim3(C::BLOCK), args, 0, s),
                    "w8a16 tiled launch");
}

// Outside the ring's range (below), the step pipeline's tile shape by the
// number T of 128 x 128 output tiles, from a sweep of tile shapes x waves x
// LDS stages on MI355X over the q/o, k/v, gate/up and down projections of
// Qwen2.5-1.5B and 7B at 128, 1024 and 4096 rows (every pick within 5% of
// the best sampled configuration but one, 1024 rows x k 8960, at 1.05x):
//   T < 128 -> 64 x 64 tiles, 4 waves, 4 stages (the most workgroups);
//   T < 320, or n > 2048 (fewer than two ring tiles per CU) -> 128 x 128,
//     8 waves, 3 stages;
//   else (n <= 2048) -> 128 x 256, 8 waves, 4 stages.
// bf16 takes 128 x 128 where fp16 takes 128 x 256: its widening needs more
// registers, and the 128 x 256 shape would spill.
template <typename T, typename TO>
int w8_tiled(const W8Params& p, hipStream_t s, int cus) {
  constexpr bool wide = std::is_same<T, F16>::value;
  // Wide outputs from 1024 rows at gate/up and o-projection depths (k <=
  // 4096): 128 x 128 tiles of 8 waves (64 x 32 each) behind a 3-stage ring,
  // two workgroups per CU, so 16 waves per CU issue the global -> LDS DMA
  // that bounds this GEMM, for 40% fewer operand bytes per flop than 128 x 64
  // tiles.  Measured against the plan below and forced configurations 1-33:
  // 1.5B gate/up 1024 rows 45.8 vs 49.8 us, 4096 rows 138.6 vs 155.8 us; 7B
  // gate/up (bf16) 149.4 vs 178.5 and 556.9 vs 582.2 us; 7B o projection and
  // n = 4736 even.  The deep 7B down projection (k = 18944) at 4096 rows
  // keeps the plan below (512.7 vs 533.8 us).
  // Where 192 x 128 tiles (8 waves of 96 x 32, 2-stage ring) fit in one
  // round of two workgroups per CU and 128 x 128 tiles would need a second,
  // the 192 x 128 tile with its registers capped at 128 (4 waves per SIMD,
  // so two workgroups fit on a CU): 1.5B gate/up at 1024 rows, 420 tiles
  // against 560 of 128 x 128 on 512 slots, 43.0 vs 46.8 us.  (Its tile
  // counts here are rarely multiples of 8: XR = 1, 43.2 vs 44.4 us at 420
  // tiles.)
  if (p.n > 2048 && p.rows >= 1024 && p.k <= 4096) {
    const int64_t cols = (p.n + 127) / 128;
    const int64_t t192 = (p.rows + 191) / 192 * cols, t128x128 = (p.rows + 127) / 128 * cols;
    if (t192 <= 2 * static_cast<int64_t>(cus) && t128x128 > 2 * static_cast<int64_t>(cus))
      return w8_tiled_cfg<T, TO, 2, 4, 3, 1, 2, tiled::EPI_W8, 1, 4, 1>(p, s);
    return w8_tiled_cfg<T, TO, 2, 4, 2, 1, 3, tiled::EPI_W8, 1>(p, s);
  }
  // Below 1024 rows, wide outputs with at least two 128 x 64 tiles per CU: the sub-step ring
  // (2 stages) at the shape whose busiest CU finishes first -- ceil(tiles /
  // CUs) times the cost of one tile of 128 x 64 (4 waves, 40 KiB of LDS, four
  // workgroups per CU), 256 x 128 (8 waves of 128 x 32, two per CU) or
  // 256 x 256 (8 waves of 64 x 128), measured about 1 : 3.8 : 6.4 at the
  // Qwen2.5-1.5B and 7B gate/up and down projections (1.5B gate 512 rows
  // 34.9 -> 26.2 us, 7B down 4096 rows 641 -> 522 us; the 3.8 from a later
  // sweep, where 128 x 64 tiles took 158-160 us at 1.5B gate/up 4096 rows
  // against 165-168 us for 256 x 128).  Fewer tiles keep the rule below,
  // whose smaller grids spread better.
  if (p.n > 2048) {
    const auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
    const int64_t t_small = cdiv(p.rows, 128) * cdiv(p.n, 64);
    if (t_small >= 2 * static_cast<int64_t>(cus)) {
      const double c_small = static_cast<double>(cdiv(t_small, cus));
      const double c_mid = 3.8 * static_cast<double>(cdiv(cdiv(p.rows, 256) * cdiv(p.n, 128), cus));
      const double c_big = 6.4 * static_cast<double>(cdiv(cdiv(p.rows, 256) * cdiv(p.n, 256), cus));
      if (c_small <= c_mid && c_small <= c_big) return w8_tiled_cfg<T, TO, 2, 2, 2, 1, 2, tiled::EPI_W8, 1>(p, s);
      if (c_mid <= c_big) return w8_tiled_cfg<T, TO, 2, 4, 4, 1, 2, tiled::EPI_W8, 1>(p, s);
      return w8_tiled_cfg<T, TO, 4, 2, 2, 4, 2, tiled::EPI_W8, 1>(p, s);
    }
  }
  // Narrow outputs (n <= 2048) whose 64 x 128 tiles number between half and
  // all of the CUs: 8 waves of 32 x 32 per tile behind a 4-stage ring, one
  // tile per CU with 8 waves issuing its DMA (forced configurations 17 and
  // 34-36 against the plan below: 1.5B down 1024 rows 49.8 vs 59.4 us, 1280
  // rows 51.6 vs 60.6; q/o 1024 rows 13.8 vs 15.6; n = 2048 14.1 vs 18.5;
  // 768 rows even).  Fewer tiles (512-row down and q/o, n = 1024) and more
  // (2048 rows and up) run faster on the shapes below.
  const int64_t t64x128 = static_cast<int64_t>((p.rows + 63) / 64) * ((p.n + 127) / 128);
  if (p.n <= 2048 && 2 * t64x128 > cus && t64x128 <= cus)
    return w8_tiled_cfg<T, TO, 2, 4, 1, 1, 4, tiled::EPI_W8, 1>(p, s);
  const int64_t t128 = static_cast<int64_t>((p.rows + 127) / 128) * ((p.n + 127) / 128);
  if (t128 < 128) return w8_tiled_cfg<T, TO, 2, 2, 1, 1, 4>(p, s);
  if (t128 < 320 || p.n > 2048) return w8_tiled_cfg<T, TO, 2, 4, 2, 1, 3>(p, s);
  if constexpr (wide) return w8_tiled_cfg<T, TO, 2, 4, 2, 2, 4>(p, s);
  else return w8_tiled_cfg<T, TO, 2, 4, 2, 1, 3>(p, s);
}

// The dual (gate/up + SiLU-and-mul) tiled GEMM: more than 256 rows by the
// round count below; else, up to n = 10000, 128 x 64 tiles (4 waves, 4
// stages), beyond 128 x 128 (8 waves, 3 stages; fp16) -- the 16-bit gate/up
// GEMM's step-pipeline shapes, less its 256 x 64 one, whose 4 KiB int8 B
// tile does not split into the 8 waves' 1 KiB DMA instructions.  bf16 keeps
// the 128 x 64 shape there (its widening needs more registers; 128 x 128 at
// 8 waves would spill).
template <typename T, typename TO>
int w8_tiled_dual(const W8Params& p, hipStream_t s, int cus) {
  // More than 256 rows: the sub-step ring (2 stages), 128 x 64 tiles (4
  // waves, 48 KiB of LDS, three workgroups per CU) or 256 x 128 (8 waves of
  // 128 x 32), whichever takes fewer rounds, a round of 256 x 128 weighted
  // 1.28 (measured at the Qwen2.5-1.5B and 7B MLPs, 512 - 4096 rows: 1.5B
  // 1024 rows 90.8 -> 70.2 us, 7B 2048 rows 719 -> 494 us).
  if (p.rows > 256) {
    const auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
    const double c_small = static_cast<double>(cdiv(cdiv(p.rows, 128) * cdiv(p.n, 64), 3 * static_cast<int64_t>(cus)));
    const double c_big = 1.28 * static_cast<double>(cdiv(cdiv(p.rows, 256) * cdiv(p.n, 128), cus));
    if (c_small <= c_big) return w8_tiled_cfg<T, TO, 2, 2, 2, 1, 2, tiled::EPI_SILU_W8, 1>(p, s);
    return w8_tiled_cfg<T, TO, 2, 4, 4, 1, 2, tiled::EPI_SILU_W8, 1>(p, s);
  }
  if constexpr (std::is_same<T, F16>::value) {
    if (p.rows > 256 || p.n > 10000) return w8_tiled_cfg<T, TO, 2, 4, 2, 1, 3, tiled::EPI_SILU_W8>(p, s);
  }
  return w8_tiled_cfg<T, TO, 2, 2, 2, 1, 4, tiled::EPI_SILU_W8>(p, s);
}

// Small tiled shapes for 17 - 64 rows: 32 x 64 (2 waves) or, for n > 10000,
// 32 x 128 (4 waves) up to 32 rows; 64 x 64 (4 waves) up to 64; 4 stages.
// They read each weight byte once and x once per workgroup, where 24- or
// 32-row skinny tiles re-load x for every weight piece and more rows re-read
// the weights per 32-row tile -- but only win with >= 128 tile columns to
// spread over the CUs (a sweep over the Qwen2.5-1.5B / 7B projections at 16 -
// 64 rows: int8 gate/up 7B, 32 rows 85.1 -> 40.7 us, 1.5B 21.3 -> 14.8 us;
// the 1536-wide down and q/o projections 1.8x slower, so they keep split-K
// weight streaming).
bool small_tiles_pay(int rows, int n) {
  const int bn = (rows <= 32 && n > 10000) ? 128 : 64;
  return rows > 16 && rows <= 64 && (n + bn - 1) / bn >= 128;
}

template <typename T, typename TO, bool DUAL>
int w8_tiled_small(const W8Params& p, hipStream_t s) {
  constexpr int EPI = DUAL ? tiled::EPI_SILU_W8 : tiled::EPI_W8;
  if (p.rows <= 32) {
    if (p.n > 10000) return w8_tiled_cfg<T, TO, 1, 4, 1, 1, 4, EPI>(p, s);
    return w8_tiled_cfg<T, TO, 1, 2, 1, 1, 4, EPI>(p, s);
  }
  return w8_tiled_cfg<T, TO, 2, 2, 1, 1, 4, EPI>(p, s);
}

template <typename T, typename TO, bool DUAL>
int w8_typed(const W8Params& p, hipStream_t s, int cus) {
  const bool vec = p.k % 16 == 0 && p.qs % 16 == 0 && p.xs % 8 == 0 && aligned16(p.x) && aligned16(p.q) &&
                   (!DUAL || aligned16(p.q2));
  if (!vec) {
    const int64_t waves = static_cast<int64_t>(p.n) * ((p.rows + kGenRows - 1) / kGenRows);
    return launch_w8(w8a16_generic<T, TO, DUAL>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, p, s);
  }
  // Up to 16 rows, but 9 - 16 rows of wide outputs with 2048 < k < 3072
  // (w8a16_skinny there; at k >= 3072 the stream kernel's 16-row workgroups
  // win, the 7B gate/up at 16 rows 22.9 -> 20.6 us, its dual form 36.2 ->
  // 33.4 us; everywhere else in the sweep the stream kernel wins, 1.5B down
  // 12.5 -> 8.7 us, gate/up 8.9 -> 7.5 us at 16 rows).
  // (The stream kernel's x descriptor spans all rows of x: under 2^32 bytes.)
  const bool x_fits = ((p.rows - 1) * p.xs + p.k) * static_cast<int64_t>(sizeof(typename T::bits)) < (int64_t{1} << 32);
  const bool wide_mid = p.n > 10000 && p.k > 2048 && p.k < 3072;
  if (x_fits && (p.rows <= 8 || (p.rows <= 16 && !wide_mid)))
    return w8_stream_launch<T, TO, DUAL>(p, w8_stream_plan(p.rows, p.k, p.n, DUAL, cus), s);
  if (p.rows <= 16) return w8_skinny_shape<T, TO, 2, DUAL>(p, s, cus);
  // The int8 gate/up + SiLU-and-mul at 17 - 24 rows of MLPs with k <= 2048:
  // the stream kernel's 8-row workgroups of one wave beat the small tiles
  // (1.5B, 18 / 24 rows 15.46 / 15.50 -> 13.40 / 13.77 us; from 28 rows the
  // tiles lead, 15.53 vs 15.85, and at the 7B MLP, 20 rows 40.7 vs 45.8).
  const bool dual_stream = DUAL && p.rows <= 24 && p.k <= 2048;
  if (small_tiles_pay(p.rows, p.n) && tiled_fits(p, DUAL) && !dual_stream) return w8_tiled_small<T, TO, DUAL>(p, s);
  // 17 - 32 rows where the small tiles do not pay: the stream kernel with 6
  // or 8 x sets (1.5B down, 32 rows 20.6 -> 13.0 us; 7B down 44.4 -> 30.1;
  // 0.5B down 12.6 -> 7.3; the int8 gate/up + SiLU-and-mul, 0.5B 9.7 -> 8.9),
  // and with 12 x sets up to 48 rows (1.5B down, 48 rows 31.4 -> 16.4 us;
  // 7B down 79.5 -> 59.8; 7B o 19.9 -> 15.5; the int8 gate/up +
  // SiLU-and-mul, 0.5B 15.6 -> 11.4).  From 49 rows int8 weights leave
  // registers for one 4-row weight set only (the dual kernel none): one
  // matrix of at most 8 MB still streams faster (0.5B down, 64 rows 14.6 ->
  // 10.8 us; 1.5B o 9.3 -> 8.0), the deep projections do not (1.5B down,
  // 13.8 MB, 30.9 vs 28.7 us for the skinny tiles; 7B down 115.9 vs 82.2).
  const bool small_w = static_cast<int64_t>(p.n) * p.k <= (int64_t{8} << 20);
  if ((p.rows <= 48 || (!DUAL && p.rows <= 64 && small_w)) && x_fits && !wide_mid)
    return w8_stream_launch<T, TO, DUAL>(p, w8_stream_plan(p.rows, p.k, p.n, DUAL, cus), s);
  if (p.rows <= 24) return w8_skinny_shape<T, TO, 3, DUAL>(p, s, cus);
  if (p.rows <= 32) return w8_skinny_shape<T, TO, 4, DUAL>(p, s, cus);
  // More rows: the tiled GEMM, except where 32-row skinny tiles with split K,
  // which re-read the int8 weights per tile mostly from L2, measured faster:
  // tiny grids (fewer than 32 64 x 64 tiles: 1.5B k/v at 96 - 256 rows, 6.4
  // vs 10.5 us) and narrow outputs (n < 2048) up to 128 rows (1.5B down, 128
  // rows 30.7 vs 34.3 us).  Wider outputs and more rows re-read too much
  // (7B down, 96 rows 105.6 vs 82.8 us; 1.5B down, 256 rows 57.6 vs 34.7).
  const int64_t tiles64 = static_cast<int64_t>((p.n + 63) / 64) * ((p.rows + 63) / 64);
  bool skinny = p.rows <= 256 && (tiles64 < 32 || (p.rows <= 128 && p.n < 2048));
  if (!tiled_fits(p, DUAL)) skinny = true;
  if (skinny) return w8_skinny_shape<T, TO, 4, DUAL>(p, s, cus);
  if constexpr (DUAL) return w8_tiled_dual<T, TO>(p, s, cus);
  else return w8_tiled<T, TO>(p, s, cus);
}

}  // namespace

int w8a16_launch(const void* x, const void* q, const void* scale, const void* bias, void* out, int rows, int k,
                 int n, int64_t xs, int64_t qs, int64_t os, int x_dtype, int scale_dtype, int bias_dtype,
                 int out_dtype, hipStream_t stream) {
  int cus = 0;
  const int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  const W8Params p{x, q, scale, bias, out, rows, k, n, xs, qs, os, scale_dtype, bias ? bias_dtype : -1, nullptr,
                   nullptr};
  if (x_dtype == MI355_F16 && out_dtype == MI355_F16) return w8_typed<F16, F16, false>(p, stream, cus);
  if (x_dtype == MI355_F16 && out_dtype == MI355_F32) return w8_typed<F16, F32, false>(p, stream, cus);
  if (x_dtype == MI355_BF16 && out_dtype == MI355_BF16) return w8_typed<BF16, BF16, false>(p, stream, cus);
  if (x_dtype == MI355_BF16 && out_dtype == MI355_F32) return w8_typed<BF16, F32, false>(p, stream, cus);
  set_error("mi355_w8a16_linear_fwd: unsupported dtype pair (x=%d, out=%d)", x_dtype, out_dtype);
  return MI355_ERR_UNSUPPORTED;
}

int gate_up_silu_w8a16_launch(const void* x, const void* qg, const void* qu, const void* sg, const void* su, void* out,
                              int rows, int k, int n, int64_t xs, int64_t qs, int64_t os, int x_dtype,
                              int scale_dtype, int out_dtype, hipStream_t stream) {
  int cus = 0;
  const int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  const W8Params p{x, qg, sg, nullptr, out, rows, k, n, xs, qs, os, scale_dtype, -1, qu, su};
  if (x_dtype == MI355_F16 && out_dtype == MI355_F16) return w8_typed<F16, F16, true>(p, stream, cus);
  if (x_dtype == MI355_F16 && out_dtype == MI355_F32) return w8_typed<F16, F32, true>(p, stream, cus);
  if (x_dtype == MI355_BF16 && out_dtype == MI355_BF16) return w8_typed<BF16, BF16, true>(p, stream, cus);
  if (x_dtype == MI355_BF16 && out_dtype == MI355_F32) return w8_typed<BF16, F32, true>(p, stream, cus);
  set_error("mi355_gate_up_silu_w8a16_fwd: unsupported dtype pair (x=%d, out=%d)", x_dtype, out_dtype);
  return MI355_ERR_UNSUPPORTED;
}

int quantize_int8_launch(const void* w, void* q, void* scale, int64_t n, int k, int64_t ws, int64_t qs, int w_dtype,
                         hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>((n + 3) / 4);
  void* args[] = {const_cast<void**>(&w), &q, &scale, &n, &k, &ws, &qs};
  const void* kern = nullptr;
  if (w_dtype == MI355_F32) kern = reinterpret_cast<const void*>(quantize_int8_rows<F32>);
  else if (w_dtype == MI355_F16) kern = reinterpret_cast<const void*>(quantize_int8_rows<F16>);
  else if (w_dtype == MI355_BF16) kern = reinterpret_cast<const void*>(quantize_int8_rows<BF16>);
  if (!kern) {
    set_error("mi355_quantize_int8_fwd: unsupported weight dtype %d", w_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  return hip_status(hipLaunchKernel(kern, dim3(grid), dim3(256), args, 0, stream), "quantize_int8 launch");
}

}  // namespace mi355
