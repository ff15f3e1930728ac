// Measurement-only, not part of the kernel ABI: the W8A16 prefill GEMM
// (tiled_gemm.h, int8 B, EPI_W8, sub-step ring) with its int8 weight operand
// loaded straight from global memory into registers, so that the LDS ring
// and its global -> LDS DMA carry x alone, timed against the library's
// kernel at the same tile configuration (instantiated from the same header).
//
// Each lane needs, per 64-column K step, the 32 bytes of weight row
// (wn FN 32 + 32 j + l % 32) at bytes 32 (l / 32) .. + 32 of the step: the
// two 16-byte chunks 2 h and 2 h + 1 (h = l / 32) that the LDS path reads
// (chunk 2 h + q feeds sub-steps 2 q and 2 q + 1).  Two waves of the
// workgroup (WGM = 2) share each weight column block and both load it.
//
// The loads are inline asm, like the DMA: the compiler does not track them,
// so its own waits never drain the DMA in flight, and the kernel orders
// them itself.  Weights of step t + 2 are loaded during step t, into the
// register set of step t's parity (free once step t's last widening has
// read it).  Per step a wave issues its weight loads, then its DMA; before
// the barrier of step t it waits until at most the DMA issued by step t - 1
// is outstanding (2 stages: nothing), which covers step t + 1's weights and
// its x.  The last steps (guarded) use compiler-visible loads and wait for
// everything.  After each wait an empty asm redefines the registers just
// landed, so no use of them can be placed before it.
//
// Measured on MI355X at the 1.5B and 7B gate/up projections (bench.py --only
// w8-breg): 1.17-1.62x slower than the LDS path at every configuration.
#include "../tiled_gemm.h"

namespace mi355 {
namespace tiled {
namespace {

__device__ __forceinline__ u32x4 breg_load(rsrc_t r, uint32_t voff, uint32_t soff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=&v"(v) : "v"(voff), "s"(r), "s"(soff) : "memory");
  return v;
}
__device__ __forceinline__ void breg_ready(u32x4& v) { asm volatile("" : "+v"(v)); }

template <typename T, typename TO, int WGM, int WGN, int FM, int FN, int S, int WPE, int XR>
__global__ __launch_bounds__(64 * WGM * WGN)
__attribute__((amdgpu_waves_per_eu(kMinWavesPerSimd<WPE>))) void tiled_w8_breg(const Params p) {
  using TB = typename T::bits;
  constexpr int NW = WGM * WGN, BM = 32 * FM * WGM, BN = 32 * FN * WGN;
  constexpr int A_BYTES = BM * 128, STAGE = A_BYTES;
  constexpr int AI = A_BYTES / 1024 / NW;  // DMA instructions per wave per step
  constexpr int BRI = 2 * FN;              // weight loads per wave per step
  constexpr int U = lcm_c(S, 2);           // steps per main-loop iteration (stage and set known)
  static_assert(A_BYTES % (1024 * NW) == 0, "x tile must split over the waves");
  static_assert(S >= 2 && S <= 8 && (S + 1) * (AI + BRI) < 64, "stages / vmcnt range");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  const int ntiles = p.tiles_m * p.tiles_n;
  int b = blockIdx.x;
  if constexpr (XR != 0) {
    const int q = ntiles >> 3, r = ntiles & 7, x = b & 7;
    b = x * q + (x < r ? x : r) + (b >> 3);
  } else {
    if ((ntiles & 7) == 0) b = (b & 7) * (ntiles >> 3) + (b >> 3);
  }
  const int per_group = p.group_m * p.tiles_n;
  const int g0 = (b / per_group) * p.group_m;
  const int gsz = p.tiles_m - g0 < p.group_m ? p.tiles_m - g0 : p.group_m;
  const int tm = g0 + (b % per_group) % gsz, tn = (b % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nrows_x = p.rows - m0 < BM ? p.rows - m0 : BM;
  const int nrows_b = p.n - n0 < BN ? p.n - n0 : BN;

  const rsrc_t rx = make_rsrc(static_cast<const TB*>(p.x) + static_cast<int64_t>(m0) * p.xs,
                              static_cast<uint32_t>(((nrows_x - 1) * p.xs + p.k) * sizeof(TB)));
  const rsrc_t rb = make_rsrc(static_cast<const uint8_t*>(p.b0) + static_cast<int64_t>(n0) * p.bs,
                              static_cast<uint32_t>((nrows_b - 1) * p.bs + p.k));
  const int nk = (p.k + 63) >> 6;
  const int kfull = p.k >> 6;

  uint32_t a_goff[AI];
  int a_col[AI];
#pragma unroll
  for (int j = 0; j < AI; ++j) {
    const int r = 8 * (NW * j + wave) + (lane >> 3);
    const int c = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
    a_goff[j] = static_cast<uint32_t>((r * p.xs + 8 * c) * sizeof(TB));
    a_col[j] = 8 * c;
  }
  const uint32_t lrow = lane & 31, h = lane >> 5;
  const uint32_t arow0 = wm * FM * 32 + lrow;
  const uint32_t brow0 = wn * FN * 32 + lrow;
  uint32_t b_off[FN][2];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
#pragma unroll
    for (int q = 0; q < 2; ++q) b_off[j][q] = static_cast<uint32_t>((brow0 + 32 * j) * p.bs + 16 * (2 * h + q));
  }

  auto issue_a = [&](auto I, int kt) {
    const uint32_t st = stage_addr<decltype(I)::value, STAGE>();
    const bool full = kt < kfull;
#pragma unroll
    for (int j = 0; j < AI; ++j) {
      const uint32_t kb = static_cast<uint32_t>(kt * 64 * sizeof(TB));
      const uint32_t dst = st + 1024u * (NW * j + wave);
      if (full) dma16(rx, a_goff[j], kb, dst);
      else dma16(rx, kt * 64 + a_col[j] < p.k ? a_goff[j] + kb : kOob, 0, dst);
    }
  };
  u32x4 bq[2][FN][2];  // raw int8 weights of two steps, by step parity
  // Weights of step kt into register set SET: inline asm (ASM, the main
  // loop; the kernel waits for them itself) or compiler-visible loads (the
  // last steps, whose branches would otherwise merge registers still in
  // flight).  Chunks at or past k read 0.
  auto issue_b = [&](auto SET, auto ASM, int kt) {
    constexpr int set = decltype(SET)::value;
    const bool full = kt < kfull;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t kb = static_cast<uint32_t>(kt * 64);
        const uint32_t off = full || kt * 64 + 16 * (2 * static_cast<int>(h) + q) < p.k ? b_off[j][q] + kb : kOob;
        if constexpr (decltype(ASM)::value) bq[set][j][q] = breg_load(rb, off, 0);
        else bq[set][j][q] = buf_load16_cached(rb, off);
      }
    }
  };
  auto ready_b = [&](auto SET) {
    constexpr int set = decltype(SET)::value;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      breg_ready(bq[set][j][0]);
      breg_ready(bq[set][j][1]);
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    }
  }

  u32x4 a[2][FM];  // x pieces of two sub-steps
  u32x4 wb[2][FN];  // widened weights of two sub-steps
  auto read_a = [&](auto I, int s) {
    const uint8_t* abase = stage_ptr<decltype(I)::value, STAGE>();
#pragma unroll
    for (int i = 0; i < FM; ++i) a[s & 1][i] = lds_read16(abase, swz16(arow0 + 32 * i, 4 * h + s));
  };
  // sub-step s's weights (raw pair s / 2, half s % 2) of register set SET into wb[s & 1]
  auto widen = [&](auto SET, int s) {
    constexpr int set = decltype(SET)::value;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const u32x4 raw = bq[set][j][(s >> 1) & 1];
      wb[s & 1][j] = (s & 1) ? widen8<T>(raw.z, raw.w) : widen8<T>(raw.x, raw.y);
    }
  };
  auto mfma = [&](int s) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma32<T>(wb[s & 1][j], a[s & 1][i], acc[i][j]);
    }
  };
  using Z = std::integral_constant<int, 0>;
  using O = std::integral_constant<int, 1>;
  using Yes = std::true_type;
  using No = std::false_type;

  // A step is split where no asm weight load is in flight, so that every
  // branch and loop edge of the kernel falls there:
  //   head(t): sub-steps 0 .. 2 of step t, then the wait, the barrier and
  //            the weights of step t + 1 made ready;
  //   tail(t): the loads of step t + 2's weights and step t + S's x, sub-step
  //            0 of step t + 1's x, sub-step 3's MFMAs of step t, and step
  //            t + 1's first weights widened.
  auto head = [&](auto I, auto GUARD, int t) {
    constexpr int si = decltype(I)::value % S, par = decltype(I)::value & 1;
    constexpr bool guard = decltype(GUARD)::value;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      read_a(std::integral_constant<int, si>{}, s + 1);
      __builtin_amdgcn_sched_barrier(0);
      mfma(s);
      __builtin_amdgcn_sched_barrier(0);
      widen(std::integral_constant<int, par>{}, s + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!guard || t + 1 < nk) {
      if (!guard) wait_vmcnt<(S == 2 ? 0 : AI)>();  // t + 1's weights (issued before the last DMA) and x
      else wait_vmcnt<0>();
      wait_lgkmcnt0();
      lds_barrier();
      if (!guard) ready_b(std::integral_constant<int, par ^ 1>{});
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto tail = [&](auto I, auto GUARD, int t) {
    constexpr int si = decltype(I)::value % S, par = decltype(I)::value & 1;
    constexpr bool guard = decltype(GUARD)::value;
    const bool more = !guard || t + 1 < nk;
    __builtin_amdgcn_sched_barrier(0);
    if (!guard) issue_b(std::integral_constant<int, par>{}, Yes{}, t + 2);
    else if (t + 2 < nk) issue_b(std::integral_constant<int, par>{}, No{}, t + 2);
    if (!guard || t + S < nk) issue_a(std::integral_constant<int, si>{}, t + S);
    if (more) read_a(std::integral_constant<int, (si + 1) % S>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    mfma(3);
    __builtin_amdgcn_sched_barrier(0);
    if (more) widen(std::integral_constant<int, par ^ 1>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue (nk >= 2): weights of steps 0 and 1, x of steps 0 .. S - 1
  issue_b(Z{}, Yes{}, 0);
  issue_a(Z{}, 0);
  issue_b(O{}, Yes{}, 1);
  static_for([&](auto I) {
    constexpr int i = decltype(I)::value + 1;
    if (i < nk) issue_a(std::integral_constant<int, i>{}, i);
  }, std::make_index_sequence<S - 1>{});
  if (S - 1 < nk) wait_vmcnt<BRI + (S - 1) * AI>();  // step 0's weights and x have landed
  else wait_vmcnt<0>();
  wait_lgkmcnt0();
  lds_barrier();
  ready_b(Z{});
  read_a(Z{}, 0);
  widen(Z{}, 0);
  // head of step 0: sub-steps 0 .. 2, then step 1's weights and x
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    __builtin_amdgcn_sched_barrier(0);
    read_a(Z{}, s + 1);
    __builtin_amdgcn_sched_barrier(0);
    mfma(s);
    __builtin_amdgcn_sched_barrier(0);
    widen(Z{}, s + 1);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (S - 1 < nk) wait_vmcnt<(S - 2) * AI>();
  else wait_vmcnt<0>();
  wait_lgkmcnt0();
  lds_barrier();
  ready_b(O{});
  __builtin_amdgcn_sched_barrier(0);

  int t0 = 0;
  // main loop: tails t0 .. t0 + U - 1 and heads t0 + 1 .. t0 + U, every load full
  for (; t0 + U + S - 1 < kfull; t0 += U) {
    static_for([&](auto I) {
      tail(I, No{}, t0 + decltype(I)::value);
      head(std::integral_constant<int, decltype(I)::value + 1>{}, No{}, t0 + decltype(I)::value + 1);
    }, std::make_index_sequence<U>{});
  }
  for (; t0 < nk; t0 += U) {
    static_for([&](auto I) {
      constexpr int i = decltype(I)::value;
      if (t0 + i < nk) {
        tail(I, Yes{}, t0 + i);
        if (t0 + i + 1 < nk) head(std::integral_constant<int, i + 1>{}, Yes{}, t0 + i + 1);
      }
    }, std::make_index_sequence<U>{});
  }
  wait_vmcnt<0>();

  // epilogue (EPI_W8): lane l, register r -> x row l % 32, column (r & 3) + 4 (l / 32) + 8 (r / 4)
  const bool vec_out = (p.os & 3) == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = wn * FN * 32 + 32 * j + 4 * static_cast<int>(h) + 8 * g;
      if (nl >= nrows_b) continue;
      const int n = n0 + nl;
      const bool full4 = nl + 4 <= nrows_b;
      float sc[4] = {1.f, 1.f, 1.f, 1.f}, bz[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (nl + e < nrows_b) {
          sc[e] = load_dyn(p.scale, n + e, p.sdt);
          if (p.bdt >= 0) bz[e] = load_dyn(p.bias, n + e, p.bdt);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = wm * FM * 32 + 32 * i + static_cast<int>(lrow);
        if (ml >= nrows_x) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = p.bdt >= 0 ? __builtin_fmaf(acc[i][j][4 * g + e], sc[e], bz[e]) : acc[i][j][4 * g + e] * sc[e];
        const int64_t o = static_cast<int64_t>(m0 + ml) * p.os + n;
        if (full4 && vec_out) {
          f32x2 lo = {v[0], v[1]}, hi = {v[2], v[3]};
          *reinterpret_cast<u32x2*>(static_cast<typename TO::bits*>(p.out) + o) = u32x2{narrow2<TO>(lo), narrow2<TO>(hi)};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (nl + e < nrows_b) store_elem<TO>(p.out, o + e, v[e]);
          }
        }
      }
    }
  }
}

// One configuration, either kernel: breg 0 = the library's tiled_gemm, 1 = the above.
template <int FM, int S, int WPE>
int launch_cfg(const Params& base, int breg, hipStream_t s) {
  constexpr int WGM = 2, WGN = 4, FN = 1, BM = 32 * FM * WGM, BN = 32 * FN * WGN;
  Params tp = base;
  tp.tiles_m = (tp.rows + BM - 1) / BM;
  tp.tiles_n = (tp.n + BN - 1) / BN;
  tp.group_m = tp.tiles_m < 4 ? tp.tiles_m : 4;
  const int64_t ntiles = static_cast<int64_t>(tp.tiles_m) * tp.tiles_n;
  const bool xr = ntiles % 8 != 0;
  const void* kern;
  if (breg) {
    kern = xr ? reinterpret_cast<const void*>(tiled_w8_breg<F16, F16, WGM, WGN, FM, FN, S, WPE, 1>)
              : reinterpret_cast<const void*>(tiled_w8_breg<F16, F16, WGM, WGN, FM, FN, S, WPE, 0>);
  } else {
    kern = xr ? reinterpret_cast<const void*>(tiled_gemm<F16, B_I8, F16, WGM, WGN, FM, FN, EPI_W8, S, 1, WPE, 1>)
              : reinterpret_cast<const void*>(tiled_gemm<F16, B_I8, F16, WGM, WGN, FM, FN, EPI_W8, S, 1, WPE, 0>);
  }
  void* args[] = {&tp};
  return hipLaunchKernel(kern, dim3(static_cast<unsigned>(ntiles)), dim3(64 * WGM * WGN), args, 0, s) == hipSuccess
             ? 0
             : -3;
}

}  // namespace
}  // namespace tiled
}  // namespace mi355

// out [rows, n] fp16 = (x [rows, k] fp16 @ q [n, k]^T int8) * scale [n] fp32, by
// the W8A16 tiled GEMM at configuration cfg (0: 128 x 128 tiles of 8 waves,
// 3-stage ring; 1: 192 x 128 tiles of 8 waves, 2-stage ring, registers
// capped for 4 waves per SIMD; 2: 128 x 128, 4-stage ring), with its weights
// through LDS (breg 0, the library's kernel) or loaded into registers
// (breg 1).  k >= 128 and a multiple of 16, rows and n >= 1, contiguous rows, 16-byte
// aligned pointers.  Returns 0, -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_w8_tiled(const void* x, const void* q,
                                                                         const void* scale, void* out, int rows,
                                                                         int k, int n, int cfg, int breg,
                                                                         void* stream) {
  using namespace mi355::tiled;
  if (!x || !q || !scale || !out || rows < 1 || n < 1 || k < 128 || (k & 15) || cfg < 0 || cfg > 2 ||
      (breg != 0 && breg != 1) || int64_t{256} * k * 2 >= (int64_t{1} << 31))
    return -1;
  Params tp{};
  tp.x = x;
  tp.b0 = q;
  tp.b1 = q;
  tp.scale = scale;
  tp.scale1 = scale;
  tp.bias = nullptr;
  tp.out = out;
  tp.rows = rows;
  tp.k = k;
  tp.n = n;
  tp.xs = k;
  tp.bs = k;
  tp.os = n;
  tp.sdt = MI355_F32;
  tp.bdt = -1;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (cfg == 0) return launch_cfg<2, 3, 0>(tp, breg, s);
  if (cfg == 1) return launch_cfg<3, 2, 4>(tp, breg, s);
  return launch_cfg<2, 4, 0>(tp, breg, s);
}
