// LDS-tiled MFMA GEMM core for gfx950, shared by the prefill-size launchers of
// the W8A16 linear (w8a16.hip), of the gate/up projections fused with
// SiLU-and-mul (gate_up_silu.hip) and of the 16-bit linear (linear16.hip):
//
//   acc[m, n] = sum_k x[m, k] * b[n, k]        (both operands K-contiguous)
//   EPI_W8    out[m, n] = round(acc * scale[n] + bias[n])     b = int8 weights
//   EPI_LINEAR   out[m, n] = round(acc + bias[n])             b of x's 16-bit type
//   EPI_SILU  out[m, n] = round(silu(acc_gate) * acc_up)      two 16-bit b
//   EPI_SILU_W8  out[m, n] = round(silu(acc_gate * scale[n]) * (acc_up * scale1[n]))   two int8 b
//
// x is [rows, xs] fp16/bf16 and every b is nn.Linear's [n, bs] layout (int8 or
// x's 16-bit type), used in place.  Arithmetic: 16-bit products, fp32
// accumulation (v_mfma_f32_32x32x16_{f16,bf16}), fp32 epilogue, one rounding.
//
// Decomposition.  A workgroup of WGM x WGN waves owns a BM x BN output tile
// (BM = 32 FM WGM, BN = 32 FN WGN); each wave owns FM x FN 32x32 MFMA tiles
// (of each B matrix).  K advances in steps of 64 columns through a ring of S
// LDS stages filled by gfx950's global -> LDS DMA (buffer_load_dwordx4 ...
// lds, 16 bytes per lane, no VGPR staging): step t + S - 1 is in flight while
// step t computes.  Buffer descriptors end at the last valid element (rows
// past the matrix read 0); the K step enters through the scalar offset, and
// only a final partial step redirects columns at or past k past the
// descriptor, so any k that is a multiple of 16 (int8) or 8 (16-bit) works.
//
// Two main loops.  The step pipeline (RING = 0, S >= 3): per step a wave
// waits for its own DMA of the next step (vmcnt, the later steps stay in
// flight), meets the other waves at one barrier, then alternates the MFMAs
// of this step's sub-steps, whose operands it read one step earlier, with
// the LDS reads of the next step's, so LDS latency hides behind the MFMAs.
// The sub-step ring (RING = 1, S = 2 allowed) reads one 16-column sub-step
// ahead instead of one step, so a wave holds two sub-steps of operands
// rather than two steps and, e.g., a 128 x 32 wave tile of two 16-bit B
// matrices fits in the register file next to its 128 accumulators; its
// barrier sits before the last sub-step's MFMAs.  Both loops are unrolled so
// stage and register-set indices are compile-time constants and have no
// branches (a guarded copy runs the last steps), which keeps the compiler's
// own wait-count tracking exact; sched_barriers keep each group of reads
// and MFMAs in place.  The DMA is inline asm so the compiler neither tracks
// its LDS writes nor drains every load in flight before an LDS read; the
// kernel orders them itself.
//
// K order inside a step.  The MFMA operands give lane l row l % 32 and 8
// consecutive k of k-group h = l / 32.  A step's 64 columns are dealt so that
// k-group h of sub-step s (s < 4) holds columns 32 h + 8 s .. + 8: a lane's
// 16-bit piece of sub-step s is chunk 4 h + s of its 128-byte row, and an
// int8 row's 16-byte chunk 2 h + j feeds sub-steps 2 j and 2 j + 1.  Both
// operands use the same order, so the sum is unchanged (fp32 order aside).
//
// LDS layout.  16-bit tiles: 128-byte rows, chunk c of row r stored at chunk
// c ^ f(r), f(r) = (r ^ (r >> 3)) & 7.  int8 tiles: 64-byte rows, chunk c at
// c ^ g(r), g(r) = ((r >> 1) ^ (r >> 3)) & 3.  The 16-byte reads of 8 (or 16)
// consecutive rows at one logical chunk then fall in distinct banks for 128-
// and 256-byte bank rows (measured: no bank conflicts on the 16-bit tiles).
// A DMA instruction fills 1 KiB of consecutive LDS, so lane l loads the
// logical chunk that the swizzle keeps at its physical slot.
//
// int8 weights (B_I8) stay int8 in LDS -- half the footprint, half the LDS
// traffic -- and are widened in registers after each read: 0x64uu is the
// fp16 pattern of 1024 + u, so (q ^ 0x80) spliced under 0x64 minus 1152 is q
// (v_perm_b32 + v_pk_add_f16 per pair); bf16 goes through v_cvt_f32_i32.
// Every int8 is exact in both 16-bit types.  (Widening once per workgroup
// on a register path into a 16-bit LDS tile measured slower: those loads are
// visible to the compiler, whose waits for them drain the DMA pipeline.)
//
// Epilogue.  The MFMAs take b as their first operand, so each lane ends with
// four consecutive output columns of one row per register group: 8-byte
// stores (16 for fp32 out).
//
// Grid: one workgroup per tile, 1-D.  Consecutive workgroup ids land on
// different XCDs (round robin over 8), so ids are remapped to give each XCD
// a contiguous range of tiles, ordered in groups of group_m m-blocks, m
// fastest: the x row blocks that share a weight block run on one XCD (tile
// counts that are not a multiple of 8: see XR below).
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"

namespace mi355 {
namespace tiled {

typedef float f32x16 __attribute__((ext_vector_type(16)));

enum { EPI_W8 = 0, EPI_SILU = 1, EPI_SILU_W8 = 2, EPI_LINEAR = 3 };

enum { B_16 = 0, B_I8 = 1 };

template <typename T> __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <> __device__ __forceinline__ f32x16 mfma32<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}
template <> __device__ __forceinline__ f32x16 mfma32<BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// 8 int8 in two dwords -> one MFMA operand (8 values of T).
template <typename T> __device__ __forceinline__ u32x4 widen8(uint32_t d0, uint32_t d1) {
  const u32x2 p = widen_i8x4<T>(d0), q = widen_i8x4<T>(d1);
  return u32x4{p.x, p.y, q.x, q.y};
}

__device__ __forceinline__ uint32_t swz16(uint32_t r, uint32_t c) { return r * 128u + ((c ^ ((r ^ (r >> 3)) & 7u)) << 4); }
__device__ __forceinline__ uint32_t swz8(uint32_t r, uint32_t c) {
  return r * 64u + ((c ^ (((r >> 1) ^ (r >> 3)) & 3u)) << 4);
}

__device__ __forceinline__ u32x4 lds_read16(const uint8_t* base, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}

struct Params {
  const void* x;      // [rows, xs] of T
  const void* b0;     // [n, bs]: int8 weights (EPI_W8) or w_gate (EPI_SILU)
  const void* b1;     // [n, bs]: w_up (EPI_SILU), else unused
  const void* scale;   // [n] of sdt (EPI_W8; gate scale for EPI_SILU_W8)
  const void* bias;    // [n] of bdt, or null (EPI_W8, EPI_LINEAR)
  const void* scale1;  // [n] of sdt: up scale (EPI_SILU_W8)
  void* out;          // [rows, os] of TO
  int rows, k, n;
  int64_t xs, bs, os;  // row strides in elements
  int sdt, bdt;        // dtype codes of scale and bias (bdt < 0: no bias)
  int tiles_m, tiles_n;
  int group_m;  // m-blocks per group of the tile order (tiles_m: m fastest over the whole range)
};

template <typename T, int BK, typename TO, int WGM, int WGN, int FM, int FN, int EPI, int S>
struct Cfg {
  // BK: B's storage -- B_16 (x's 16-bit type) or B_I8 (int8, kept int8 in
  // LDS and widened after each LDS read).
  static constexpr bool I8 = BK == B_I8;
  static constexpr int NW = WGM * WGN, NT = 64 * NW;
  static constexpr int BLOCK = NT;  // threads per workgroup
  static constexpr int BM = 32 * FM * WGM, BN = 32 * FN * WGN;
  static constexpr int NB = (EPI == EPI_W8 || EPI == EPI_LINEAR) ? 1 : 2;  // B matrices
  static constexpr int A_BYTES = BM * 128;             // 64 columns of 16-bit x per row
  static constexpr int B_ROW = I8 ? 64 : 128;          // bytes per B row per step in LDS
  static constexpr int B_BYTES = BN * B_ROW;
  static constexpr int STAGE = A_BYTES + NB * B_BYTES;
  static constexpr int LDS = S * STAGE;
  // One DMA instruction moves 64 lanes x 16 bytes = 1 KiB: 8 rows of a 16-bit
  // tile, 16 rows of an int8 tile.
  static constexpr int AI = A_BYTES / 1024 / NW;  // A DMA instructions per wave per step
  static constexpr int BI = B_BYTES / 1024 / NW;  // B DMA instructions per wave per step and matrix
  static constexpr int P = AI + NB * BI;          // DMA instructions per wave per step
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "tile must split over the waves");
  static_assert(S >= 2 && S <= 8, "2..8 stages");
  static_assert(P * (S - 1) < 64, "vmcnt range");
};

// Stage I of the LDS ring (one LDS variable per stage).
template <int I, int SZ> __device__ __forceinline__ uint8_t* stage_ptr() {
  __shared__ __attribute__((aligned(1024))) uint8_t st[SZ];
  return st;
}

typedef __attribute__((address_space(3))) uint8_t* lds_ptr_t;

// f(integral_constant<int, I>) for I = 0 .. N - 1, unrolled at compile time.
template <typename F, size_t... I>
__device__ __forceinline__ void static_for(F&& f, std::index_sequence<I...>) {
  (f(std::integral_constant<int, static_cast<int>(I)>{}), ...);
}

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }
constexpr int lcm_c(int a, int b) { return a / gcd_c(a, b) * b; }

// Global -> LDS DMA of 16 bytes per lane (gfx950 buffer_load_dwordx4 ... lds):
// lane l's bytes land at LDS address m0 + 16 l; the global address is the
// descriptor base + voff + soff.  Written as asm so that the compiler neither
// tracks these LDS writes nor drains every load in flight before each LDS
// read: the kernel orders them itself, with vmcnt waits before the barrier
// that publishes a stage (vmcnt falls as the data reaches LDS, in issue order).
// No non-temporal hint: on x, on the weights and on both it measured slower
// on MI355X at every prefill shape of the gate/up, W8A16 and 16-bit-linear
// launchers (1.01x - 1.69x the time), the re-reads of both operands by
// neighbouring tiles being L2 hits worth keeping.
__device__ __forceinline__ void dma16(rsrc_t r, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0) : "memory");
}

// LDS byte address of stage I (the cast of the LDS variable itself folds to a constant).
template <int I, int SZ> __device__ __forceinline__ uint32_t stage_addr() {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)stage_ptr<I, SZ>()));
}

// Workgroup barrier that the compiler may not move memory accesses across.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt low
// bits [3:0], high bits [15:14]; expcnt [6:4] = 7, lgkmcnt [11:8] = 15).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// The occupancy one configuration is compiled for: its own WPE waves per SIMD
// when WPE > 0, else 1 (no register cap).
template <int WPE>
constexpr int kMinWavesPerSimd = WPE > 0 ? WPE : 1;

// WPE > 0 caps the registers of this configuration alone so that WPE waves fit
// on each SIMD (a 192 x 128 tile of 8 waves at WPE = 4 fits in 128 VGPRs and
// runs two workgroups per CU).  XR = 1 gives the XCDs contiguous tile ranges
// when the tile count is not a multiple of 8 too (the first count mod 8 XCDs,
// which receive one workgroup more, take ranges one tile longer); XR = 0
// keeps the dispatch order for such counts.  (XR is a template argument so
// that the configurations without it keep their code.)  The int8 B operand
// is widened one sub-step ahead, into a second register set, after the
// previous sub-step's MFMAs are issued, so the widening VALU work runs beside
// the MFMAs instead of in front of them.
template <typename T, int BK, typename TO, int WGM, int WGN, int FM, int FN, int EPI, int S, int RING = 0, int WPE = 0,
          int XR = 0>
__global__ __launch_bounds__(64 * WGM * WGN)
__attribute__((amdgpu_waves_per_eu(kMinWavesPerSimd<WPE>))) void tiled_gemm(const Params p) {
  using C = Cfg<T, BK, TO, WGM, WGN, FM, FN, EPI, S>;
  constexpr bool I8 = C::I8;
  using TB = typename T::bits;
  constexpr int NW = C::NW, BM = C::BM, BN = C::BN, NB = C::NB;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  // Tile of this workgroup: contiguous ranges per XCD, m fastest.
  const int ntiles = p.tiles_m * p.tiles_n;
  int b = blockIdx.x;
  if constexpr (XR != 0) {
    // XCD x = b % 8 runs ids x, x + 8, ...: ceil((ntiles - x) / 8) of them
    const int q = ntiles >> 3, r = ntiles & 7, x = b & 7;
    b = x * q + (x < r ? x : r) + (b >> 3);
  } else {
    if ((ntiles & 7) == 0) b = (b & 7) * (ntiles >> 3) + (b >> 3);
  }
  // inside the range: groups of group_m m-blocks, m fastest within a group
  const int per_group = p.group_m * p.tiles_n;
  const int g0 = (b / per_group) * p.group_m;
  const int gsz = p.tiles_m - g0 < p.group_m ? p.tiles_m - g0 : p.group_m;
  const int tm = g0 + (b % per_group) % gsz, tn = (b % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nrows_x = p.rows - m0 < BM ? p.rows - m0 : BM;
  const int nrows_b = p.n - n0 < BN ? p.n - n0 : BN;

  constexpr int EB = I8 ? 1 : static_cast<int>(sizeof(TB));  // bytes per B element in memory
  const rsrc_t rx = make_rsrc(static_cast<const TB*>(p.x) + static_cast<int64_t>(m0) * p.xs,
                              static_cast<uint32_t>(((nrows_x - 1) * p.xs + p.k) * sizeof(TB)));
  rsrc_t rb[NB];
  rb[0] = make_rsrc(static_cast<const uint8_t*>(p.b0) + static_cast<int64_t>(n0) * p.bs * EB,
                    static_cast<uint32_t>(((nrows_b - 1) * p.bs + p.k) * EB));
  if constexpr (NB == 2)
    rb[1] = make_rsrc(static_cast<const uint8_t*>(p.b1) + static_cast<int64_t>(n0) * p.bs * EB,
                      static_cast<uint32_t>(((nrows_b - 1) * p.bs + p.k) * EB));

  const int nk = (p.k + 63) >> 6;
  // DMA lane maps (16-bit tiles).  Instruction j of wave w fills the 1 KiB
  // at tile offset 1024 (NW j + w): lane l writes physical chunk l % 8 of row
  // 8 (NW j + w) + l / 8, so it loads the logical chunk the swizzle keeps
  // there.  The K step enters through the scalar offset.
  uint32_t a_goff[C::AI];
  int a_col[C::AI];
#pragma unroll
  for (int j = 0; j < C::AI; ++j) {
    const int r = 8 * (NW * j + wave) + (lane >> 3);
    const int c = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
    a_goff[j] = static_cast<uint32_t>((r * p.xs + 8 * c) * sizeof(TB));
    a_col[j] = 8 * c;
  }
  uint32_t b_goff[C::BI];
  int b_col[C::BI];
#pragma unroll
  for (int j = 0; j < C::BI; ++j) {
    if constexpr (I8) {  // 16 rows of 64 bytes per instruction
      const int r = 16 * (NW * j + wave) + (lane >> 2);
      const int c = (lane & 3) ^ (((r >> 1) ^ (r >> 3)) & 3);
      b_goff[j] = static_cast<uint32_t>(r * p.bs + 16 * c);
      b_col[j] = 16 * c;
    } else {
      const int r = 8 * (NW * j + wave) + (lane >> 3);
      const int c = (lane & 7) ^ ((r ^ (r >> 3)) & 7);
      b_goff[j] = static_cast<uint32_t>((r * p.bs + 8 * c) * EB);
      b_col[j] = 8 * c;
    }
  }
  const int kfull = p.k >> 6;  // steps whose 64 columns are all inside k

  // Issues the DMA of K step kt into stage I.  Columns at or past k read 0.
  auto issue = [&](auto I, int kt) {
    const uint32_t st = stage_addr<decltype(I)::value, C::STAGE>();
    const bool full = kt < kfull;  // known true in the main loop (the compiler folds it)
#pragma unroll
    for (int j = 0; j < C::AI; ++j) {
      const uint32_t kb = static_cast<uint32_t>(kt * 64 * sizeof(TB));
      const uint32_t dst = st + 1024u * (NW * j + wave);
      if (full) dma16(rx, a_goff[j], kb, dst);
      else dma16(rx, kt * 64 + a_col[j] < p.k ? a_goff[j] + kb : kOob, 0, dst);
    }
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
      for (int j = 0; j < C::BI; ++j) {
        const uint32_t kb = static_cast<uint32_t>(kt * 64 * EB);
        const uint32_t dst = st + C::A_BYTES + bi * C::B_BYTES + 1024u * (NW * j + wave);
        if (full) dma16(rb[bi], b_goff[j], kb, dst);
        else dma16(rb[bi], kt * 64 + b_col[j] < p.k ? b_goff[j] + kb : kOob, 0, dst);
      }
    }
  };

  f32x16 acc[NB][FM][FN];
#pragma unroll
  for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[bi][i][j][r] = 0.f;
      }
    }
  }

  // Operand rows of this lane inside a stage.
  const uint32_t lrow = lane & 31, h = lane >> 5;
  const uint32_t arow0 = wm * FM * 32 + lrow;
  const uint32_t brow0 = wn * FN * 32 + lrow;

  // A step's operands in registers: A pieces of the 4 sub-steps; B pieces
  // per sub-step (16-bit in LDS) or per pair of sub-steps (int8 in LDS: chunk
  // 2h + q of the row, whose first 8 bytes feed sub-step 2q, the rest 2q + 1).
  constexpr int BQ = I8 ? 2 : 4;
  struct Frags {
    u32x4 a[4][FM];
    u32x4 b[NB][BQ][FN];
  };
  // LDS reads of sub-step s of one step (stage I) into f.
  auto read_sub = [&](auto I, Frags& f, int s) {
    const uint8_t* abase = stage_ptr<decltype(I)::value, C::STAGE>();
#pragma unroll
    for (int i = 0; i < FM; ++i) f.a[s][i] = lds_read16(abase, swz16(arow0 + 32 * i, 4 * h + s));
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (I8) {
          if (s < BQ) f.b[bi][s][j] = lds_read16(abase + C::A_BYTES + bi * C::B_BYTES, swz8(brow0 + 32 * j, 2 * h + s));
        } else {
          f.b[bi][s][j] = lds_read16(abase + C::A_BYTES + bi * C::B_BYTES, swz16(brow0 + 32 * j, 4 * h + s));
        }
      }
    }
  };
  auto read_frags = [&](auto I, Frags& f) {
#pragma unroll
    for (int s = 0; s < 4; ++s) read_sub(I, f, s);
  };
  // MFMAs of sub-step s from f.
  auto mfma_sub = [&](const Frags& f, int s) {
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
      u32x4 bf[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (I8) {
          const u32x4 raw = f.b[bi][s >> 1][j];
          bf[j] = (s & 1) ? widen8<T>(raw.z, raw.w) : widen8<T>(raw.x, raw.y);
        } else {
          bf[j] = f.b[bi][s][j];
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[bi][i][j] = mfma32<T>(bf[j], f.a[s][i], acc[bi][i][j]);
      }
    }
  };

  // Widen-ahead (int8 B): wb[s & 1] holds sub-step s's B operands, widened
  // from the raw int8 pair read (16 bytes: sub-steps 2q, 2q + 1) during the
  // previous sub-step, behind that sub-step's MFMAs.
  constexpr bool WA = I8;
  u32x4 wb[2][NB][FN];
  auto widen_into = [&](const u32x4 (&raw)[NB][FN], int s, u32x4 (&out)[NB][FN]) {
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        out[bi][j] = (s & 1) ? widen8<T>(raw[bi][j].z, raw[bi][j].w) : widen8<T>(raw[bi][j].x, raw[bi][j].y);
    }
  };
  auto mfma_wide = [&](const u32x4 (&a)[FM], const u32x4 (&bw)[NB][FN]) {
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[bi][i][j] = mfma32<T>(bw[bi][j], a[i], acc[bi][i][j]);
      }
    }
  };

  int t0 = 0;
  if constexpr (!RING) {
    // Step pipeline.  Step t computes from registers read out of stage t % S
    // one step earlier.  In step t a wave refills stage (t - 1) % S, which
    // every wave finished reading before the previous barrier, with step
    // t + S - 1; waits for its own DMA of step t + 1 (the later steps stay in
    // flight) and for its LDS reads of step t; meets the other waves at the
    // barrier -- all of step t + 1 is now in LDS -- and then, sub-step by
    // sub-step, runs the MFMAs of step t's sub-step s and issues the LDS reads
    // of step t + 1's sub-step s, so a wave's MFMAs never queue behind all of
    // its LDS reads (2-3% over all reads first).
    static_assert(S >= 3, "the step pipeline needs 3 stages");
    Frags fr[2];
    // raw int8 pair q of a step's fragments as one [NB][FN] set
    auto raw_pair = [&](const Frags& f, int q, u32x4 (&out)[NB][FN]) {
#pragma unroll
      for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
        for (int j = 0; j < FN; ++j) out[bi][j] = f.b[bi][q][j];
      }
    };
    auto widen_step_sub = [&](const Frags& f, int s, u32x4 (&out)[NB][FN]) {
      u32x4 raw[NB][FN];
      raw_pair(f, (s >> 1) & (BQ - 1), raw);
      widen_into(raw, s, out);
    };
    static_for([&](auto I) {
      if (decltype(I)::value < nk) issue(I, decltype(I)::value);
    }, std::make_index_sequence<S - 1>{});
    if (S - 2 < nk) wait_vmcnt<(S - 2) * C::P>();
    else wait_vmcnt<0>();
    wait_lgkmcnt0();
    lds_barrier();
    read_frags(std::integral_constant<int, 0>{}, fr[0]);
    if constexpr (WA) widen_step_sub(fr[0], 0, wb[0]);

    constexpr int UNROLL = lcm_c(S, 2);  // stage and fragment-set indices known at compile time
    // One step; GUARD = false where every condition is known to hold (all
    // steps it touches are full 64-column steps inside k), so the main loop
    // has no branches and the compiler's own wait-count tracking stays exact.
    auto step = [&](auto I, auto GUARD, int t) {
      constexpr int ii = decltype(I)::value, si = ii % S, pi = ii % 2;
      constexpr bool guard = decltype(GUARD)::value;
      if (!guard || t + S - 1 < nk) issue(std::integral_constant<int, (si + S - 1) % S>{}, t + S - 1);
      const bool more = !guard || t + 1 < nk;
      if (more) {
        if (!guard || t + S - 1 < nk) wait_vmcnt<(S - 2) * C::P>();
        else wait_vmcnt<0>();
        wait_lgkmcnt0();
        lds_barrier();
      }
      // sched_barriers keep each group in place
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (WA) mfma_wide(fr[pi].a[s], wb[s & 1]);
        else mfma_sub(fr[pi], s);
        __builtin_amdgcn_sched_barrier(0);
        if (more) read_sub(std::integral_constant<int, (si + 1) % S>{}, fr[pi ^ 1], s);
        if constexpr (WA) {
          // the next sub-step's weights: this step's (already in registers)
          // or, after the last sub-step, the next step's pair 0 (read in
          // this step's first group)
          __builtin_amdgcn_sched_barrier(0);
          if (s < 3) widen_step_sub(fr[pi], s + 1, wb[(s + 1) & 1]);
          else if (more) widen_step_sub(fr[pi ^ 1], 0, wb[0]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // main loop: steps t0 .. t0 + UNROLL - 1 issue steps up to t0 + UNROLL + S - 2 < kfull
    for (; t0 + UNROLL + S - 2 < kfull; t0 += UNROLL) {
      static_for([&](auto I) { step(I, std::false_type{}, t0 + decltype(I)::value); },
                 std::make_index_sequence<UNROLL>{});
    }
    for (; t0 < nk; t0 += UNROLL) {
      static_for([&](auto I) {
        if (t0 + decltype(I)::value < nk) step(I, std::true_type{}, t0 + decltype(I)::value);
      }, std::make_index_sequence<UNROLL>{});
    }
  } else {
    // Sub-step ring (RING = 1): the LDS reads run one 16-column sub-step
    // ahead of the MFMAs instead of one step, so a wave holds two sub-steps
    // of operands (not two steps) and large wave tiles fit in the register
    // file.  Sub-step s of step t is read while sub-step s - 1 computes;
    // before the MFMAs of sub-step 3 a wave waits for its DMA of step t + 1
    // and its reads of step t, meets the others at the barrier, refills
    // stage t % S (now unread) with step t + S and reads sub-step 0 of step
    // t + 1.  A pieces alternate between two register sets by sub-step; an
    // int8 B read (16 bytes: sub-steps 2q and 2q + 1 of k-group h) is made
    // with sub-step q's A read into set q, so a read never lands in a set
    // that a pending MFMA (or widening) still reads.
    struct Sub {
      u32x4 a[2][FM];
      u32x4 b[2][NB][FN];
    };
    auto read_one = [&](auto I, Sub& f, int s) {
      const uint8_t* abase = stage_ptr<decltype(I)::value, C::STAGE>();
#pragma unroll
      for (int i = 0; i < FM; ++i) f.a[s & 1][i] = lds_read16(abase, swz16(arow0 + 32 * i, 4 * h + s));
#pragma unroll
      for (int bi = 0; bi < NB; ++bi) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const uint8_t* bbase = abase + C::A_BYTES + bi * C::B_BYTES;
          if constexpr (I8) {
            // raw pair q (sub-steps 2q, 2q + 1) read with sub-step q's A, a
            // sub-step or more before its first use: set q was last read
            // two sub-steps earlier
            if (s < 2) f.b[s][bi][j] = lds_read16(bbase, swz8(brow0 + 32 * j, 2 * h + s));
          } else {
            f.b[s & 1][bi][j] = lds_read16(bbase, swz16(brow0 + 32 * j, 4 * h + s));
          }
        }
      }
    };
    auto mfma_one = [&](const Sub& f, int s) {
#pragma unroll
      for (int bi = 0; bi < NB; ++bi) {
        u32x4 bf[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if constexpr (I8) {
            const u32x4 raw = f.b[(s >> 1) & 1][bi][j];
            bf[j] = (s & 1) ? widen8<T>(raw.z, raw.w) : widen8<T>(raw.x, raw.y);
          } else {
            bf[j] = f.b[s & 1][bi][j];
          }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[bi][i][j] = mfma32<T>(bf[j], f.a[s & 1][i], acc[bi][i][j]);
        }
      }
    };
    Sub rf;
    static_for([&](auto I) {
      if (decltype(I)::value < nk) issue(I, decltype(I)::value);
    }, std::make_index_sequence<S>{});
    if (S - 1 < nk) wait_vmcnt<(S - 1) * C::P>();
    else wait_vmcnt<0>();
    wait_lgkmcnt0();
    lds_barrier();
    read_one(std::integral_constant<int, 0>{}, rf, 0);
    if constexpr (WA) widen_into(rf.b[0], 0, wb[0]);
    auto rstep = [&](auto I, auto GUARD, int t) {
      constexpr int si = decltype(I)::value % S;
      constexpr bool guard = decltype(GUARD)::value;
      const bool more = !guard || t + 1 < nk;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        __builtin_amdgcn_sched_barrier(0);
        if (s < 3) {
          read_one(std::integral_constant<int, si>{}, rf, s + 1);
        } else if (more) {
          if (!guard || t + S - 1 < nk) wait_vmcnt<(S - 2) * C::P>();
          else wait_vmcnt<0>();
          wait_lgkmcnt0();
          lds_barrier();
          if (!guard || t + S < nk) issue(std::integral_constant<int, si>{}, t + S);
          read_one(std::integral_constant<int, (si + 1) % S>{}, rf, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (WA) {
          mfma_wide(rf.a[s & 1], wb[s & 1]);
          // the next sub-step's weights, from the raw pair read at sub-step
          // 2q (the wait for a pair read in this group lands here, behind
          // the MFMAs just issued)
          __builtin_amdgcn_sched_barrier(0);
          if (s < 3) widen_into(rf.b[((s + 1) >> 1) & 1], s + 1, wb[(s + 1) & 1]);
          else if (more) widen_into(rf.b[0], 0, wb[0]);
        } else {
          mfma_one(rf, s);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // main loop: steps t0 .. t0 + S - 1 issue steps up to t0 + 2 S - 1 < kfull
    for (; t0 + 2 * S - 1 < kfull; t0 += S) {
      static_for([&](auto I) { rstep(I, std::false_type{}, t0 + decltype(I)::value); }, std::make_index_sequence<S>{});
    }
    for (; t0 < nk; t0 += S) {
      static_for([&](auto I) {
        if (t0 + decltype(I)::value < nk) rstep(I, std::true_type{}, t0 + decltype(I)::value);
      }, std::make_index_sequence<S>{});
    }
  }

  // Epilogue.  The MFMAs take the weights as their first operand, so D of a
  // 32x32 tile is transposed: lane l, register r -> x row l % 32, output
  // column (r & 3) + 4 (l / 32) + 8 (r / 4).  Registers 4g .. 4g + 3 are four
  // consecutive columns of one row: one 8-byte store (16 bytes for fp32).
  const bool vec_out = (p.os & 3) == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = wn * FN * 32 + 32 * j + 4 * static_cast<int>(h) + 8 * g;  // first of 4 columns
      if (nl >= nrows_b) continue;
      const int n = n0 + nl;
      const bool full4 = nl + 4 <= nrows_b;
      float sc[4] = {1.f, 1.f, 1.f, 1.f}, bz[4] = {0.f, 0.f, 0.f, 0.f};  // EPI_SILU_W8: bz = up scale
      if constexpr (EPI == EPI_LINEAR) {
        if (p.bdt >= 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (nl + e < nrows_b) bz[e] = load_dyn(p.bias, n + e, p.bdt);
          }
        }
      } else if constexpr (EPI != EPI_SILU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (nl + e < nrows_b) {
            sc[e] = load_dyn(p.scale, n + e, p.sdt);
            if constexpr (EPI == EPI_W8) {
              if (p.bdt >= 0) bz[e] = load_dyn(p.bias, n + e, p.bdt);
            } else {
              bz[e] = load_dyn(p.scale1, n + e, p.sdt);
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = wm * FM * 32 + 32 * i + static_cast<int>(lrow);
        if (ml >= nrows_x) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (EPI == EPI_W8) {
            v[e] = p.bdt >= 0 ? __builtin_fmaf(acc[0][i][j][4 * g + e], sc[e], bz[e]) : acc[0][i][j][4 * g + e] * sc[e];
          } else if constexpr (EPI == EPI_LINEAR) {
            v[e] = p.bdt >= 0 ? acc[0][i][j][4 * g + e] + bz[e] : acc[0][i][j][4 * g + e];
          } else if constexpr (EPI == EPI_SILU) {
            v[e] = silu_mul_f32(acc[0][i][j][4 * g + e], acc[NB - 1][i][j][4 * g + e]);
          } else {
            v[e] = silu_mul_f32(acc[0][i][j][4 * g + e] * sc[e], acc[NB - 1][i][j][4 * g + e] * bz[e]);
          }
        }
        const int64_t o = static_cast<int64_t>(m0 + ml) * p.os + n;
        if (full4 && vec_out) {
          if constexpr (is_half_width<TO>::value) {
            f32x2 lo = {v[0], v[1]}, hi = {v[2], v[3]};
            *reinterpret_cast<u32x2*>(static_cast<typename TO::bits*>(p.out) + o) = u32x2{narrow2<TO>(lo), narrow2<TO>(hi)};
          } else {
            *reinterpret_cast<u32x4*>(static_cast<float*>(p.out) + o) = u32x4{as_u32(v[0]), as_u32(v[1]), as_u32(v[2]), as_u32(v[3])};
          }
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

}  // namespace tiled
}  // namespace mi355
