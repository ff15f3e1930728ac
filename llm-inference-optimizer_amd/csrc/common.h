// Shared device helpers for the gfx950 fused RMSNorm / SiLU-and-mul kernels:
// 16-byte packet types, fp16/bf16 <-> fp32 conversion through gfx950's packed
// convert instructions, wave64 reductions and the launch status plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi355_fused.h"

namespace mi355 {

// ---------------------------------------------------------------------------
// Packet types.  Every hot load and store moves 16 bytes per lane
// (global_load_dwordx4 / global_store_dwordx4), so a wave64 touches 1 KiB of
// contiguous memory per instruction.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Bit casts through a scalar parameter.  `__builtin_bit_cast(float, v[i])`
// applied directly to an element of an ext_vector_type value reads element 0
// for every i with this hipcc (seen in the gfx950 ISA), so every element is
// copied into a scalar first.
__device__ __forceinline__ float as_f32(uint32_t v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ uint32_t as_u32(float v) { return __builtin_bit_cast(uint32_t, v); }

// Register barrier: an empty asm that claims to modify v, so the compiler
// cannot keep values derived from v (e.g. its fp32 widening) live across it and
// recomputes them from the packed form instead.  Used to keep a row in packed
// 16-bit form between the two passes of RMSNorm, halving its VGPR footprint.
__device__ __forceinline__ void reg_barrier(u32x4& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void reg_barrier(uint32_t& v) { asm volatile("" : "+v"(v)); }

// Value barrier on an fp32 result about to be narrowed to 16 bits: the
// compiler may not fold the operation that produced it into the conversion.
// Without it, a final fp32 multiply followed by the narrowing can become one
// v_fma_mixlo_f16, which rounds the exact product straight to 16 bits; that
// differs from rounding the fp32 result whenever the fp32 rounding lands on a
// tie of the 16-bit grid, so the 16-bit output would not always be the fp32
// output rounded once.  Free at run time (an empty asm).
__device__ __forceinline__ float fp32_value(float v) {
  asm("" : "+v"(v));
  return v;
}
__device__ __forceinline__ f32x2 fp32_value(f32x2 v) {
  asm("" : "+v"(v));
  return v;
}

// Storage tags.  `bits` is the raw storage type; arithmetic is always fp32.
struct F32 { typedef uint32_t bits; static constexpr int code = MI355_F32; };
struct F16 { typedef uint16_t bits; static constexpr int code = MI355_F16; };
struct BF16 { typedef uint16_t bits; static constexpr int code = MI355_BF16; };

template <typename T> struct is_half_width { static constexpr bool value = false; };
template <> struct is_half_width<F16> { static constexpr bool value = true; };
template <> struct is_half_width<BF16> { static constexpr bool value = true; };

// Elements of T in one 16-byte packet.
template <typename T> struct pack_width { static constexpr int value = 16 / sizeof(typename T::bits); };

// ---------------------------------------------------------------------------
// Conversions.  Two 16-bit values share a dword; v_cvt_f32_f16 (with SDWA word
// select) widens fp16, a shift/mask widens bf16, and gfx950's
// v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 narrow two fp32 values with
// round-to-nearest-even in one instruction.
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ f32x2 widen2(uint32_t d);
template <> __device__ __forceinline__ f32x2 widen2<F16>(uint32_t d) {
  return __builtin_convertvector(__builtin_bit_cast(f16x2, d), f32x2);
}
template <> __device__ __forceinline__ f32x2 widen2<BF16>(uint32_t d) {
  f32x2 r;
  r.x = as_f32(d << 16);
  r.y = as_f32(d & 0xffff0000u);
  return r;
}

template <typename T> __device__ __forceinline__ uint32_t narrow2(f32x2 v);
template <> __device__ __forceinline__ uint32_t narrow2<F16>(f32x2 v) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(fp32_value(v), f16x2));
}
template <> __device__ __forceinline__ uint32_t narrow2<BF16>(f32x2 v) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(fp32_value(v), bf16x2));
}

// Scalar element access for the generic (unaligned / odd-size) kernels.
template <typename T> __device__ __forceinline__ float load_elem(const void* p, int64_t i);
template <> __device__ __forceinline__ float load_elem<F32>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float load_elem<F16>(const void* p, int64_t i) {
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}
template <> __device__ __forceinline__ float load_elem<BF16>(const void* p, int64_t i) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
}

template <typename T> __device__ __forceinline__ void store_elem(void* p, int64_t i, float v);
template <> __device__ __forceinline__ void store_elem<F32>(void* p, int64_t i, float v) {
  static_cast<float*>(p)[i] = v;
}
template <> __device__ __forceinline__ void store_elem<F16>(void* p, int64_t i, float v) {
  static_cast<_Float16*>(p)[i] = static_cast<_Float16>(fp32_value(v));
}
template <> __device__ __forceinline__ void store_elem<BF16>(void* p, int64_t i, float v) {
  static_cast<__bf16*>(p)[i] = static_cast<__bf16>(fp32_value(v));
}

// v rounded to T's precision (round-to-nearest-even) and widened back.
template <typename T> __device__ __forceinline__ float quantize(float v);
template <> __device__ __forceinline__ float quantize<F32>(float v) { return v; }
template <> __device__ __forceinline__ float quantize<F16>(float v) {
  return static_cast<float>(static_cast<_Float16>(fp32_value(v)));
}
template <> __device__ __forceinline__ float quantize<BF16>(float v) {
  return static_cast<float>(static_cast<__bf16>(fp32_value(v)));
}

// A packet of `pack_width<T>` elements held as raw dwords.  `unpack` widens it
// to fp32; `pack` rounds fp32 values into the packet once.
template <typename T> struct Packet {
  static constexpr int W = pack_width<T>::value;
  u32x4 raw;
  __device__ __forceinline__ void unpack(float (&f)[W]) const {
    if constexpr (is_half_width<T>::value) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x2 p = widen2<T>(raw[i]);
        f[2 * i] = p.x;
        f[2 * i + 1] = p.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = as_f32(raw[i]);
    }
  }
  __device__ __forceinline__ void pack(const float (&f)[W]) {
    if constexpr (is_half_width<T>::value) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x2 p;
        p.x = f[2 * i];
        p.y = f[2 * i + 1];
        raw[i] = narrow2<T>(p);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) raw[i] = as_u32(f[i]);
    }
  }
};

// W consecutive elements of type T starting at `p` (16-byte aligned when T is
// the packet type; for a wider or narrower weight type the byte count is
// W * sizeof(T::bits) and is loaded with the matching vector width).
template <typename T, int W> struct Chunk;
template <typename T> struct Chunk<T, 8> {  // 8 elements
  static constexpr int DW = 8 * sizeof(typename T::bits) / 4;  // 4 (16-bit) or 8 (fp32)
  uint32_t raw[DW];
  __device__ __forceinline__ void load(const void* p) {
    const u32x4* q = static_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < DW / 4; ++i) {
      u32x4 v = q[i];
      raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (is_half_width<T>::value) {
      f32x2 p = widen2<T>(raw[i >> 1]);
      return (i & 1) ? p.y : p.x;
    } else {
      return as_f32(raw[i]);
    }
  }
};
template <typename T> struct Chunk<T, 4> {  // 4 elements
  static constexpr int DW = 4 * sizeof(typename T::bits) / 4;  // 2 (16-bit) or 4 (fp32)
  uint32_t raw[DW];
  __device__ __forceinline__ void load(const void* p) {
    if constexpr (DW == 4) {
      u32x4 v = *static_cast<const u32x4*>(p);
      raw[0] = v.x; raw[1] = v.y; raw[2] = v.z; raw[3] = v.w;
    } else {
      u32x2 v = *static_cast<const u32x2*>(p);
      raw[0] = v.x; raw[1] = v.y;
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (is_half_width<T>::value) {
      f32x2 p = widen2<T>(raw[i >> 1]);
      return (i & 1) ? p.y : p.x;
    } else {
      return as_f32(raw[i]);
    }
  }
};

// Stores W fp32 values as W elements of TY at p (one 16-byte store for a
// half-width TY with W == 8, two for fp32 with W == 8, one for fp32 with W == 4).
template <typename TY, int W>
__device__ __forceinline__ void store_chunk(void* p, const float (&f)[W]) {
  if constexpr (is_half_width<TY>::value) {
    static_assert(W == 8 || W == 4, "packet width");
    uint32_t d[W / 2];
#pragma unroll
    for (int i = 0; i < W / 2; ++i) {
      f32x2 v;
      v.x = f[2 * i];
      v.y = f[2 * i + 1];
      d[i] = narrow2<TY>(v);
    }
    if constexpr (W == 8) {
      u32x4 o = {d[0], d[1], d[2], d[3]};
      *static_cast<u32x4*>(p) = o;
    } else {
      u32x2 o = {d[0], d[1]};
      *static_cast<u32x2*>(p) = o;
    }
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      u32x4 o = {as_u32(f[4 * i]), as_u32(f[4 * i + 1]), as_u32(f[4 * i + 2]), as_u32(f[4 * i + 3])};
      static_cast<u32x4*>(p)[i] = o;
    }
  }
}

// ---------------------------------------------------------------------------
// Raw buffer access.  A buffer resource (V#) covers [base, base + bytes); a
// load outside it returns zeros and a store outside it is dropped by the
// hardware, so a kernel that builds one descriptor per row or per chunk needs
// no per-lane bounds branches.  Descriptor word 3 0x00020000 selects 32-bit
// data format for gfx9-family untyped access (gfx950 included).  `bytes` is a
// 32-bit count: callers keep each descriptor's extent below 4 GiB.
//
// Cache policy (aux) bits on gfx950: 1 = sc0, 2 = nt, 16 = sc1.  nt (streaming)
// on loads and stores measured fastest for these single-pass kernels.
// ---------------------------------------------------------------------------
constexpr int kStreamAux = 2;  // nt

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kStreamAux);
}
__device__ __forceinline__ u32x4 buf_load16_cached(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 buf_load8_cached(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ void buf_store16(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kStreamAux);
}
__device__ __forceinline__ void buf_store8(rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kStreamAux);
}

// W elements of T at byte offset `off` of buffer r, loaded as raw dwords
// (W * sizeof(T) is 8, 16 or 32 bytes) with the default cache policy: this
// holds data every wave re-reads (the RMSNorm weight), which should stay in L2.
template <typename T, int W> struct BufChunk {
  static constexpr int DW = W * sizeof(typename T::bits) / 4;
  uint32_t raw[DW];
  __device__ __forceinline__ void load(rsrc_t r, uint32_t off) {
    if constexpr (DW == 2) {
      const u32x2 v = buf_load8_cached(r, off);
      raw[0] = v.x; raw[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < DW / 4; ++i) {
        const u32x4 v = buf_load16_cached(r, off + 16u * i);
        raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
      }
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (is_half_width<T>::value) {
      const f32x2 p = widen2<T>(raw[i >> 1]);
      return (i & 1) ? p.y : p.x;
    } else {
      return as_f32(raw[i]);
    }
  }
};

// Stores W fp32 values as W elements of TY at byte offset `off` of buffer r,
// rounding each once.
template <typename TY, int W>
__device__ __forceinline__ void buf_store_chunk(rsrc_t r, uint32_t off, const float (&f)[W]) {
  if constexpr (is_half_width<TY>::value) {
    uint32_t d[W / 2];
#pragma unroll
    for (int i = 0; i < W / 2; ++i) {
      f32x2 v;
      v.x = f[2 * i];
      v.y = f[2 * i + 1];
      d[i] = narrow2<TY>(v);
    }
    if constexpr (W == 8) {
      buf_store16(r, off, u32x4{d[0], d[1], d[2], d[3]});
    } else {
      buf_store8(r, off, u32x2{d[0], d[1]});
    }
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i)
      buf_store16(r, off + 16u * i,
                  u32x4{as_u32(f[4 * i]), as_u32(f[4 * i + 1]), as_u32(f[4 * i + 2]), as_u32(f[4 * i + 3])});
  }
}

// ---------------------------------------------------------------------------
// Wave64 all-reduce (sum).  Every step pairs lanes symmetrically, so all 64
// lanes finish with bit-identical sums:
//   quad_perm [1,0,3,2], quad_perm [2,3,0,1]   -- within a quad (DPP)
//   row_half_mirror, row_mirror                -- within a 16-lane row (DPP)
//   v_permlane16_swap                          -- rows 0<->1, 2<->3 (gfx950)
//   v_permlane32_swap                          -- lanes 0-31 <-> 32-63 (gfx950)
// No LDS traffic and no ds_bpermute round trips.
// ---------------------------------------------------------------------------
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_allreduce_sum(float v) {
  v += dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  {
    const uint32_t b = as_u32(v);
    auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const uint32_t lo = r[0], hi = r[1];
    v = as_f32(lo) + as_f32(hi);
  }
  {
    const uint32_t b = as_u32(v);
    auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    const uint32_t lo = r[0], hi = r[1];
    v = as_f32(lo) + as_f32(hi);
  }
  return v;
}

// fp32 silu(g) * u with one rounding left to the caller.
//   sigmoid(g) = 1 / (1 + exp(-g));  exp via v_exp_f32 (2^x) on -g*log2(e),
//   reciprocal via v_rcp_f32.  g -> -inf gives exp -> inf, rcp -> 0 and the
//   result -0 * u; g -> +inf gives sigmoid -> 1; NaN propagates.
__device__ __forceinline__ float silu_mul_f32(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  return (g * s) * u;
}

// ---------------------------------------------------------------------------
// MFMA operands shared by the projection kernels (gate/up, W8A16, 16-bit
// linear, tiled GEMM).
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Buffer offset past every descriptor the launchers build (each < 2^31
// bytes): a load there returns zeros and moves no data.
constexpr uint32_t kOob = 0xfffffff0u;

// v_mfma_f32_16x16x32_{f16,bf16}: A and B are 8 values of T per lane.
template <typename T> __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma16<F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma16<BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// Four int8 (one dword, byte i = element i) -> four values of T in two dwords
// (element 2j in the low half of dword j).  Exact: |q| <= 128.
template <typename T> __device__ __forceinline__ u32x2 widen_i8x4(uint32_t d);
template <> __device__ __forceinline__ u32x2 widen_i8x4<F16>(uint32_t d) {
  // Bias each byte to u = q + 128 and splice it under the fp16 pattern 0x64:
  // 0x64uu is 1024 + u exactly; subtracting 1152 leaves q.
  const uint32_t u = d ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes u0,64,u1,64
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2,64,u3,64
  const f16x2 off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
  const f16x2 a = __builtin_bit_cast(f16x2, lo) + off;
  const f16x2 b = __builtin_bit_cast(f16x2, hi) + off;
  return u32x2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}
template <> __device__ __forceinline__ u32x2 widen_i8x4<BF16>(uint32_t d) {
  // Signed byte -> fp32 (exact), then the upper half of each fp32 pattern is
  // the bf16 pattern of the same (8-significant-bit) integer.
  const float f0 = static_cast<float>(static_cast<int8_t>(d & 0xffu));
  const float f1 = static_cast<float>(static_cast<int8_t>((d >> 8) & 0xffu));
  const float f2 = static_cast<float>(static_cast<int8_t>((d >> 16) & 0xffu));
  const float f3 = static_cast<float>(static_cast<int8_t>(d >> 24));
  return u32x2{__builtin_amdgcn_perm(as_u32(f1), as_u32(f0), 0x07060302u),
               __builtin_amdgcn_perm(as_u32(f3), as_u32(f2), 0x07060302u)};
}

// Element i of a float vector stored as F32 / F16 / BF16 (dtype code dt):
// scales and biases, whose dtype is a run-time argument.
__device__ __forceinline__ float load_dyn(const void* p, int64_t i, int dt) {
  if (dt == MI355_F16) return load_elem<F16>(p, i);
  if (dt == MI355_BF16) return load_elem<BF16>(p, i);
  return load_elem<F32>(p, i);
}

// ---------------------------------------------------------------------------
// Host-side helpers shared by the launchers.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int compute_units(int* out);  // CU count of the current device, cached per device

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MI355_OK;
  set_error("%s: %s", what, hipGetErrorString(e));
  return MI355_ERR_HIP;
}

}  // namespace mi355
