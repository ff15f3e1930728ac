// SiLU-and-mul (the SwiGLU activation) for gfx950, plus its launcher.
//
// Semantics follow the reference's Triton kernel
// (src/kernels/fused_swiglu_triton.py:26-36): gate and up are widened to
// fp32, out = (g * sigmoid(g)) * u, rounded once to the output type.  The
// tensors are treated as flat memory, as the reference does.
//
// silu_mul_vec: every lane moves UNROLL 16-byte packets of gate and of up per
// iteration, issuing all 2*UNROLL loads before any arithmetic so a wave keeps
// 2*UNROLL KiB in flight; consecutive lanes touch consecutive packets (1 KiB
// per wave per load instruction).  The grid strides over the packets, so the
// launcher can size it to what the device keeps resident.  The numel % W tail
// is finished by block 0 with scalar accesses.
// silu_mul_generic: scalar grid-stride loop for misaligned pointers.
#include "common.h"

#ifndef MI355_SILU_BLOCK
#define MI355_SILU_BLOCK 256
#endif
#ifndef MI355_SILU_UNROLL
#define MI355_SILU_UNROLL 4
#endif
#ifndef MI355_SILU_BLOCKS_PER_CU
#define MI355_SILU_BLOCKS_PER_CU 8
#endif
// Below this many packets the launcher uses UNROLL = 1 so small (decode)
// shapes spread over more workgroups.
#ifndef MI355_SILU_SMALL_PACKETS
#define MI355_SILU_SMALL_PACKETS (1 << 16)
#endif

namespace mi355 {

template <typename TI, typename TO, int UNROLL>
__global__ __launch_bounds__(MI355_SILU_BLOCK) void silu_mul_vec(const void* __restrict__ gate,
                                                                 const void* __restrict__ up,
                                                                 void* __restrict__ out,
                                                                 int64_t numel) {
  constexpr int W = pack_width<TI>::value;
  constexpr int B = MI355_SILU_BLOCK;
  using OB = typename TO::bits;
  const int64_t npk = numel / W;
  const u32x4* g4 = static_cast<const u32x4*>(gate);
  const u32x4* u4 = static_cast<const u32x4*>(up);
  const int64_t step = static_cast<int64_t>(gridDim.x) * B * UNROLL;

  for (int64_t base = static_cast<int64_t>(blockIdx.x) * B * UNROLL + threadIdx.x; base < npk;
       base += step) {
    Packet<TI> gv[UNROLL], uv[UNROLL];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
      const int64_t p = base + j * B;
      if (p < npk) {
        gv[j].raw = g4[p];
        uv[j].raw = u4[p];
      }
    }
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
      const int64_t p = base + j * B;
      if (p < npk) {
        float g[W], u[W], o[W];
        gv[j].unpack(g);
        uv[j].unpack(u);
#pragma unroll
        for (int e = 0; e < W; ++e) o[e] = silu_mul_f32(g[e], u[e]);
        store_chunk<TO, W>(static_cast<OB*>(out) + p * W, o);
      }
    }
  }

  if (blockIdx.x == 0) {
    for (int64_t i = npk * W + threadIdx.x; i < numel; i += B)
      store_elem<TO>(out, i, silu_mul_f32(load_elem<TI>(gate, i), load_elem<TI>(up, i)));
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void silu_mul_generic(const void* __restrict__ gate,
                                                        const void* __restrict__ up,
                                                        void* __restrict__ out, int64_t numel) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < numel; i += step)
    store_elem<TO>(out, i, silu_mul_f32(load_elem<TI>(gate, i), load_elem<TI>(up, i)));
}

namespace {

struct SiluArgs {
  const void* gate;
  const void* up;
  void* out;
  int64_t numel;
};

template <typename K>
int launch_silu(K kernel, int64_t grid, int block, const SiluArgs& a, hipStream_t s) {
  void* args[] = {const_cast<void**>(&a.gate), const_cast<void**>(&a.up),
                  const_cast<void**>(&a.out), const_cast<int64_t*>(&a.numel)};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel),
                                    dim3(static_cast<unsigned>(grid)), dim3(block), args, 0, s),
                    "silu_mul launch");
}

template <typename TI, typename TO>
int silu_typed(const SiluArgs& a, hipStream_t s, int cus) {
  constexpr int W = pack_width<TI>::value;
  const bool vec_ok = aligned16(a.gate) && aligned16(a.up) && aligned16(a.out);
  const int64_t cap = static_cast<int64_t>(cus) * MI355_SILU_BLOCKS_PER_CU;
  if (!vec_ok) {
    int64_t grid = (a.numel + 255) / 256;
    if (grid > cap) grid = cap;
    return launch_silu(silu_mul_generic<TI, TO>, grid, 256, a, s);
  }
  const int64_t npk = a.numel / W;
  const int unroll = npk < MI355_SILU_SMALL_PACKETS ? 1 : MI355_SILU_UNROLL;
  int64_t grid = (npk + static_cast<int64_t>(MI355_SILU_BLOCK) * unroll - 1) /
                 (static_cast<int64_t>(MI355_SILU_BLOCK) * unroll);
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;  // numel < W: block 0 runs the scalar tail
  if (unroll == 1) return launch_silu(silu_mul_vec<TI, TO, 1>, grid, MI355_SILU_BLOCK, a, s);
  return launch_silu(silu_mul_vec<TI, TO, MI355_SILU_UNROLL>, grid, MI355_SILU_BLOCK, a, s);
}

}  // namespace

int silu_mul_launch(const void* gate, const void* up, void* out, int64_t numel, int in_dtype,
                    int out_dtype, hipStream_t stream) {
  int cus = 0;
  int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  const SiluArgs a{gate, up, out, numel};
  if (in_dtype == MI355_F16 && out_dtype == MI355_F16) return silu_typed<F16, F16>(a, stream, cus);
  if (in_dtype == MI355_F16 && out_dtype == MI355_F32) return silu_typed<F16, F32>(a, stream, cus);
  if (in_dtype == MI355_BF16 && out_dtype == MI355_BF16) return silu_typed<BF16, BF16>(a, stream, cus);
  if (in_dtype == MI355_BF16 && out_dtype == MI355_F32) return silu_typed<BF16, F32>(a, stream, cus);
  if (in_dtype == MI355_F32 && out_dtype == MI355_F32) return silu_typed<F32, F32>(a, stream, cus);
  set_error("mi355_silu_mul_fwd: unsupported dtype pair (in=%d, out=%d)", in_dtype, out_dtype);
  return MI355_ERR_UNSUPPORTED;
}

}  // namespace mi355
