// SiLU-and-mul (the SwiGLU activation) for gfx950, plus its launcher.
//
// Semantics follow the reference's Triton kernel
// (src/kernels/fused_swiglu_triton.py:26-36): gate and up are widened to
// fp32, out = (g * sigmoid(g)) * u, rounded once to the output type.  The
// tensors are treated as flat memory, as the reference does.
//
// silu_mul_chunks: a one-shot grid; block b owns the contiguous chunk of
// B * U 16-byte packets starting at packet b * B * U (16 KiB of gate and of
// up with either shipped shape).  Lane t moves packets t + j * B, so every
// load instruction of a wave covers 1 KiB of contiguous memory.  All 2 * U
// loads of a lane are issued before any arithmetic.  Accesses go
// through per-block buffer descriptors sized to the chunk, so the ragged last
// chunk needs no lane branches (out-of-range loads read 0, stores drop), and
// carry the non-temporal hint: every byte is touched once.  The numel % W
// element tail is finished with scalar accesses by the last block.
// silu_mul_generic: scalar grid-stride loop for misaligned pointers.
//
// Launch shape (nt loads and stores, one block per chunk rather than a
// persistent grid), measured on MI355X: 512 lanes x 2 packets per lane below
// 2^27 elements (the 110 MB C2 shape: 18.41 vs 18.77 us for 256 x 4; 440 MB:
// 67.70 vs 67.96 us), 256 lanes x 4 packets from there (the 1.86 GB C4
// shape: 288.6 vs 291.4 us).  A lane issues its loads in the order gate j,
// up j, gate j + 1, ...
#include "common.h"

namespace mi355 {

constexpr int kSiluBlock = 512, kSiluUnroll = 2;
constexpr int kSiluLargeBlock = 256, kSiluLargeUnroll = 4;
constexpr int64_t kSiluLargeMinNumel = int64_t{1} << 27;

template <typename TI, typename TO, int B, int U>
__global__ __launch_bounds__(B) void silu_mul_chunks(const void* __restrict__ gate, const void* __restrict__ up,
                                                     void* __restrict__ out, int64_t numel) {
  constexpr int W = pack_width<TI>::value;
  constexpr int OUT_BYTES = W * sizeof(typename TO::bits);  // output bytes per packet
  const int64_t npk = numel / W;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * B * U;
  const int64_t left = npk - first;
  const uint32_t count = left < B * U ? static_cast<uint32_t>(left > 0 ? left : 0) : static_cast<uint32_t>(B * U);

  const rsrc_t rg = make_rsrc(static_cast<const char*>(gate) + first * 16, count * 16u);
  const rsrc_t ru = make_rsrc(static_cast<const char*>(up) + first * 16, count * 16u);
  const rsrc_t ro = make_rsrc(static_cast<char*>(out) + first * OUT_BYTES, count * OUT_BYTES);

  Packet<TI> gv[U], uv[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t off = (threadIdx.x + j * B) * 16u;
    gv[j].raw = buf_load16(rg, off);
    uv[j].raw = buf_load16(ru, off);
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    float g[W], u[W], o[W];
    gv[j].unpack(g);
    uv[j].unpack(u);
#pragma unroll
    for (int e = 0; e < W; ++e) o[e] = silu_mul_f32(g[e], u[e]);
    buf_store_chunk<TO, W>(ro, (threadIdx.x + j * B) * static_cast<uint32_t>(OUT_BYTES), o);
  }

  if (blockIdx.x == gridDim.x - 1) {
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

template <typename TI, typename TO, int B, int U>
int silu_chunked(const SiluArgs& a, hipStream_t s) {
  constexpr int W = pack_width<TI>::value;
  const int64_t npk = a.numel / W;
  constexpr int64_t chunk = static_cast<int64_t>(B) * U;
  int64_t grid = (npk + chunk - 1) / chunk;
  if (grid < 1) grid = 1;  // numel < W: the single block runs the scalar tail
  if (grid > 0x7fffffff) {
    set_error("mi355_silu_mul_fwd: numel %lld needs more than 2^31 workgroups", static_cast<long long>(a.numel));
    return MI355_ERR_UNSUPPORTED;
  }
  return launch_silu(silu_mul_chunks<TI, TO, B, U>, grid, B, a, s);
}

template <typename TI, typename TO>
int silu_typed(const SiluArgs& a, hipStream_t s, int cus) {
  const bool vec_ok = aligned16(a.gate) && aligned16(a.up) && aligned16(a.out);
  if (!vec_ok) {
    int64_t grid = (a.numel + 255) / 256;
    const int64_t cap = static_cast<int64_t>(cus) * 8;
    if (grid > cap) grid = cap;
    return launch_silu(silu_mul_generic<TI, TO>, grid, 256, a, s);
  }
  if (a.numel >= kSiluLargeMinNumel) return silu_chunked<TI, TO, kSiluLargeBlock, kSiluLargeUnroll>(a, s);
  return silu_chunked<TI, TO, kSiluBlock, kSiluUnroll>(a, s);
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
