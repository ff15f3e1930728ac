// Measurement helpers, not part of the kernel ABI: the W8A16 decode kernel
// (w8a16_stream.h, the same source the library compiles) launched with a
// launch shape chosen by the caller instead of its launch plan, so bench.py
// can time the plan against other shapes on the same inputs (fp16 x and
// output, fp32 scales, no bias); the plan itself; and the kernel's loads
// alone at a launch shape, for the decomposition of its time.
#include <cstdarg>
#include <cstdio>

#include "../w8a16_stream.h"

namespace mi355 {
// The library's set_error keeps a per-thread message; here a failing launch
// is reported through the status code alone.
void set_error(const char*, ...) {}
}  // namespace mi355

namespace {

// The loads of w8a16_stream at launch shape (rpw, waves, U), and nothing
// else: the same descriptors, lane offsets, chunk split and U-chunk groups,
// every loaded dword folded into one XOR that guards a store the data never
// trigger (so no load can be dropped); without X only the weights.
template <int R4, int MT4, int U, bool X>
__global__ __launch_bounds__(1024) void w8a16_stream_loads(const mi355::W8Params p, const int rpw,
                                                           uint32_t* sink) {
  using namespace mi355;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwave = blockDim.x >> 6;
  const int n0 = blockIdx.x * rpw;
  const int nrows_w = p.n - n0 < rpw ? p.n - n0 : rpw;
  const rsrc_t rq = make_rsrc(static_cast<const int8_t*>(p.q) + static_cast<int64_t>(n0) * p.qs,
                              static_cast<uint32_t>((nrows_w - 1) * p.qs + p.k));
  const rsrc_t rx = make_rsrc(p.x, static_cast<uint32_t>(((p.rows - 1) * p.xs + p.k) * 2));
  const int quad = lane & 3, set_row = (lane & 15) >> 2, kg = lane >> 4;
  const int piece = 16 * quad + 64 * kg;
  uint32_t qoff[R4], xoff[MT4];
#pragma unroll
  for (int r = 0; r < R4; ++r) qoff[r] = static_cast<uint32_t>((4 * r + set_row) * p.qs + piece);
#pragma unroll
  for (int t = 0; t < MT4; ++t) xoff[t] = static_cast<uint32_t>(((4 * t + set_row) * p.xs + piece) * 2);
  const int nchunk = (p.k + 255) >> 8;
  const int c0 = (nchunk * wave) / nwave, c1 = (nchunk * (wave + 1)) / nwave;
  uint32_t h = 0;
  for (int c = c0; c < c1; c += U) {
    u32x4 wq[U][R4], xa[U][MT4][2];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const bool live = c + j < c1 && 256 * (c + j) + piece < p.k;
#pragma unroll
      for (int r = 0; r < R4; ++r) wq[j][r] = buf_load16(rq, live ? qoff[r] + 256u * (c + j) : kOob);
      if constexpr (X) {
#pragma unroll
        for (int t = 0; t < MT4; ++t) {
          const uint32_t o = xoff[t] + 512u * (c + j);
          xa[j][t][0] = buf_load16_cached(rx, live ? o : kOob);
          xa[j][t][1] = buf_load16_cached(rx, live ? o + 16u : kOob);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
      for (int r = 0; r < R4; ++r) h ^= (wq[j][r].x ^ wq[j][r].y) ^ (wq[j][r].z ^ wq[j][r].w);
      if constexpr (X) {
#pragma unroll
        for (int t = 0; t < MT4; ++t)
          h ^= (xa[j][t][0].x ^ xa[j][t][0].w) ^ (xa[j][t][1].y ^ xa[j][t][1].z) ^ (xa[j][t][0].y ^ xa[j][t][0].z) ^
               (xa[j][t][1].x ^ xa[j][t][1].w);
      }
    }
  }
  if (h == 0x9e3779b9u) sink[threadIdx.x] = h;
}

template <int R4, int MT4, bool X>
const void* loads_kernel(int u) {
  if (u >= 2) return reinterpret_cast<const void*>(w8a16_stream_loads<R4, MT4, 2, X>);
  return reinterpret_cast<const void*>(w8a16_stream_loads<R4, MT4, 1, X>);
}

template <bool X>
const void* loads_kernel_r4(int r4, int mt4, int u) {
  if (r4 == 4) return mt4 == 1 ? loads_kernel<4, 1, X>(u) : loads_kernel<4, 2, X>(u);
  if (r4 == 2) return mt4 == 1 ? loads_kernel<2, 1, X>(u) : loads_kernel<2, 2, X>(u);
  return mt4 == 1 ? loads_kernel<1, 1, X>(u) : loads_kernel<1, 2, X>(u);
}

}  // namespace

// The launch plan the library picks for `rows` x [n, k] int8 weights (dual:
// two matrices) on a device with `cus` CUs: out4 = {rpw, r4, waves, u}.
extern "C" __attribute__((visibility("default"))) void mi355_probe_w8a16_stream_plan(int rows, int k, int n, int dual,
                                                                                   int cus, int* out4) {
  const mi355::StreamPlan sp = mi355::w8_stream_plan(rows, k, n, dual != 0, cus);
  out4[0] = sp.rpw;
  out4[1] = sp.r4;
  out4[2] = sp.waves;
  out4[3] = sp.u;
}

// The loads of the W8A16 decode kernel alone (w8a16_stream_loads above) at
// launch shape (rpw, r4, waves, u) for x [rows <= 8, k] fp16 and q [n, k]
// int8: the weights only (with_x 0) or the weights and x (with_x 1).  `sink`
// holds at least 1024 dwords.  Returns 0, -1 on bad arguments, -3 on a
// launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_w8a16_stream_loads(
    const void* x, const void* q, int rows, int k, int n, int rpw, int r4, int waves, int u, int with_x, void* sink,
    void* stream) {
  if (!x || !q || !sink || rows < 1 || rows > 8 || k < 16 || (k & 15) || n < 1 || rpw < 1 ||
      (r4 != 1 && r4 != 2 && r4 != 4) || rpw > 4 * r4 || waves < 1 || waves > 16 || (u != 1 && u != 2))
    return -1;
  const mi355::W8Params p{x, q, nullptr, nullptr, nullptr, rows, k, n, k, k, n, MI355_F32, -1, nullptr, nullptr};
  const int mt4 = rows <= 4 ? 1 : 2;
  const void* kern = with_x ? loads_kernel_r4<true>(r4, mt4, u) : loads_kernel_r4<false>(r4, mt4, u);
  int rpw_arg = rpw;
  void* args[] = {const_cast<mi355::W8Params*>(&p), &rpw_arg, &sink};
  const unsigned grid = static_cast<unsigned>((n + rpw - 1) / rpw);
  if (hipLaunchKernel(kern, dim3(grid), dim3(64 * waves), args, 0, static_cast<hipStream_t>(stream)) != hipSuccess)
    return -3;
  return 0;
}

namespace {

// The decode kernel at any launch shape the probes accept: R4 in {1, 2, 4}
// (and 8 with up to 8 rows of x), MT4 = stream_x_sets(rows) in 1 .. 4, 6, 8,
// 12, 16 (64 rows of x), U in {1, 2} (U = 1 only for MT4 > 2); fp16 x,
// weights of WB bytes.
template <bool DUAL, int WB, int R4, int MT4>
const void* sk_u(int u) {
  using mi355::F16;
  if constexpr (MT4 <= 2 && mi355::stream_max_threads(R4, MT4, 2, DUAL, WB) > 0) {
    if (u >= 2) return reinterpret_cast<const void*>(mi355::w8a16_stream<F16, F16, R4, MT4, 2, DUAL, WB>);
  }
  // shapes without a kernel (stream_max_threads 0): shape_ok rejects them
  if constexpr (mi355::stream_max_threads(R4, MT4, 1, DUAL, WB) == 0) return nullptr;
  else return reinterpret_cast<const void*>(mi355::w8a16_stream<F16, F16, R4, MT4, 1, DUAL, WB>);
}
template <bool DUAL, int WB, int R4>
const void* sk_mt(int mt4, int u) {
  if (mt4 == 1) return sk_u<DUAL, WB, R4, 1>(u);
  if (mt4 == 2) return sk_u<DUAL, WB, R4, 2>(u);
  if (mt4 == 3) return sk_u<DUAL, WB, R4, 3>(u);
  if (mt4 == 4) return sk_u<DUAL, WB, R4, 4>(u);
  if (mt4 == 6) return sk_u<DUAL, WB, R4, 6>(u);
  if (mt4 == 8) return sk_u<DUAL, WB, R4, 8>(u);
  if (mt4 == 12) return sk_u<DUAL, WB, R4, 12>(u);
  return sk_u<DUAL, WB, R4, 16>(u);
}
template <bool DUAL, int WB>
const void* stream_kernel(int r4, int mt4, int u) {
  if (r4 == 8) return mt4 == 1 ? sk_u<DUAL, WB, 8, 1>(u) : (mt4 == 2 ? sk_u<DUAL, WB, 8, 2>(u) : nullptr);
  if (r4 >= 4) return sk_mt<DUAL, WB, 4>(mt4, u);
  if (r4 == 2) return sk_mt<DUAL, WB, 2>(mt4, u);
  return sk_mt<DUAL, WB, 1>(mt4, u);
}

bool shape_ok(int rows, int n, int rpw, int r4, int waves, int u, bool dual, int wb) {
  const int mt4 = mi355::stream_x_sets(rows);
  return rows >= 1 && rows <= 64 && n >= 1 && rpw >= 1 && (r4 == 1 || r4 == 2 || r4 == 4 || (r4 == 8 && mt4 <= 2)) &&
         rpw <= 4 * r4 &&
         waves >= 1 && 64 * waves <= mi355::stream_max_threads(r4, mt4, u, dual, wb) &&
         (u == 1 || (u == 2 && mt4 <= 2));
}

int launch_stream(const void* kern, const mi355::W8Params& p, int rpw, int r4, int waves, int nq, void* stream) {
  const int mt4 = mi355::stream_x_sets(p.rows);
  const size_t lds = static_cast<size_t>(waves) * nq * r4 * mt4 * 16 * sizeof(float);
  int rpw_arg = rpw;
  void* args[] = {const_cast<mi355::W8Params*>(&p), &rpw_arg};
  const unsigned grid = static_cast<unsigned>((p.n + rpw - 1) / rpw);
  return hipLaunchKernel(kern, dim3(grid), dim3(64 * waves), args, lds, static_cast<hipStream_t>(stream)) == hipSuccess
             ? 0
             : -3;
}

}  // namespace

// out [rows, n] = W8A16(x [rows, k], q [n, k], scale [n]) (q2 / scale2 not
// NULL: the gate/up + SiLU-and-mul kernel with q, scale the gate and q2,
// scale2 the up weights), launched with rpw weight rows per workgroup, r4
// 4-row sets (1, 2 or 4, or 8 up to 8 rows; rpw <= 4 r4), `waves` waves (at most
// stream_max_threads / 64: 16 or 8) and u chunks in flight (1 or 2; 1 above
// 8 rows).  rows <= 32, k a multiple of 16, every pointer
// 16-byte aligned.  Returns 0, -1 on bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_w8a16_stream(
    const void* x, const void* q, const void* scale, const void* q2, const void* scale2, void* out, int rows, int k,
    int n, int rpw, int r4, int waves, int u, void* stream) {
  if (!x || !q || !scale || !out || k < 16 || (k & 15) || !shape_ok(rows, n, rpw, r4, waves, u, q2 != nullptr, 1) ||
      (!q2) != (!scale2))
    return -1;
  const mi355::W8Params p{x, q, scale, nullptr, out, rows, k, n, k, k, n, MI355_F32, -1, q2, scale2};
  const int mt4 = mi355::stream_x_sets(rows);
  const void* kern = q2 ? stream_kernel<true, 1>(r4, mt4, u) : stream_kernel<false, 1>(r4, mt4, u);
  return launch_stream(kern, p, rpw, r4, waves, q2 ? 2 : 1, stream);
}

// out [rows, n] = silu(x @ wg^T) * (x @ wu^T) for x [rows, k] and 16-bit
// weights [n, k] (fp16), by the weight-streaming kernel of w8a16_stream.h
// with 16-bit weights (WB = 2) at launch shape (rpw, r4, waves, u).  rows <=
// 32, k a multiple of 8, every pointer 16-byte aligned.  Returns 0, -1 on
// bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_gate_up16_stream(
    const void* x, const void* wg, const void* wu, void* out, int rows, int k, int n, int rpw, int r4, int waves,
    int u, void* stream) {
  if (!x || !wg || !wu || !out || k < 8 || (k & 7) || !shape_ok(rows, n, rpw, r4, waves, u, true, 2)) return -1;
  const mi355::W8Params p{x, wg, nullptr, nullptr, out, rows, k, n, k, k, n, MI355_F32, -1, wu, nullptr};
  return launch_stream(stream_kernel<true, 2>(r4, mi355::stream_x_sets(rows), u), p, rpw, r4, waves, 2, stream);
}

// out [rows, n] = x @ w^T (+ bias) for x [rows, k] and 16-bit weights [n, k]
// (fp16; bias fp16 or NULL), by the weight-streaming kernel of w8a16_stream.h
// with one 16-bit matrix (WB = 2) at launch shape (rpw, r4, waves, u).  rows
// <= 32, k a multiple of 8, every pointer 16-byte aligned.  Returns 0, -1 on
// bad arguments, -3 on a launch error.
extern "C" __attribute__((visibility("default"))) int mi355_probe_linear16_stream(
    const void* x, const void* w, const void* bias, void* out, int rows, int k, int n, int rpw, int r4, int waves,
    int u, void* stream) {
  if (!x || !w || !out || k < 8 || (k & 7) || !shape_ok(rows, n, rpw, r4, waves, u, false, 2)) return -1;
  const mi355::W8Params p{x, w, nullptr, bias, out, rows, k, n, k, k, n, MI355_F32, bias ? MI355_F16 : -1,
                          nullptr, nullptr};
  return launch_stream(stream_kernel<false, 2>(r4, mi355::stream_x_sets(rows), u), p, rpw, r4, waves, 1, stream);
}

// The 16-bit linear's launch plan (l16_stream_plan) for `rows` x k x n on
// `cus` CUs: out4 = {rpw, r4, waves, u}.
extern "C" __attribute__((visibility("default"))) void mi355_probe_linear16_stream_plan(int rows, int k, int n,
                                                                                         int cus, int* out4) {
  const mi355::StreamPlan sp = mi355::l16_stream_plan(rows, k, n, cus);
  out4[0] = sp.rpw;
  out4[1] = sp.r4;
  out4[2] = sp.waves;
  out4[3] = sp.u;
}

// Most threads per workgroup of w8a16_stream<.., r4, mt4, u, dual, wb>.
extern "C" __attribute__((visibility("default"))) int mi355_probe_stream_max_threads(int r4, int mt4, int u,
                                                                                      int dual, int wb) {
  return mi355::stream_max_threads(r4, mt4, u, dual != 0, wb);
}

// The 16-bit gate/up + SiLU-and-mul's launch plan (gu16_stream_plan) for
// `rows` x k x n on `cus` CUs: out4 = {rpw, r4, waves, u}.
extern "C" __attribute__((visibility("default"))) void mi355_probe_gate_up16_stream_plan(int rows, int k, int n, int cus,
                                                                                          int* out4) {
  const mi355::StreamPlan sp = mi355::gu16_stream_plan(rows, k, n, cus);
  out4[0] = sp.rpw;
  out4[1] = sp.r4;
  out4[2] = sp.waves;
  out4[3] = sp.u;
}
