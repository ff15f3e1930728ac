// Launcher for the RMSNorm kernels (plain and residual-add fused): picks
// wave-per-row, workgroup-per-row or the generic kernel from the row width,
// alignment and dtype mix, and sizes the grid.
#include "rmsnorm_kernels.h"

// Optional cap on the grid, in waves per CU, for the row-striding kernels;
// 0 = one wave (or workgroup) per row, which measured fastest on MI355X.
#ifndef MI355_RMS_WAVES_PER_CU
#define MI355_RMS_WAVES_PER_CU 0
#endif
// Row counts below this use 64-thread workgroups (one wave each), so small
// decode batches spread over as many CUs as rows.
#ifndef MI355_RMS_SMALL_ROWS
#define MI355_RMS_SMALL_ROWS 1024
#endif
// Row split: rows needing more than WAVE_MAX_VPL packets per lane of one wave
// are spread over several waves with at most TARGET_VPL packets per lane
// (measured on MI355X: 1536-wide fp16 rows are fastest as 3 packets per lane
// of one wave, 3584-wide bf16 rows as 2 packets per lane of 4 waves).
#ifndef MI355_RMS_WAVE_MAX_VPL
#define MI355_RMS_WAVE_MAX_VPL 4
#endif
#ifndef MI355_RMS_TARGET_VPL
#define MI355_RMS_TARGET_VPL 2
#endif

namespace mi355 {
namespace {

template <typename K>
int launch_rms(K kernel, int64_t grid, int block, const RmsParams& p, hipStream_t s) {
  void* args[] = {const_cast<RmsParams*>(&p)};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel),
                                    dim3(static_cast<unsigned>(grid)), dim3(block), args, 0, s),
                    "rmsnorm launch");
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_generic(const RmsParams& p, hipStream_t s, int cus) {
  int64_t grid = p.rows;
  const int64_t cap = static_cast<int64_t>(cus) * 8;
  if (grid > cap) grid = cap;  // two-pass kernel: cap so the second pass finds the row in L2
  return launch_rms(rmsnorm_generic<TX, TW, TY, ADD>, grid, 256, p, s);
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_wave(const RmsParams& p, hipStream_t s, int cus, int vpl) {
  const int block = p.rows < MI355_RMS_SMALL_ROWS ? 64 : 256;
  const int wpb = block / 64;
  int64_t grid = (p.rows + wpb - 1) / wpb;
  const int64_t cap = MI355_RMS_WAVES_PER_CU > 0 ? static_cast<int64_t>(cus) * MI355_RMS_WAVES_PER_CU / wpb
                                                 : int64_t{0x7fffffff};
  if (grid > cap) grid = cap;
#define MI355_WAVE_CASE(V) \
  return launch_rms(rmsnorm_wave_rows<TX, TW, TY, V, ADD>, grid, block, p, s)
  switch (vpl) {
    case 1: MI355_WAVE_CASE(1);
    case 2: MI355_WAVE_CASE(2);
    case 3: MI355_WAVE_CASE(3);
    case 4: MI355_WAVE_CASE(4);
#if MI355_RMS_WAVE_MAX_VPL > 4
    case 5: MI355_WAVE_CASE(5);
    case 6: MI355_WAVE_CASE(6);
    case 7: MI355_WAVE_CASE(7);
    case 8: MI355_WAVE_CASE(8);
    case 9:
    case 10: MI355_WAVE_CASE(10);
    case 11:
    case 12: MI355_WAVE_CASE(12);
    case 13: case 14: case 15:
    case 16: MI355_WAVE_CASE(16);
#endif
    default:
      set_error("rmsnorm: internal error, no wave kernel for %d packets per lane", vpl);
      return MI355_ERR_UNSUPPORTED;
  }
#undef MI355_WAVE_CASE
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_block(const RmsParams& p, hipStream_t s, int waves, int vpl) {
  const int block = 64 * waves;
  int64_t grid = p.rows;
  if (grid > 0x7fffffff) grid = 0x7fffffff;
#define MI355_BLOCK_CASE(V) \
  return launch_rms(rmsnorm_block_rows<TX, TW, TY, V, ADD>, grid, block, p, s)
  switch (vpl) {
    case 1: MI355_BLOCK_CASE(1);
    case 2: MI355_BLOCK_CASE(2);
    case 3: MI355_BLOCK_CASE(3);
    case 4: MI355_BLOCK_CASE(4);
    default: MI355_BLOCK_CASE(8);
  }
#undef MI355_BLOCK_CASE
}

bool row_aligned(const void* base, int64_t stride, size_t elem) {
  return aligned16(base) && (stride * static_cast<int64_t>(elem)) % 16 == 0;
}

// Packet path: n a multiple of the packet width, every pointer and row
// stride 16-byte aligned.
template <typename TX, typename TW, typename TY, bool ADD>
int rms_packets(const RmsParams& p, hipStream_t s, int cus) {
  constexpr int W = pack_width<TX>::value;
  const size_t xe = sizeof(typename TX::bits);
  const bool ok = (p.n % W) == 0 && aligned16(p.w) && row_aligned(p.x, p.xs, xe) &&
                  row_aligned(p.y, p.ys, sizeof(typename TY::bits)) &&
                  (!ADD || (row_aligned(p.r, p.rs, xe) && row_aligned(p.ro, p.ros, xe)));
  if (!ok) return rms_generic<TX, TW, TY, ADD>(p, s, cus);
  const int nvec = p.n / W;
  const int vpl64 = (nvec + 63) / 64;
  if (vpl64 <= MI355_RMS_WAVE_MAX_VPL) return rms_wave<TX, TW, TY, ADD>(p, s, cus, vpl64);
  // Spread the row over enough waves (at most 16) for <= TARGET_VPL packets
  // per lane, then use the fewest waves for that many packets per lane.
  const int target = MI355_RMS_TARGET_VPL < 8 ? MI355_RMS_TARGET_VPL : 8;
  int waves = (nvec + 64 * target - 1) / (64 * target);
  if (waves > 16) waves = 16;
  const int vpl = (nvec + 64 * waves - 1) / (64 * waves);
  if (vpl > 8) return rms_generic<TX, TW, TY, ADD>(p, s, cus);
  waves = (nvec + 64 * vpl - 1) / (64 * vpl);
  return rms_block<TX, TW, TY, ADD>(p, s, waves, vpl);
}

template <typename TX, typename TY, bool ADD>
int rms_by_weight(const RmsParams& p, int w_dtype, hipStream_t s, int cus) {
  // Packet kernels exist for a weight stored like x or in fp32; other mixes
  // take the generic kernel.
  if (w_dtype == TX::code) return rms_packets<TX, TX, TY, ADD>(p, s, cus);
  if (w_dtype == MI355_F32) return rms_packets<TX, F32, TY, ADD>(p, s, cus);
  if (w_dtype == MI355_F16) return rms_generic<TX, F16, TY, ADD>(p, s, cus);
  return rms_generic<TX, BF16, TY, ADD>(p, s, cus);
}

template <bool ADD>
int rms_dispatch(const RmsParams& p, int x_dtype, int w_dtype, int y_dtype, hipStream_t s) {
  int cus = 0;
  const int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  if (x_dtype == MI355_F16 && y_dtype == MI355_F16) return rms_by_weight<F16, F16, ADD>(p, w_dtype, s, cus);
  if (x_dtype == MI355_F16 && y_dtype == MI355_F32) return rms_by_weight<F16, F32, ADD>(p, w_dtype, s, cus);
  if (x_dtype == MI355_BF16 && y_dtype == MI355_BF16) return rms_by_weight<BF16, BF16, ADD>(p, w_dtype, s, cus);
  if (x_dtype == MI355_BF16 && y_dtype == MI355_F32) return rms_by_weight<BF16, F32, ADD>(p, w_dtype, s, cus);
  if (x_dtype == MI355_F32 && y_dtype == MI355_F32) return rms_by_weight<F32, F32, ADD>(p, w_dtype, s, cus);
  set_error("rmsnorm: unsupported dtype pair (x=%d, y=%d)", x_dtype, y_dtype);
  return MI355_ERR_UNSUPPORTED;
}

}  // namespace

int rmsnorm_launch(const void* x, const void* w, void* y, int64_t rows, int n, int64_t xs, int64_t ys,
                   float eps, int x_dtype, int w_dtype, int y_dtype, hipStream_t stream) {
  const RmsParams p{x, nullptr, w, y, nullptr, rows, n, xs, 0, ys, 0, eps};
  return rms_dispatch<false>(p, x_dtype, w_dtype, y_dtype, stream);
}

int add_rmsnorm_launch(const void* x, const void* r, const void* w, void* y, void* ro, int64_t rows, int n,
                       int64_t xs, int64_t rs, int64_t ys, int64_t ros, float eps, int x_dtype, int w_dtype,
                       int y_dtype, hipStream_t stream) {
  const RmsParams p{x, r, w, y, ro, rows, n, xs, rs, ys, ros, eps};
  return rms_dispatch<true>(p, x_dtype, w_dtype, y_dtype, stream);
}

}  // namespace mi355
