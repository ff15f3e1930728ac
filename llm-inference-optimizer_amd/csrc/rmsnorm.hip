// Launcher for the RMSNorm kernels: picks wave-per-row, workgroup-per-row or
// the generic kernel from the row width, alignment and dtype mix, and sizes
// the grid.
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

struct RmsArgs {
  const void* x;
  const void* w;
  void* y;
  int64_t rows;
  int n;
  int64_t xs;
  int64_t ys;
  float eps;
};

template <typename K>
int launch_rms(K kernel, int64_t grid, int block, const RmsArgs& a, hipStream_t s) {
  void* args[] = {const_cast<void**>(&a.x),      const_cast<void**>(&a.w),
                  const_cast<void**>(&a.y),      const_cast<int64_t*>(&a.rows),
                  const_cast<int*>(&a.n),        const_cast<int64_t*>(&a.xs),
                  const_cast<int64_t*>(&a.ys),   const_cast<float*>(&a.eps)};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel),
                                    dim3(static_cast<unsigned>(grid)), dim3(block), args, 0, s),
                    "rmsnorm launch");
}

template <typename TX, typename TW, typename TY>
int rms_generic(const RmsArgs& a, hipStream_t s, int cus) {
  int64_t grid = a.rows;
  const int64_t cap = static_cast<int64_t>(cus) * 8;
  if (grid > cap) grid = cap;  // two-pass kernel: cap so the second pass finds the row in L2
  return launch_rms(rmsnorm_generic<TX, TW, TY>, grid, 256, a, s);
}

template <typename TX, typename TW, typename TY>
int rms_wave(const RmsArgs& a, hipStream_t s, int cus, int vpl) {
  const int block = a.rows < MI355_RMS_SMALL_ROWS ? 64 : 256;
  const int wpb = block / 64;
  int64_t grid = (a.rows + wpb - 1) / wpb;
  const int64_t cap = MI355_RMS_WAVES_PER_CU > 0 ? static_cast<int64_t>(cus) * MI355_RMS_WAVES_PER_CU / wpb
                                                 : int64_t{0x7fffffff};
  if (grid > cap) grid = cap;
#define MI355_WAVE_CASE(V) \
  return launch_rms(rmsnorm_wave_rows<TX, TW, TY, V>, grid, block, a, s)
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
      set_error("mi355_rmsnorm_fwd: internal error, no wave kernel for %d packets per lane", vpl);
      return MI355_ERR_UNSUPPORTED;
  }
#undef MI355_WAVE_CASE
}


template <typename TX, typename TW, typename TY>
int rms_block(const RmsArgs& a, hipStream_t s, int cus, int waves, int vpl) {
  (void)cus;
  const int block = 64 * waves;
  int64_t grid = a.rows;
  if (grid > 0x7fffffff) grid = 0x7fffffff;
#define MI355_BLOCK_CASE(V) \
  return launch_rms(rmsnorm_block_rows<TX, TW, TY, V>, grid, block, a, s)
  switch (vpl) {
    case 1: MI355_BLOCK_CASE(1);
    case 2: MI355_BLOCK_CASE(2);
    case 3: MI355_BLOCK_CASE(3);
    case 4: MI355_BLOCK_CASE(4);
    default: MI355_BLOCK_CASE(8);
  }
#undef MI355_BLOCK_CASE
}

// Packet path: n a multiple of the packet width, every pointer and row
// stride 16-byte aligned.
template <typename TX, typename TW, typename TY>
int rms_packets(const RmsArgs& a, hipStream_t s, int cus) {
  constexpr int W = pack_width<TX>::value;
  const bool ok = (a.n % W) == 0 && aligned16(a.x) && aligned16(a.w) && aligned16(a.y) &&
                  (a.xs * static_cast<int64_t>(sizeof(typename TX::bits))) % 16 == 0 &&
                  (a.ys * static_cast<int64_t>(sizeof(typename TY::bits))) % 16 == 0;
  if (!ok) return rms_generic<TX, TW, TY>(a, s, cus);
  const int nvec = a.n / W;
  const int vpl64 = (nvec + 63) / 64;
  if (vpl64 <= MI355_RMS_WAVE_MAX_VPL) return rms_wave<TX, TW, TY>(a, s, cus, vpl64);
  // Spread the row over enough waves (at most 16) for <= TARGET_VPL packets
  // per lane, then use the fewest packets per lane that covers the row.
  const int target = MI355_RMS_TARGET_VPL < 8 ? MI355_RMS_TARGET_VPL : 8;
  int waves = (nvec + 64 * target - 1) / (64 * target);
  if (waves > 16) waves = 16;
  int vpl = (nvec + 64 * waves - 1) / (64 * waves);
  if (vpl > 8) return rms_generic<TX, TW, TY>(a, s, cus);
  waves = (nvec + 64 * vpl - 1) / (64 * vpl);  // fewest waves for that many packets per lane
  return rms_block<TX, TW, TY>(a, s, cus, waves, vpl);
}

template <typename TX, typename TY>
int rms_by_weight(const RmsArgs& a, int w_dtype, hipStream_t s, int cus) {
  // Packet kernels exist for a weight stored like x or in fp32; other mixes
  // take the generic kernel.
  if (w_dtype == TX::code) return rms_packets<TX, TX, TY>(a, s, cus);
  if (w_dtype == MI355_F32) return rms_packets<TX, F32, TY>(a, s, cus);
  if (w_dtype == MI355_F16) return rms_generic<TX, F16, TY>(a, s, cus);
  return rms_generic<TX, BF16, TY>(a, s, cus);
}

}  // namespace

int rmsnorm_launch(const void* x, const void* w, void* y, int64_t rows, int n, int64_t xs,
                   int64_t ys, float eps, int x_dtype, int w_dtype, int y_dtype,
                   hipStream_t stream) {
  int cus = 0;
  int st = compute_units(&cus);
  if (st != MI355_OK) return st;
  const RmsArgs a{x, w, y, rows, n, xs, ys, eps};
  if (x_dtype == MI355_F16 && y_dtype == MI355_F16) return rms_by_weight<F16, F16>(a, w_dtype, stream, cus);
  if (x_dtype == MI355_F16 && y_dtype == MI355_F32) return rms_by_weight<F16, F32>(a, w_dtype, stream, cus);
  if (x_dtype == MI355_BF16 && y_dtype == MI355_BF16) return rms_by_weight<BF16, BF16>(a, w_dtype, stream, cus);
  if (x_dtype == MI355_BF16 && y_dtype == MI355_F32) return rms_by_weight<BF16, F32>(a, w_dtype, stream, cus);
  if (x_dtype == MI355_F32 && y_dtype == MI355_F32) return rms_by_weight<F32, F32>(a, w_dtype, stream, cus);
  set_error("mi355_rmsnorm_fwd: unsupported dtype pair (x=%d, y=%d)", x_dtype, y_dtype);
  return MI355_ERR_UNSUPPORTED;
}

}  // namespace mi355
