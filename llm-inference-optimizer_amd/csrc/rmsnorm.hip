// Launcher for the RMSNorm kernels (plain and residual-add fused): picks
// wave-per-row, workgroup-per-row or the generic kernel from the row width,
// alignment and dtype mix, and sizes the grid.
//
// The -D switches below select launch shapes; the defaults are the shapes
// measured fastest on MI355X.  A variant library built with other values
// (`build.py -DMI355_RMS_... --out <lib>`) runs the same kernels with the
// same results, so bench.py can time the alternatives side by side.
#include "rmsnorm_kernels.h"

// Optional caps on the grid (a persistent grid, rows striding over it):
// waves per CU for the wave-per-row kernel, workgroups per CU for the
// workgroup-per-row kernel; 0 = one wave (or workgroup) per row group.
#ifndef MI355_RMS_WAVES_PER_CU
#define MI355_RMS_WAVES_PER_CU 0
#endif
#ifndef MI355_RMS_BLOCKS_PER_CU
#define MI355_RMS_BLOCKS_PER_CU 0
#endif
// Row counts below this use 64-thread workgroups (one wave each) and one row
// per wave, so small decode batches spread over as many CUs as rows.
#ifndef MI355_RMS_SMALL_ROWS
#define MI355_RMS_SMALL_ROWS 1024
#endif
// Row split: rows needing more than WAVE_MAX_VPL packets per lane of one wave
// are spread over several waves with at most TARGET_VPL packets per lane
// (1536-wide fp16 rows run as 3 packets per lane of one wave, 3584-wide bf16
// rows as 2 packets per lane of 4 waves).
#ifndef MI355_RMS_WAVE_MAX_VPL
#define MI355_RMS_WAVE_MAX_VPL 4
#endif
#ifndef MI355_RMS_TARGET_VPL
#define MI355_RMS_TARGET_VPL 2
#endif
static_assert(MI355_RMS_WAVE_MAX_VPL >= 1 && MI355_RMS_WAVE_MAX_VPL <= 8, "wave kernels exist for 1-8 packets per lane");
// Rows each wave (wave-per-row kernel) or each workgroup iteration
// (workgroup-per-row kernel) holds at once, from MI355_RMS_SMALL_ROWS rows up:
// all their loads are in flight together, behind one reduction (and, for the
// workgroup kernel, one barrier).  The fused residual add moves twice the
// bytes of a row and measured 1.06x faster with two rows per wave at the
// 2048 x 1536 fp16 shape; the plain norm is fastest with one.
#ifndef MI355_RMS_WAVE_ROWS
#define MI355_RMS_WAVE_ROWS 1
#endif
#ifndef MI355_RMS_WAVE_ROWS_ADD
#define MI355_RMS_WAVE_ROWS_ADD 2
#endif
#ifndef MI355_RMS_BLOCK_ROWS
#define MI355_RMS_BLOCK_ROWS 1
#endif
// > 1: from MI355_RMS_SMALL_ROWS rows up, rows wide enough for the
// workgroup-per-row kernel stream through a persistent grid of
// MI355_RMS_STREAM_BLOCKS_PER_CU workgroups per CU, each keeping this many
// rows in flight (rmsnorm_block_stream); 0 = one workgroup per row.
#ifndef MI355_RMS_STREAM_ROWS
#define MI355_RMS_STREAM_ROWS 0
#endif
#ifndef MI355_RMS_STREAM_BLOCKS_PER_CU
#define MI355_RMS_STREAM_BLOCKS_PER_CU 4
#endif
// 1: the wave-per-row kernel stages the weight row in LDS once per
// workgroup and broadcasts it to its waves, instead of each wave loading its
// weight packets from L2.
#ifndef MI355_RMS_WEIGHT_LDS
#define MI355_RMS_WEIGHT_LDS 0
#endif

namespace mi355 {
namespace {

template <typename K>
int launch_rms(K kernel, int64_t grid, int block, const RmsParams& p, hipStream_t s, size_t lds = 0) {
  void* args[] = {const_cast<RmsParams*>(&p)};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel),
                                    dim3(static_cast<unsigned>(grid)), dim3(block), args, lds, s),
                    "rmsnorm launch");
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_generic(const RmsParams& p, hipStream_t s, int cus) {
  int64_t grid = p.rows;
  const int64_t cap = static_cast<int64_t>(cus) * 8;
  if (grid > cap) grid = cap;  // two-pass kernel: cap so the second pass finds the row in L2
  return launch_rms(rmsnorm_generic<TX, TW, TY, ADD>, grid, 256, p, s);
}

template <typename TX, typename TW, typename TY, int VPL, int R, bool ADD>
int rms_wave_shape(const RmsParams& p, hipStream_t s, int cus, int block) {
  const int wpb = block / 64;
  const int64_t per_block = static_cast<int64_t>(wpb) * R;
  int64_t grid = (p.rows + per_block - 1) / per_block;
  const int64_t cap = MI355_RMS_WAVES_PER_CU > 0 ? static_cast<int64_t>(cus) * MI355_RMS_WAVES_PER_CU / wpb
                                                 : int64_t{0x7fffffff};
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
  constexpr bool wlds = MI355_RMS_WEIGHT_LDS != 0;
  constexpr size_t lds = wlds ? 64u * VPL * pack_width<TX>::value * sizeof(typename TW::bits) : 0u;
  return launch_rms(rmsnorm_wave_rows<TX, TW, TY, VPL, R, ADD, wlds>, grid, block, p, s, lds);
}

template <typename TX, typename TW, typename TY, int VPL, bool ADD>
int rms_wave_rows(const RmsParams& p, hipStream_t s, int cus) {
  constexpr int R = ADD ? MI355_RMS_WAVE_ROWS_ADD : MI355_RMS_WAVE_ROWS;
  if (p.rows < MI355_RMS_SMALL_ROWS) return rms_wave_shape<TX, TW, TY, VPL, 1, ADD>(p, s, cus, 64);
  return rms_wave_shape<TX, TW, TY, VPL, R, ADD>(p, s, cus, MI355_RMS_WAVE_BLOCK);
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_wave(const RmsParams& p, hipStream_t s, int cus, int vpl) {
#define MI355_WAVE_CASE(V) return rms_wave_rows<TX, TW, TY, V, ADD>(p, s, cus)
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
#endif
    default:
      set_error("rmsnorm: internal error, no wave kernel for %d packets per lane", vpl);
      return MI355_ERR_UNSUPPORTED;
  }
#undef MI355_WAVE_CASE
}

template <typename TX, typename TW, typename TY, int VPL, bool ADD>
int rms_block_rows(const RmsParams& p, hipStream_t s, int cus, int block) {
  // (only where the ring of rows fits the register file next to the rest)
  if constexpr (MI355_RMS_STREAM_ROWS > 1 && VPL * MI355_RMS_STREAM_ROWS <= 8) {
    const int64_t cap = static_cast<int64_t>(cus) * MI355_RMS_STREAM_BLOCKS_PER_CU;
    if (p.rows >= MI355_RMS_SMALL_ROWS && p.rows > cap)
      return launch_rms(rmsnorm_block_stream<TX, TW, TY, VPL, MI355_RMS_STREAM_ROWS, ADD>, cap, block, p, s);
  }
  const bool multi = p.rows >= MI355_RMS_SMALL_ROWS && MI355_RMS_BLOCK_ROWS > 1;
  constexpr int R = MI355_RMS_BLOCK_ROWS > 1 ? MI355_RMS_BLOCK_ROWS : 1;
  const int64_t per_block = multi ? R : 1;
  int64_t grid = (p.rows + per_block - 1) / per_block;
  if (MI355_RMS_BLOCKS_PER_CU > 0 && grid > static_cast<int64_t>(cus) * MI355_RMS_BLOCKS_PER_CU)
    grid = static_cast<int64_t>(cus) * MI355_RMS_BLOCKS_PER_CU;
  if (grid > 0x7fffffff) grid = 0x7fffffff;
  if (multi) return launch_rms(rmsnorm_block_rows<TX, TW, TY, VPL, R, ADD>, grid, block, p, s);
  return launch_rms(rmsnorm_block_rows<TX, TW, TY, VPL, 1, ADD>, grid, block, p, s);
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_block(const RmsParams& p, hipStream_t s, int cus, int waves, int vpl) {
  const int block = 64 * waves;
#define MI355_BLOCK_CASE(V) return rms_block_rows<TX, TW, TY, V, ADD>(p, s, cus, block)
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
  return rms_block<TX, TW, TY, ADD>(p, s, cus, waves, vpl);
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
