// Launcher for the RMSNorm kernels (plain and residual-add fused): picks
// wave-per-row, workgroup-per-row or the generic kernel from the row width,
// alignment and dtype mix, and sizes the grid.  The launch shapes below are
// the ones measured fastest on MI355X (one wave or workgroup per row group,
// a one-shot grid rather than a persistent one).
#include "rmsnorm_kernels.h"

namespace mi355 {
namespace {

// Row counts below this use 64-thread workgroups (one wave each) and one row
// per wave, so small decode batches spread over as many CUs as rows.
constexpr int64_t kSmallRows = 1024;
// Row split: rows needing more than kWaveMaxVpl packets per lane of one wave
// are spread over several waves with at most kTargetVpl packets per lane
// (1536-wide fp16 rows run as 3 packets per lane of one wave, 3584-wide bf16
// rows as 2 packets per lane of 4 waves).
constexpr int kWaveMaxVpl = 4;
constexpr int kTargetVpl = 2;
// Rows each wave of the wave-per-row kernel holds at once, from kSmallRows
// rows up: all their loads are in flight together, behind one reduction.  The
// fused residual add moves twice the bytes of a row and measured 1.06x faster
// with two rows per wave at the 2048 x 1536 fp16 shape; the plain norm is
// fastest with one.
constexpr int kWaveRows = 1;
constexpr int kWaveRowsAdd = 2;

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
int rms_wave_shape(const RmsParams& p, hipStream_t s, int block) {
  const int64_t per_block = static_cast<int64_t>(block / 64) * R;
  int64_t grid = (p.rows + per_block - 1) / per_block;
  if (grid > 0x7fffffff) grid = 0x7fffffff;  // the kernel strides over the rest
  return launch_rms(rmsnorm_wave_rows<TX, TW, TY, VPL, R, ADD>, grid, block, p, s);
}

template <typename TX, typename TW, typename TY, int VPL, bool ADD>
int rms_wave_rows(const RmsParams& p, hipStream_t s) {
  constexpr int R = ADD ? kWaveRowsAdd : kWaveRows;
  if (p.rows < kSmallRows) return rms_wave_shape<TX, TW, TY, VPL, 1, ADD>(p, s, 64);
  return rms_wave_shape<TX, TW, TY, VPL, R, ADD>(p, s, kRmsWaveBlock);
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_wave(const RmsParams& p, hipStream_t s, int vpl) {
  switch (vpl) {
    case 1: return rms_wave_rows<TX, TW, TY, 1, ADD>(p, s);
    case 2: return rms_wave_rows<TX, TW, TY, 2, ADD>(p, s);
    case 3: return rms_wave_rows<TX, TW, TY, 3, ADD>(p, s);
    case 4: return rms_wave_rows<TX, TW, TY, 4, ADD>(p, s);
    default:
      set_error("rmsnorm: internal error, no wave kernel for %d packets per lane", vpl);
      return MI355_ERR_UNSUPPORTED;
  }
}

template <typename TX, typename TW, typename TY, int VPL, bool ADD>
int rms_block_rows(const RmsParams& p, hipStream_t s, int block) {
  int64_t grid = p.rows;
  if (grid > 0x7fffffff) grid = 0x7fffffff;  // the kernel strides over the rest
  return launch_rms(rmsnorm_block_rows<TX, TW, TY, VPL, 1, ADD>, grid, block, p, s);
}

template <typename TX, typename TW, typename TY, bool ADD>
int rms_block(const RmsParams& p, hipStream_t s, int waves, int vpl) {
  const int block = 64 * waves;
  switch (vpl) {
    case 1: return rms_block_rows<TX, TW, TY, 1, ADD>(p, s, block);
    case 2: return rms_block_rows<TX, TW, TY, 2, ADD>(p, s, block);
    case 3: return rms_block_rows<TX, TW, TY, 3, ADD>(p, s, block);
    case 4: return rms_block_rows<TX, TW, TY, 4, ADD>(p, s, block);
    default: return rms_block_rows<TX, TW, TY, 8, ADD>(p, s, block);
  }
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
  if (vpl64 <= kWaveMaxVpl) return rms_wave<TX, TW, TY, ADD>(p, s, vpl64);
  // Spread the row over enough waves (at most 16) for <= kTargetVpl packets
  // per lane, then use the fewest waves for that many packets per lane.
  int waves = (nvec + 64 * kTargetVpl - 1) / (64 * kTargetVpl);
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
