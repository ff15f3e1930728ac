// C ABI entry points (include/mi355_fused.h): argument validation, the
// per-thread error message and the per-device CU-count cache.  Kernels and
// their launchers live in rmsnorm.hip, silu_mul.hip, gate_up_silu.hip,
// w8a16.hip and linear16.hip.
#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "common.h"

#define MI355_EXPORT extern "C" __attribute__((visibility("default")))

namespace mi355 {

int rmsnorm_launch(const void* x, const void* w, void* y, int64_t rows, int n, int64_t xs,
                   int64_t ys, float eps, int x_dtype, int w_dtype, int y_dtype,
                   hipStream_t stream);
int add_rmsnorm_launch(const void* x, const void* r, const void* w, void* y, void* ro, int64_t rows, int n,
                       int64_t xs, int64_t rs, int64_t ys, int64_t ros, float eps, int x_dtype, int w_dtype,
                       int y_dtype, hipStream_t stream);
int silu_mul_launch(const void* gate, const void* up, void* out, int64_t numel, int in_dtype,
                    int out_dtype, hipStream_t stream);
int gate_up_silu_launch(const void* x, const void* wg, const void* wu, void* out, int rows, int k, int n_out,
                        int64_t xs, int64_t ws, int64_t os, int dtype, int out_dtype, hipStream_t stream);

int w8a16_launch(const void* x, const void* q, const void* scale, const void* bias, void* out, int rows, int k,
                 int n, int64_t xs, int64_t qs, int64_t os, int x_dtype, int scale_dtype, int bias_dtype,
                 int out_dtype, hipStream_t stream);
int quantize_int8_launch(const void* w, void* q, void* scale, int64_t n, int k, int64_t ws, int64_t qs, int w_dtype,
                         hipStream_t stream);
int linear16_launch(const void* x, const void* w, const void* bias, void* out, int rows, int k, int n, int64_t xs,
                    int64_t ws, int64_t os, int dtype, int bias_dtype, int out_dtype, hipStream_t stream);
int gate_up_silu_w8a16_launch(const void* x, const void* qg, const void* qu, const void* sg, const void* su, void* out,
                              int rows, int k, int n, int64_t xs, int64_t qs, int64_t os, int x_dtype,
                              int scale_dtype, int out_dtype, hipStream_t stream);

namespace {
thread_local char g_error[512] = "";
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

bool valid_dtype(int d) { return d == MI355_F32 || d == MI355_F16 || d == MI355_BF16; }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int compute_units(int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = g_cu_count[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *out = c;
      return MI355_OK;
    }
  }
  int c = 0;
  e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_status(e, "hipDeviceGetAttribute(MultiprocessorCount)");
  if (c < 1) c = 1;
  if (dev >= 0 && dev < kMaxDevices) g_cu_count[dev].store(c, std::memory_order_relaxed);
  *out = c;
  return MI355_OK;
}

}  // namespace mi355

using mi355::set_error;
using mi355::valid_dtype;

MI355_EXPORT int mi355_abi_version(void) { return MI355_ABI_VERSION; }

MI355_EXPORT const char* mi355_last_error(void) { return mi355::g_error; }

namespace {

// Shared argument checks of the two RMSNorm entry points; `strides` are the
// row strides of the row-shaped operands, `ptrs` every pointer.  Returns
// MI355_OK (and *noop for rows == 0) or an error code with the message set.
int check_rows(const char* fn, int64_t rows, int64_t n, const int64_t* strides, int nstrides,
               const void* const* ptrs, int nptrs, int x_dtype, int w_dtype, int y_dtype, bool* noop) {
  *noop = false;
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype) || !valid_dtype(y_dtype)) {
    set_error("%s: unknown dtype code (x=%d, w=%d, y=%d)", fn, x_dtype, w_dtype, y_dtype);
    return MI355_ERR_INVALID;
  }
  if (y_dtype != x_dtype && y_dtype != MI355_F32) {
    set_error("%s: y dtype must equal x dtype or be fp32 (x=%d, y=%d)", fn, x_dtype, y_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows < 0) {
    set_error("%s: rows must be >= 0 (got %lld)", fn, static_cast<long long>(rows));
    return MI355_ERR_INVALID;
  }
  if (n < 1 || n > 0x7fffffff) {
    set_error("%s: n must be in [1, 2^31) (got %lld)", fn, static_cast<long long>(n));
    return MI355_ERR_INVALID;
  }
  if (rows == 0) {
    *noop = true;
    return MI355_OK;
  }
  for (int i = 0; i < nptrs; ++i) {
    if (ptrs[i] == nullptr) {
      set_error("%s: null pointer (argument %d)", fn, i);
      return MI355_ERR_INVALID;
    }
  }
  for (int i = 0; i < nstrides; ++i) {
    if (strides[i] < n) {
      set_error("%s: row strides must be >= n (stride %lld, n=%lld)", fn, static_cast<long long>(strides[i]),
                static_cast<long long>(n));
      return MI355_ERR_INVALID;
    }
    if (rows - 1 > (INT64_MAX - n) / strides[i]) {
      set_error("%s: rows * stride overflows int64", fn);
      return MI355_ERR_INVALID;
    }
  }
  return MI355_OK;
}

}  // namespace

MI355_EXPORT int mi355_rmsnorm_fwd(const void* x, const void* weight, void* y, int64_t rows,
                                   int64_t n, int64_t x_row_stride, int64_t y_row_stride,
                                   float eps, int x_dtype, int w_dtype, int y_dtype,
                                   void* stream) {
  mi355::g_error[0] = '\0';
  const int64_t strides[] = {x_row_stride, y_row_stride};
  const void* const ptrs[] = {x, weight, y};
  bool noop = false;
  const int st = check_rows("mi355_rmsnorm_fwd", rows, n, strides, 2, ptrs, 3, x_dtype, w_dtype, y_dtype, &noop);
  if (st != MI355_OK || noop) return st;
  return mi355::rmsnorm_launch(x, weight, y, rows, static_cast<int>(n), x_row_stride, y_row_stride,
                               eps, x_dtype, w_dtype, y_dtype, static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight, void* y,
                                       void* residual_out, int64_t rows, int64_t n, int64_t x_row_stride,
                                       int64_t residual_row_stride, int64_t y_row_stride,
                                       int64_t residual_out_row_stride, float eps, int x_dtype, int w_dtype,
                                       int y_dtype, void* stream) {
  mi355::g_error[0] = '\0';
  const int64_t strides[] = {x_row_stride, residual_row_stride, y_row_stride, residual_out_row_stride};
  const void* const ptrs[] = {x, residual, weight, y, residual_out};
  bool noop = false;
  const int st =
      check_rows("mi355_add_rmsnorm_fwd", rows, n, strides, 4, ptrs, 5, x_dtype, w_dtype, y_dtype, &noop);
  if (st != MI355_OK || noop) return st;
  return mi355::add_rmsnorm_launch(x, residual, weight, y, residual_out, rows, static_cast<int>(n),
                                   x_row_stride, residual_row_stride, y_row_stride, residual_out_row_stride, eps,
                                   x_dtype, w_dtype, y_dtype, static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_silu_mul_fwd(const void* gate, const void* up, void* out, int64_t numel,
                                    int in_dtype, int out_dtype, void* stream) {
  mi355::g_error[0] = '\0';
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype)) {
    set_error("mi355_silu_mul_fwd: unknown dtype code (in=%d, out=%d)", in_dtype, out_dtype);
    return MI355_ERR_INVALID;
  }
  if (out_dtype != in_dtype && out_dtype != MI355_F32) {
    set_error("mi355_silu_mul_fwd: out dtype must equal in dtype or be fp32 (in=%d, out=%d)",
              in_dtype, out_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  if (numel < 0) {
    set_error("mi355_silu_mul_fwd: numel must be >= 0 (got %lld)", static_cast<long long>(numel));
    return MI355_ERR_INVALID;
  }
  if (numel == 0) return MI355_OK;
  if (gate == nullptr || up == nullptr || out == nullptr) {
    set_error("mi355_silu_mul_fwd: null pointer (gate=%p, up=%p, out=%p)", gate, up, out);
    return MI355_ERR_INVALID;
  }
  return mi355::silu_mul_launch(gate, up, out, numel, in_dtype, out_dtype,
                                static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_gate_up_silu_fwd(const void* x, const void* w_gate, const void* w_up, void* out,
                                        int64_t rows, int64_t k, int64_t n_out, int64_t x_row_stride,
                                        int64_t w_row_stride, int64_t out_row_stride, int dtype, int out_dtype,
                                        void* stream) {
  static const char* fn = "mi355_gate_up_silu_fwd";
  mi355::g_error[0] = '\0';
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) {
    set_error("%s: unknown dtype code (in=%d, out=%d)", fn, dtype, out_dtype);
    return MI355_ERR_INVALID;
  }
  if (dtype == MI355_F32) {
    set_error("%s: x and the weights must be fp16 or bf16 (MFMA operands)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (out_dtype != dtype && out_dtype != MI355_F32) {
    set_error("%s: out dtype must equal the input dtype or be fp32 (in=%d, out=%d)", fn, dtype, out_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows < 0 || n_out < 0 || k < 1) {
    set_error("%s: need rows >= 0, n_out >= 0, k >= 1 (got %lld, %lld, %lld)", fn, static_cast<long long>(rows),
              static_cast<long long>(n_out), static_cast<long long>(k));
    return MI355_ERR_INVALID;
  }
  if (x_row_stride < k || w_row_stride < k || out_row_stride < n_out) {
    set_error("%s: row strides must be >= k (x, w) and >= n_out (out)", fn);
    return MI355_ERR_INVALID;
  }
  if (rows == 0 || n_out == 0) return MI355_OK;
  if (x == nullptr || w_gate == nullptr || w_up == nullptr || out == nullptr) {
    set_error("%s: null pointer", fn);
    return MI355_ERR_INVALID;
  }
  // 16-byte operand loads: k, the x / weight row strides and the base
  // pointers must be multiples of 8 elements / 16 bytes.
  if (k % 8 != 0 || x_row_stride % 8 != 0 || w_row_stride % 8 != 0 || !mi355::aligned16(x) ||
      !mi355::aligned16(w_gate) || !mi355::aligned16(w_up)) {
    set_error("%s: k, the x and weight row strides must be multiples of 8 and x, w_gate, w_up 16-byte aligned", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  // Buffer descriptors cover at most 32 weight rows and 32 rows of x
  // (< 2^31 bytes); the grid holds ceil(n_out / 32) or more x ceil(rows / 32)
  // workgroups.
  if (w_row_stride >= (int64_t{1} << 24) || x_row_stride >= (int64_t{1} << 24) ||
      n_out > 0x7fffffff - 31 || rows > int64_t{65535} * 32) {
    set_error("%s: size beyond the kernel's limits (row strides < 2^24, n_out < 2^31 - 31, "
              "rows <= 2097120)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows - 1 > (INT64_MAX - n_out) / out_row_stride) {
    set_error("%s: rows * out_row_stride overflows int64", fn);
    return MI355_ERR_INVALID;
  }
  return mi355::gate_up_silu_launch(x, w_gate, w_up, out, static_cast<int>(rows), static_cast<int>(k),
                                    static_cast<int>(n_out), x_row_stride, w_row_stride, out_row_stride, dtype,
                                    out_dtype, static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_w8a16_linear_fwd(const void* x, const void* w_q, const void* scale, const void* bias,
                                        void* out, int64_t rows, int64_t k, int64_t n, int64_t x_row_stride,
                                        int64_t w_row_stride, int64_t out_row_stride, int x_dtype, int scale_dtype,
                                        int bias_dtype, int out_dtype, void* stream) {
  static const char* fn = "mi355_w8a16_linear_fwd";
  mi355::g_error[0] = '\0';
  if (!valid_dtype(x_dtype) || !valid_dtype(scale_dtype) || !valid_dtype(out_dtype) ||
      (bias != nullptr && !valid_dtype(bias_dtype))) {
    set_error("%s: unknown dtype code (x=%d, scale=%d, bias=%d, out=%d)", fn, x_dtype, scale_dtype, bias_dtype,
              out_dtype);
    return MI355_ERR_INVALID;
  }
  if (x_dtype == MI355_F32) {
    set_error("%s: x must be fp16 or bf16 (MFMA operand)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (out_dtype != x_dtype && out_dtype != MI355_F32) {
    set_error("%s: out dtype must equal x dtype or be fp32 (x=%d, out=%d)", fn, x_dtype, out_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows < 0 || n < 0 || k < 1) {
    set_error("%s: need rows >= 0, n >= 0, k >= 1 (got %lld, %lld, %lld)", fn, static_cast<long long>(rows),
              static_cast<long long>(n), static_cast<long long>(k));
    return MI355_ERR_INVALID;
  }
  if (x_row_stride < k || w_row_stride < k || out_row_stride < n) {
    set_error("%s: row strides must be >= k (x, w_q) and >= n (out)", fn);
    return MI355_ERR_INVALID;
  }
  if (rows == 0 || n == 0) return MI355_OK;
  if (x == nullptr || w_q == nullptr || scale == nullptr || out == nullptr) {
    set_error("%s: null pointer", fn);
    return MI355_ERR_INVALID;
  }
  // Buffer descriptors span at most 128 rows of x or of w_q (< 2^32 bytes);
  // grids hold ceil(n / 128) x ceil(rows / 64) workgroups or more.
  if (x_row_stride >= (int64_t{1} << 23) || w_row_stride >= (int64_t{1} << 24) || n > 0x7fffffff - 128 ||
      rows > int64_t{65535} * 64) {
    set_error("%s: size beyond the kernel's limits (x_row_stride < 2^23, w_row_stride < 2^24, n < 2^31 - 128, "
              "rows <= 4194240)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (n * ((rows + 3) / 4) > int64_t{0x7fffffff} * 4) {
    set_error("%s: n * rows too large for one launch", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows - 1 > (INT64_MAX - n) / out_row_stride) {
    set_error("%s: rows * out_row_stride overflows int64", fn);
    return MI355_ERR_INVALID;
  }
  return mi355::w8a16_launch(x, w_q, scale, bias, out, static_cast<int>(rows), static_cast<int>(k),
                             static_cast<int>(n), x_row_stride, w_row_stride, out_row_stride, x_dtype, scale_dtype,
                             bias_dtype, out_dtype, static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_gate_up_silu_w8a16_fwd(const void* x, const void* wq_gate, const void* wq_up,
                                              const void* scale_gate, const void* scale_up, void* out, int64_t rows,
                                              int64_t k, int64_t n_out, int64_t x_row_stride, int64_t w_row_stride,
                                              int64_t out_row_stride, int x_dtype, int scale_dtype, int out_dtype,
                                              void* stream) {
  static const char* fn = "mi355_gate_up_silu_w8a16_fwd";
  mi355::g_error[0] = '\0';
  if (!valid_dtype(x_dtype) || !valid_dtype(scale_dtype) || !valid_dtype(out_dtype)) {
    set_error("%s: unknown dtype code (x=%d, scale=%d, out=%d)", fn, x_dtype, scale_dtype, out_dtype);
    return MI355_ERR_INVALID;
  }
  if (x_dtype == MI355_F32) {
    set_error("%s: x must be fp16 or bf16 (MFMA operand)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (out_dtype != x_dtype && out_dtype != MI355_F32) {
    set_error("%s: out dtype must equal x dtype or be fp32 (x=%d, out=%d)", fn, x_dtype, out_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows < 0 || n_out < 0 || k < 1) {
    set_error("%s: need rows >= 0, n_out >= 0, k >= 1 (got %lld, %lld, %lld)", fn, static_cast<long long>(rows),
              static_cast<long long>(n_out), static_cast<long long>(k));
    return MI355_ERR_INVALID;
  }
  if (x_row_stride < k || w_row_stride < k || out_row_stride < n_out) {
    set_error("%s: row strides must be >= k (x, weights) and >= n_out (out)", fn);
    return MI355_ERR_INVALID;
  }
  if (rows == 0 || n_out == 0) return MI355_OK;
  if (x == nullptr || wq_gate == nullptr || wq_up == nullptr || scale_gate == nullptr || scale_up == nullptr ||
      out == nullptr) {
    set_error("%s: null pointer", fn);
    return MI355_ERR_INVALID;
  }
  // the W8A16 kernels' limits
  if (x_row_stride >= (int64_t{1} << 23) || w_row_stride >= (int64_t{1} << 24) || n_out > 0x7fffffff - 128 ||
      rows > int64_t{65535} * 64) {
    set_error("%s: size beyond the kernel's limits (x_row_stride < 2^23, w_row_stride < 2^24, n_out < 2^31 - 128, "
              "rows <= 4194240)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (n_out * ((rows + 3) / 4) > int64_t{0x7fffffff} * 4) {
    set_error("%s: n_out * rows too large for one launch", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows - 1 > (INT64_MAX - n_out) / out_row_stride) {
    set_error("%s: rows * out_row_stride overflows int64", fn);
    return MI355_ERR_INVALID;
  }
  return mi355::gate_up_silu_w8a16_launch(x, wq_gate, wq_up, scale_gate, scale_up, out, static_cast<int>(rows),
                                          static_cast<int>(k), static_cast<int>(n_out), x_row_stride, w_row_stride,
                                          out_row_stride, x_dtype, scale_dtype, out_dtype,
                                          static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_quantize_int8_fwd(const void* w, void* w_q, void* scale, int64_t n, int64_t k,
                                         int64_t w_row_stride, int64_t q_row_stride, int w_dtype, void* stream) {
  static const char* fn = "mi355_quantize_int8_fwd";
  mi355::g_error[0] = '\0';
  if (!valid_dtype(w_dtype)) {
    set_error("%s: unknown dtype code %d", fn, w_dtype);
    return MI355_ERR_INVALID;
  }
  if (n < 0 || k < 1 || k > 0x7fffffff) {
    set_error("%s: need n >= 0 and 1 <= k < 2^31 (got %lld, %lld)", fn, static_cast<long long>(n),
              static_cast<long long>(k));
    return MI355_ERR_INVALID;
  }
  if (w_row_stride < k || q_row_stride < k) {
    set_error("%s: row strides must be >= k", fn);
    return MI355_ERR_INVALID;
  }
  if (n == 0) return MI355_OK;
  if (w == nullptr || w_q == nullptr || scale == nullptr) {
    set_error("%s: null pointer", fn);
    return MI355_ERR_INVALID;
  }
  if ((n + 3) / 4 > 0x7fffffff || n - 1 > (INT64_MAX - k) / (w_row_stride > q_row_stride ? w_row_stride : q_row_stride)) {
    set_error("%s: n too large", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  return mi355::quantize_int8_launch(w, w_q, scale, n, static_cast<int>(k), w_row_stride, q_row_stride, w_dtype,
                                     static_cast<hipStream_t>(stream));
}

MI355_EXPORT int mi355_linear16_fwd(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
                                    int64_t k, int64_t n, int64_t x_row_stride, int64_t w_row_stride,
                                    int64_t out_row_stride, int dtype, int bias_dtype, int out_dtype, void* stream) {
  static const char* fn = "mi355_linear16_fwd";
  mi355::g_error[0] = '\0';
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype) || (bias != nullptr && !valid_dtype(bias_dtype))) {
    set_error("%s: unknown dtype code (in=%d, bias=%d, out=%d)", fn, dtype, bias_dtype, out_dtype);
    return MI355_ERR_INVALID;
  }
  if (dtype == MI355_F32) {
    set_error("%s: x and weight must be fp16 or bf16 (MFMA operands)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (out_dtype != dtype && out_dtype != MI355_F32) {
    set_error("%s: out dtype must equal the input dtype or be fp32 (in=%d, out=%d)", fn, dtype, out_dtype);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows < 0 || n < 0 || k < 1) {
    set_error("%s: need rows >= 0, n >= 0, k >= 1 (got %lld, %lld, %lld)", fn, static_cast<long long>(rows),
              static_cast<long long>(n), static_cast<long long>(k));
    return MI355_ERR_INVALID;
  }
  if (x_row_stride < k || w_row_stride < k || out_row_stride < n) {
    set_error("%s: row strides must be >= k (x, weight) and >= n (out)", fn);
    return MI355_ERR_INVALID;
  }
  if (rows == 0 || n == 0) return MI355_OK;
  if (x == nullptr || weight == nullptr || out == nullptr) {
    set_error("%s: null pointer", fn);
    return MI355_ERR_INVALID;
  }
  // Buffer descriptors span at most 256 rows of x or of the weights (< 2^32
  // bytes); grids hold ceil(n / 8) x ceil(rows / 32) workgroups or more.
  if (x_row_stride >= (int64_t{1} << 22) || w_row_stride >= (int64_t{1} << 22) || n > 0x7fffffff - 256 ||
      rows > int64_t{65535} * 32) {
    set_error("%s: size beyond the kernel's limits (row strides < 2^22, n < 2^31 - 256, rows <= 2097120)", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (n * ((rows + 3) / 4) > int64_t{0x7fffffff} * 4) {
    set_error("%s: n * rows too large for one launch", fn);
    return MI355_ERR_UNSUPPORTED;
  }
  if (rows - 1 > (INT64_MAX - n) / out_row_stride) {
    set_error("%s: rows * out_row_stride overflows int64", fn);
    return MI355_ERR_INVALID;
  }
  return mi355::linear16_launch(x, weight, bias, out, static_cast<int>(rows), static_cast<int>(k),
                                static_cast<int>(n), x_row_stride, w_row_stride, out_row_stride, dtype, bias_dtype,
                                out_dtype, static_cast<hipStream_t>(stream));
}
