/*
 * mi355_fused.h -- C ABI of the MI355X (gfx950) fused RMSNorm and SiLU-and-mul
 * kernels, the fused gate/up projections, the weight-only int8 (W8A16)
 * linear with its quantiser, and the 16-bit linear of the MLP's down
 * projection.
 *
 * The reference has no FFI: its boundary is a pair of Python launchers that
 * hand torch tensors to Triton kernels.  Each entry point below replaces one of
 * those launches with a plain-pointer call, so a host binding (ctypes, a torch
 * extension, C++) can drive the HIP kernels without any torch type crossing the
 * boundary.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HBM).  Sizes are element counts.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default
 *     stream).  Work is enqueued on that stream only: no allocation, no host
 *     synchronisation, no memset, so every call may be recorded into a HIP
 *     graph.
 *   - The return value is MI355_OK (0) or a negative MI355_ERR_* code; the
 *     message for the most recent failure on the calling thread is returned by
 *     mi355_last_error().  Nothing throws across the ABI.
 *   - Calls are reentrant; the library holds no locks.  A call only reads its
 *     inputs and writes its outputs; outputs must not overlap inputs unless
 *     the pointers are identical and the strides match (in-place use).
 */
#ifndef MI355_FUSED_H
#define MI355_FUSED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355_ABI_VERSION 1

/* Element types understood by the kernels (storage type; arithmetic is fp32). */
enum mi355_dtype {
  MI355_F32 = 0,
  MI355_F16 = 1,
  MI355_BF16 = 2
};

/* Status codes. */
enum mi355_status {
  MI355_OK = 0,
  MI355_ERR_INVALID = -1,     /* bad pointer, size, stride or dtype code */
  MI355_ERR_UNSUPPORTED = -2, /* valid request the library cannot serve */
  MI355_ERR_HIP = -3          /* the HIP runtime reported an error */
};

/* Version of this ABI; callers check it equals MI355_ABI_VERSION. */
int mi355_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* mi355_last_error(void);

/*
 * RMSNorm over the last dimension, one row at a time:
 *   var_r  = (sum_j x[r,j]^2) / n            (fp32 accumulation)
 *   rstd_r = 1 / sqrt(var_r + eps)
 *   y[r,j] = (x[r,j] * rstd_r) * w[j]        (fp32, rounded once to y_dtype)
 *
 * Replaces the launch of `_rmsnorm_fwd_kernel` in the reference's
 * `fused_rmsnorm` (src/kernels/fused_rmsnorm_triton.py:52-71, kernel body
 * :23-49).  The reference's launcher reuses x's row stride for the output
 * (:66-68) and makes x contiguous first (:60); here both row strides are
 * explicit, so a row-strided view needs no copy.
 *
 *   x       [rows, x_row_stride] elements of x_dtype; row r starts at
 *           x + r * x_row_stride and its n elements are contiguous.
 *   weight  [n] elements of w_dtype, contiguous.
 *   y       [rows, y_row_stride] elements of y_dtype.
 *   rows    >= 0 (0 is a no-op), n >= 1, both row strides >= n.
 *   y_dtype must equal x_dtype or be MI355_F32 (the fp32 value before the
 *   final rounding, used to check the kernel's arithmetic on its own).
 */
int mi355_rmsnorm_fwd(const void* x, const void* weight, void* y,
                      int64_t rows, int64_t n,
                      int64_t x_row_stride, int64_t y_row_stride,
                      float eps,
                      int x_dtype, int w_dtype, int y_dtype,
                      void* stream);

/*
 * Residual add fused with RMSNorm, per row:
 *   h[r,j]            = x[r,j] + residual[r,j]   (fp32 add, rounded to x_dtype)
 *   residual_out[r,j] = h[r,j]
 *   y[r,j]            = RMSNorm(h)[r,j]          (as mi355_rmsnorm_fwd)
 *
 * The reference has no kernel for this; it is the "fused RMSNorm + residual"
 * its design plans (docs/architecture-cuda.md:94) for the decoder's
 * `hidden = residual + attn_out; normed = post_attention_layernorm(hidden)`
 * (the HF Qwen2 decoder layer, and src/engine/paged_engine.py:138-141).  h is
 * rounded exactly where the unfused add rounds it, so the results equal the
 * add followed by mi355_rmsnorm_fwd bit for bit, in one pass over the rows:
 * read x and residual, write residual_out and y.
 *
 *   x, residual, residual_out: x_dtype, [rows, *_row_stride], rows contiguous.
 *   weight [n] of w_dtype; y [rows, y_row_stride] of y_dtype (x_dtype or fp32).
 *   residual_out may be residual and y may be x (in place, same strides);
 *   y must not overlap residual or residual_out.
 */
int mi355_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight,
                          void* y, void* residual_out,
                          int64_t rows, int64_t n,
                          int64_t x_row_stride, int64_t residual_row_stride,
                          int64_t y_row_stride, int64_t residual_out_row_stride,
                          float eps,
                          int x_dtype, int w_dtype, int y_dtype,
                          void* stream);

/*
 * SiLU-and-mul, the activation step of a SwiGLU MLP, over flat memory:
 *   out[i] = (g * sigmoid(g)) * u,  g = gate[i], u = up[i]   (fp32, rounded once)
 *
 * Replaces the launch of `_silu_mul_fwd_kernel` in the reference's
 * `fused_silu_mul` (src/kernels/fused_swiglu_triton.py:39-53, kernel body
 * :20-36).  gate, up and out are `numel` contiguous elements; gate and up
 * share in_dtype; out_dtype must equal in_dtype or be MI355_F32.
 */
int mi355_silu_mul_fwd(const void* gate, const void* up, void* out,
                       int64_t numel, int in_dtype, int out_dtype,
                       void* stream);

/*
 * Gate/up projections fused with SiLU-and-mul, for decode-sized batches:
 *   g[m,n]   = sum_k x[m,k] * w_gate[n,k]     (fp32 accumulation, MFMA)
 *   u[m,n]   = sum_k x[m,k] * w_up[n,k]
 *   out[m,n] = (g * sigmoid(g)) * u           (fp32, rounded once to out_dtype)
 *
 * The reference's FusedMLP (src/engine/fused_norm_activation_patch.py:60-64)
 * computes `fused_silu_mul(gate_proj(x), up_proj(x))`: two GEMMs whose
 * results are rounded to x's dtype, written to HBM and read back by the
 * SiLU-and-mul launch this call also replaces (src/kernels/
 * fused_swiglu_triton.py:39-53).  This entry point is the "fused activation
 * with the up/gate projections" its design plans (docs/architecture-cuda.md:94):
 * g and u never leave registers and are not rounded before the activation,
 * so results differ from the unfused chain by that intermediate rounding
 * (they are closer to the exact value).  Weights use nn.Linear's layout,
 * [n_out, k] row-major, as in HF's gate_proj / up_proj.
 *
 * rows <= 32 stream the weights once at HBM bandwidth; more rows run an
 * LDS-tiled MFMA GEMM over both weight matrices with SiLU-and-mul in its
 * epilogue (32-row weight-streaming tiles when a row stride is too large for
 * the tiled kernel's buffer descriptors).
 *
 *   x        [rows, x_row_stride] of dtype, 16-byte aligned.
 *   w_gate, w_up  [n_out, w_row_stride] of dtype, 16-byte aligned.
 *   out      [rows, out_row_stride] of out_dtype.
 *   dtype    MI355_F16 or MI355_BF16; out_dtype = dtype or MI355_F32.
 *   k, x_row_stride and w_row_stride are multiples of 8 (MI355_ERR_UNSUPPORTED
 *   otherwise); strides >= k (x, w) and >= n_out (out).  rows == 0 or
 *   n_out == 0 is a no-op.  Limits: x_row_stride and w_row_stride < 2^24,
 *   rows <= 2097120.  out must not overlap the inputs.
 */
int mi355_gate_up_silu_fwd(const void* x, const void* w_gate, const void* w_up, void* out,
                           int64_t rows, int64_t k, int64_t n_out,
                           int64_t x_row_stride, int64_t w_row_stride, int64_t out_row_stride,
                           int dtype, int out_dtype,
                           void* stream);

/*
 * Weight-only int8 linear (W8A16), per output feature n and row m:
 *   acc[m,n] = sum_k x[m,k] * w_q[n,k]           (fp32 accumulation; int8 and
 *                                                 16-bit x meet exactly in fp16/bf16)
 *   out[m,n] = acc[m,n] * scale[n] + bias[n]     (one fma in fp32, rounded once)
 *
 * Replaces the launch of `_w8a16_matmul_kernel` in the reference's
 * `w8a16_linear` (src/kernels/w8a16_matmul_triton.py:102-134, kernel body
 * :39-86), which QuantizedLinearInt8.forward calls (src/quantization/
 * int8.py:62-63).  The scale is applied once to the accumulator, as there.
 *
 *   x       [rows, x_row_stride] of x_dtype (MI355_F16 or MI355_BF16).
 *   w_q     [n, w_row_stride] int8, nn.Linear's layout (out_features rows).
 *   scale   [n] of scale_dtype (the reference's float32; fp16/bf16 accepted).
 *   bias    [n] of bias_dtype, or NULL (then bias_dtype is ignored).
 *   out     [rows, out_row_stride] of out_dtype = x_dtype or MI355_F32.
 *   rows >= 0, k >= 1, n >= 0 (rows == 0 or n == 0 is a no-op); strides >= k
 *   (x, w_q) and >= n (out).  Any alignment and k are served; the fast kernels
 *   need k and w_row_stride multiples of 16, x_row_stride a multiple of 8 and
 *   16-byte aligned x and w_q.  Limits: x_row_stride < 2^23, w_row_stride <
 *   2^24, n < 2^31 - 128, rows <= 4194240.  out must not overlap the inputs.
 *   Calls with the same shapes give identical bits (fixed summation order).
 */
int mi355_w8a16_linear_fwd(const void* x, const void* w_q, const void* scale, const void* bias, void* out,
                           int64_t rows, int64_t k, int64_t n,
                           int64_t x_row_stride, int64_t w_row_stride, int64_t out_row_stride,
                           int x_dtype, int scale_dtype, int bias_dtype, int out_dtype,
                           void* stream);

/*
 * Int8 gate/up projections fused with SiLU-and-mul (W8A16 weights), per row
 * m and output feature n:
 *   g[m,n] = (sum_k x[m,k] * wq_gate[n,k]) * scale_gate[n]     (fp32 sums)
 *   u[m,n] = (sum_k x[m,k] * wq_up[n,k])   * scale_up[n]
 *   out[m,n] = round(g * sigmoid(g) * u)                       (fp32, one rounding)
 *
 * No counterpart in the reference: its quantised model runs
 * QuantizedLinearInt8 gate_proj and up_proj (two `w8a16_linear` launches,
 * src/quantization/int8.py:62-63, each rounding to x's dtype) and then the
 * SiLU-and-mul kernel (src/engine/fused_norm_activation_patch.py:60-64).
 * This entry point is that chain as one kernel, without the intermediate
 * roundings -- the int8 form of mi355_gate_up_silu_fwd.  Decode rows (<= 32)
 * stream both int8 matrices once at HBM bandwidth; more rows run the tiled
 * MFMA GEMM.
 *
 *   x        [rows, x_row_stride] of x_dtype (MI355_F16 or MI355_BF16).
 *   wq_gate, wq_up  [n_out, w_row_stride] int8 (QuantizedLinearInt8.weight_q).
 *   scale_gate, scale_up  [n_out] of scale_dtype (the quantiser's fp32).
 *   out      [rows, out_row_stride] of out_dtype = x_dtype or MI355_F32.
 *   Same shape rules, alignment preferences and limits as
 *   mi355_w8a16_linear_fwd (any k and alignment are served; no bias).
 */
int mi355_gate_up_silu_w8a16_fwd(const void* x, const void* wq_gate, const void* wq_up,
                                 const void* scale_gate, const void* scale_up, void* out,
                                 int64_t rows, int64_t k, int64_t n_out,
                                 int64_t x_row_stride, int64_t w_row_stride, int64_t out_row_stride,
                                 int x_dtype, int scale_dtype, int out_dtype,
                                 void* stream);

/*
 * Per-output-channel symmetric int8 quantisation of a weight matrix, per row n:
 *   amax     = max_k |w[n,k]|
 *   scale[n] = max(amax / 127, 1e-8)                     (fp32, IEEE division)
 *   w_q[n,k] = clamp(round_half_even(w[n,k] / scale[n]), -127, 127)
 *
 * The arithmetic of the reference's QuantizedLinearInt8.from_linear
 * (src/quantization/int8.py:45-50), bit for bit: w is widened to fp32
 * (`linear.weight.detach().float()`), the scale is clamped below at 1e-8 and
 * the quotient rounded with torch.round's ties-to-even.
 *
 *   w      [n, w_row_stride] of w_dtype (fp32, fp16 or bf16).
 *   w_q    [n, q_row_stride] int8 (output).   scale  [n] fp32 (output).
 *   n >= 0 (0 is a no-op), 1 <= k < 2^31, strides >= k.  Rows holding NaN or
 *   Inf get unspecified codes (the reference's are undefined there too).
 */
int mi355_quantize_int8_fwd(const void* w, void* w_q, void* scale,
                            int64_t n, int64_t k, int64_t w_row_stride, int64_t q_row_stride,
                            int w_dtype, void* stream);

/*
 * 16-bit linear (nn.Linear's forward with fp16 / bf16 weights), per row m
 * and output feature n:
 *   acc[m,n] = sum_k x[m,k] * weight[n,k]     (fp32 accumulation, MFMA)
 *   out[m,n] = acc[m,n] + bias[n]             (fp32, rounded once to out_dtype)
 *
 * Replaces the down projection of the reference's FusedMLP,
 * `self.down_proj(activated)` (src/engine/fused_norm_activation_patch.py:64),
 * an nn.Linear that torch runs on hipBLASLt.  At decode batch sizes that call
 * streams the whole weight matrix for a few rows; rows <= 32 here (64 on
 * outputs narrower than 128 64-column tiles) read every weight byte once at
 * HBM bandwidth on MFMA.  More rows run the LDS-tiled MFMA GEMM.  The fp32 sums
 * run in this library's own order, so results may differ from hipBLASLt's
 * in the last output bit.
 *
 *   x       [rows, x_row_stride] of dtype (MI355_F16 or MI355_BF16).
 *   weight  [n, w_row_stride] of dtype, nn.Linear's layout.
 *   bias    [n] of bias_dtype, or NULL (then bias_dtype is ignored).
 *   out     [rows, out_row_stride] of out_dtype = dtype or MI355_F32.
 *   rows >= 0, k >= 1, n >= 0 (rows == 0 or n == 0 is a no-op); strides >= k
 *   (x, weight) and >= n (out).  Any alignment and k are served; the fast
 *   kernels need k and both input row strides multiples of 8 and 16-byte
 *   aligned x and weight.  Limits: x_row_stride and w_row_stride < 2^22,
 *   n < 2^31 - 256, rows <= 2097120.  out must not overlap the inputs.
 *   Calls with the same shapes give identical bits (fixed summation order).
 */
int mi355_linear16_fwd(const void* x, const void* weight, const void* bias, void* out,
                       int64_t rows, int64_t k, int64_t n,
                       int64_t x_row_stride, int64_t w_row_stride, int64_t out_row_stride,
                       int dtype, int bias_dtype, int out_dtype,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355_FUSED_H */
