/*
 * fused_oracle.c -- CPU oracle for the fused RMSNorm and SiLU-and-mul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker (or
 * the timed CPU baseline).  No product code path calls it.
 *
 * It restates, in plain C with explicit rounding, the reference's two
 * formulations of each op:
 *
 *   mode ORACLE_TRITON  -- the fused Triton kernels: fp32 arithmetic, ONE
 *       rounding to the output type.
 *       RMSNorm  src/kernels/fused_rmsnorm_triton.py:41-49
 *       SwiGLU   src/kernels/fused_swiglu_triton.py:30-36
 *   mode ORACLE_HF      -- the naive/HF formulas the fused kernels replace:
 *       RMSNorm rounds x*rstd to x's type before the weight multiply
 *       (src/kernels/fused_rmsnorm_triton.py:74-82, identical to HF
 *       Qwen2RMSNorm.forward); SwiGLU rounds silu(g) before "* up"
 *       (src/kernels/fused_swiglu_triton.py:56-59).
 *   *_f64               -- fp64 brute force of the same mathematics.
 *
 * oracle_gate_up_silu restates the MLP's activation input: the gate / up
 * projections of x (nn.Linear weights, [n, k]) followed by SiLU-and-mul, in
 * two modes -- the reference's FusedMLP chain, where each projection is
 * rounded to x's type before the SiLU-and-mul kernel
 * (src/engine/fused_norm_activation_patch.py:60-64), and the fused form
 * without that intermediate rounding.  Projections are summed in fp64
 * (products of 16-bit values are exact there).
 *
 * oracle_w8a16_linear restates the weight-only int8 linear of the
 * reference's quantisation stage: the Triton kernel's order (integer dot
 * product in fp32, then the per-output-channel scale, then the bias,
 * src/kernels/w8a16_matmul_triton.py:64-86) and its dequantise-first
 * reference (:137-149); oracle_quantize_int8 restates the quantiser that
 * produces the int8 weights (src/quantization/int8.py:45-50).
 *
 * oracle_linear16 restates the MLP's down projection, nn.Linear with 16-bit
 * weights (`self.down_proj(activated)`, src/engine/fused_norm_activation_
 * patch.py:64): the dot product of x with the weight row in fp32 (formed
 * order-free from the exact fp64 sum), the bias added in fp32, one rounding.
 *
 * Sum of squares: the reference reduces with tl.sum in fp32 in an order the
 * Triton backend picks (:43).  The oracle accumulates the exact squares in
 * fp64 and rounds the sum to fp32 once, i.e. the order-free fp32 sum; any
 * fp32 reduction order differs from it by a few fp32 ulp, far below one
 * fp16/bf16 ulp of the output.
 *
 * Storage conversions (fp16, bf16 <-> fp32, round-to-nearest-even) are
 * written out here and checked against numpy / torch in tests/.
 *
 * `mutate` != 0 plants a deliberate mistake (see ORACLE_MUT_*); the tests use
 * it to show that the checks pinning this oracle would catch such a mistake.
 * 0 is the faithful restatement.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2 };
enum { ORACLE_TRITON = 0, ORACLE_HF = 1 };

/* planted mistakes, RMSNorm */
enum {
  ORACLE_MUT_RMS_N_MINUS_1 = 1, /* divide the sum of squares by n-1 */
  ORACLE_MUT_RMS_NO_EPS = 2,    /* drop eps */
  ORACLE_MUT_RMS_SQRT = 3,      /* multiply by sqrt(var+eps) instead of its reciprocal */
  ORACLE_MUT_RMS_NO_WEIGHT = 4, /* skip the weight */
  ORACLE_MUT_RMS_W_REVERSED = 5 /* index the weight backwards */
};
/* planted mistakes, SiLU-and-mul */
enum {
  ORACLE_MUT_SILU_SIGN = 1,    /* sigmoid(-g) instead of sigmoid(g) */
  ORACLE_MUT_SILU_SWAP = 2,    /* silu(up) * gate */
  ORACLE_MUT_SILU_NO_UP = 3,   /* drop "* up" */
  ORACLE_MUT_SILU_ROUND2 = 4   /* round silu(g) before "* up" in Triton mode */
};

/* ---------------------------------------------------------------- storage */

static float bits_to_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}
static uint32_t f32_to_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  if (e == 0) {
    /* zero or subnormal: m * 2^-24, exact in fp32 */
    float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (e == 31) return bits_to_f32(sign | 0x7f800000u | (m << 13));
  return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  const uint32_t x = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN, quieted */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {
    /* below 2^-14: fp16 subnormal (or zero).  |f| * 2^24 is exact; round it
     * to the nearest integer, ties to even.  1024 correctly encodes 2^-14. */
    const float t = bits_to_f32(ax) * 16777216.0f;
    uint32_t m = (uint32_t)t;
    const float frac = t - (float)m;
    if (frac > 0.5f || (frac == 0.5f && (m & 1u))) m += 1u;
    return (uint16_t)(sign | m);
  }
  const uint32_t mant = ax & 0x7fffffu;
  uint32_t h = ((((ax >> 23) - 127u + 15u)) << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry into the exponent is correct */
  return (uint16_t)(sign | h);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t x = f32_to_bits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u); /* NaN, quieted */
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

static float load_f(const void* p, int64_t i, int dt) {
  switch (dt) {
    case OR_F16: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    case OR_BF16: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static void store_f(void* p, int64_t i, int dt, float v) {
  switch (dt) {
    case OR_F16: ((uint16_t*)p)[i] = oracle_f32_to_f16(v); break;
    case OR_BF16: ((uint16_t*)p)[i] = oracle_f32_to_bf16(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

/* value of v after a round trip through storage type dt */
static float round_to(float v, int dt) {
  switch (dt) {
    case OR_F16: return oracle_f16_to_f32(oracle_f32_to_f16(v));
    case OR_BF16: return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
    default: return v;
  }
}

static int valid_dt(int d) { return d == OR_F32 || d == OR_F16 || d == OR_BF16; }

/* --------------------------------------------------------------- RMSNorm */

/*
 * y[r, :] for r < rows.  x row r starts at x + r*xs, y row r at y + r*ys.
 *   TRITON (:41-49): var = sum/n; rstd = 1/sqrt(var+eps); y = (x*rstd)*w,
 *                    one rounding to ydt.
 *   HF     (:74-82): h = round_xdt(x*rstd); y = round_ydt(w*h); the caller
 *                    passes ydt = torch's promotion of (w dtype, x dtype).
 * Returns 0, or -1 on a bad argument.
 */
int oracle_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t n, int64_t xs,
                   int64_t ys, float eps, int xdt, int wdt, int ydt, int mode, int mutate) {
  if (!valid_dt(xdt) || !valid_dt(wdt) || !valid_dt(ydt) || n < 1 || rows < 0) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    double ssd = 0.0;
    for (int64_t j = 0; j < n; ++j) {
      const double v = (double)load_f(x, r * xs + j, xdt);
      ssd += v * v;
    }
    const float ss = (float)ssd;
    const float denom = (mutate == ORACLE_MUT_RMS_N_MINUS_1) ? (float)(n - 1) : (float)n;
    const float var = ss / denom;
    const float add = (mutate == ORACLE_MUT_RMS_NO_EPS) ? 0.0f : eps;
    const float rstd = (mutate == ORACLE_MUT_RMS_SQRT) ? sqrtf(var + add) : 1.0f / sqrtf(var + add);
    for (int64_t j = 0; j < n; ++j) {
      const float xf = load_f(x, r * xs + j, xdt);
      const int64_t wj = (mutate == ORACLE_MUT_RMS_W_REVERSED) ? (n - 1 - j) : j;
      const float wf = (mutate == ORACLE_MUT_RMS_NO_WEIGHT) ? 1.0f : load_f(w, wj, wdt);
      float o;
      if (mode == ORACLE_HF) {
        const float h = round_to(xf * rstd, xdt);
        o = wf * h;
      } else {
        o = (xf * rstd) * wf;
      }
      store_f(y, r * ys + j, ydt, o);
    }
  }
  return 0;
}

/*
 * Residual add + RMSNorm (the fused kernel beyond the reference, restating
 * the decoder layer's `hidden = residual + attn_out` followed by the norm):
 * h = round_xdt(x + r) in fp32, written to h[rows, n]; y = RMSNorm(h) in
 * `mode` as oracle_rmsnorm.  mutate 1: normalise the unrounded fp32 sum;
 * mutate 2: subtract the residual.  Returns 0, or -1 on a bad argument.
 */
int oracle_add_rmsnorm(const void* x, const void* r, const void* w, void* y, void* h, int64_t rows, int64_t n,
                       float eps, int xdt, int wdt, int ydt, int mode, int mutate) {
  if (!valid_dt(xdt) || !valid_dt(wdt) || !valid_dt(ydt) || n < 1 || rows < 0) return -1;
  for (int64_t i = 0; i < rows * n; ++i) {
    const float a = load_f(x, i, xdt);
    const float b = load_f(r, i, xdt);
    store_f(h, i, xdt, mutate == 2 ? a - b : a + b);
  }
  if (mutate != 1) return oracle_rmsnorm(h, w, y, rows, n, n, n, eps, xdt, wdt, ydt, mode, 0);
  /* planted mistake: the norm sees the fp32 sum before rounding */
  float* tmp = (float*)malloc((size_t)(rows * n) * sizeof(float));
  if (!tmp) return -1;
  for (int64_t i = 0; i < rows * n; ++i) tmp[i] = load_f(x, i, xdt) + load_f(r, i, xdt);
  const int st = oracle_rmsnorm(tmp, w, y, rows, n, n, n, eps, OR_F32, wdt, ydt, mode, 0);
  free(tmp);
  return st;
}

/* fp64 brute force: y[r*n + j] = x * w / sqrt(mean(x^2) + eps), all in double. */
int oracle_rmsnorm_f64(const void* x, const void* w, double* y, int64_t rows, int64_t n, int64_t xs,
                       double eps, int xdt, int wdt) {
  if (!valid_dt(xdt) || !valid_dt(wdt) || n < 1 || rows < 0) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    double ssd = 0.0;
    for (int64_t j = 0; j < n; ++j) {
      const double v = (double)load_f(x, r * xs + j, xdt);
      ssd += v * v;
    }
    const double rstd = 1.0 / sqrt(ssd / (double)n + eps);
    for (int64_t j = 0; j < n; ++j)
      y[r * n + j] = (double)load_f(x, r * xs + j, xdt) * rstd * (double)load_f(w, j, wdt);
  }
  return 0;
}

/* ---------------------------------------------------------- SiLU-and-mul */

/*
 *   TRITON (:30-36): out = (g * (1/(1+exp(-g)))) * u in fp32, one rounding.
 *   HF     (:56-59): s = round_odt(g / (1 + exp(-g)))  [torch's CPU silu],
 *                    out = round_odt(s * u).
 */
int oracle_silu_mul(const void* gate, const void* up, void* out, int64_t numel, int idt, int odt,
                    int mode, int mutate) {
  if (!valid_dt(idt) || !valid_dt(odt) || numel < 0) return -1;
  for (int64_t i = 0; i < numel; ++i) {
    float g = load_f(gate, i, idt);
    float u = load_f(up, i, idt);
    if (mutate == ORACLE_MUT_SILU_SWAP) {
      const float t = g;
      g = u;
      u = t;
    }
    const float arg = (mutate == ORACLE_MUT_SILU_SIGN) ? g : -g;
    float o;
    if (mode == ORACLE_HF) {
      const float s = round_to(g / (1.0f + expf(arg)), odt);
      o = (mutate == ORACLE_MUT_SILU_NO_UP) ? s : s * u;
    } else {
      const float sig = 1.0f / (1.0f + expf(arg));
      float s = g * sig;
      if (mutate == ORACLE_MUT_SILU_ROUND2) s = round_to(s, odt);
      o = (mutate == ORACLE_MUT_SILU_NO_UP) ? s : s * u;
    }
    store_f(out, i, odt, o);
  }
  return 0;
}

/* fp64 brute force: out[i] = g / (1 + exp(-g)) * u in double. */
int oracle_silu_mul_f64(const void* gate, const void* up, double* out, int64_t numel, int idt) {
  if (!valid_dt(idt) || numel < 0) return -1;
  for (int64_t i = 0; i < numel; ++i) {
    const double g = (double)load_f(gate, i, idt);
    const double u = (double)load_f(up, i, idt);
    out[i] = g / (1.0 + exp(-g)) * u;
  }
  return 0;
}

/* --------------------------------------------- gate/up + SiLU-and-mul */

enum { ORACLE_GU_FUSED = 0, ORACLE_GU_UNFUSED = 1 };
/* planted mistakes, gate/up + SiLU-and-mul */
enum {
  ORACLE_MUT_GU_TRANSPOSE = 1, /* read the weights as [k, n] instead of [n, k] */
  ORACLE_MUT_GU_SWAP = 2,      /* silu(up) * gate */
  ORACLE_MUT_GU_DROP_TAIL = 3, /* skip the last 8 columns of k */
  ORACLE_MUT_GU_ROW_SHIFT = 4  /* pair output row m with x row (m + 1) % rows */
};

/*
 *   g[m,j] = sum_c x[m,c] * wg[j,c],  u[m,j] = sum_c x[m,c] * wu[j,c]   (fp64)
 *   FUSED   (the fused projection kernel):
 *           out = round_odt((gf * (1 / (1 + exp(-gf)))) * uf),  gf = (float)g, uf = (float)u
 *   UNFUSED (FusedMLP, :60-64): gate = round_dt((float)g), up = round_dt((float)u)
 *           [the GEMMs' fp32 result rounded to x's type], then the SiLU-and-mul
 *           kernel's formula (src/kernels/fused_swiglu_triton.py:30-36) on them.
 *   Optional fp64 outputs (NULL to skip): g64, u64, out64 = g / (1 + exp(-g)) * u,
 *   gabs / uabs = sum_c |x[m,c] * w[j,c]| (scale for fp32 accumulation error bounds).
 * x: [rows, k], wg / wu: [n, k], outputs [rows, n], all contiguous.
 */
int oracle_gate_up_silu(const void* x, const void* wg, const void* wu, void* out, double* g64, double* u64,
                        double* out64, double* gabs, double* uabs, int64_t rows, int64_t k, int64_t n, int dt,
                        int odt, int mode, int mutate) {
  if (!valid_dt(dt) || !valid_dt(odt) || rows < 0 || k < 1 || n < 0) return -1;
  const int64_t kk = (mutate == ORACLE_MUT_GU_DROP_TAIL && k > 8) ? k - 8 : k;
  for (int64_t m = 0; m < rows; ++m) {
    const int64_t xm = (mutate == ORACLE_MUT_GU_ROW_SHIFT) ? (m + 1) % rows : m;
    for (int64_t j = 0; j < n; ++j) {
      double g = 0.0, u = 0.0, ga = 0.0, ua = 0.0;
      for (int64_t c = 0; c < kk; ++c) {
        const int64_t wi = (mutate == ORACLE_MUT_GU_TRANSPOSE) ? c * n + j : j * k + c;
        const double xv = (double)load_f(x, xm * k + c, dt);
        const double pg = xv * (double)load_f(wg, wi, dt);
        const double pu = xv * (double)load_f(wu, wi, dt);
        g += pg;
        u += pu;
        ga += fabs(pg);
        ua += fabs(pu);
      }
      if (mutate == ORACLE_MUT_GU_SWAP) {
        const double t = g;
        g = u;
        u = t;
      }
      const int64_t o = m * n + j;
      if (g64) g64[o] = g;
      if (u64) u64[o] = u;
      if (gabs) gabs[o] = ga;
      if (uabs) uabs[o] = ua;
      if (out64) out64[o] = g / (1.0 + exp(-g)) * u;
      float gf = (float)g, uf = (float)u;
      if (mode == ORACLE_GU_UNFUSED) {
        gf = round_to(gf, dt);
        uf = round_to(uf, dt);
      }
      const float sig = 1.0f / (1.0f + expf(-gf));
      store_f(out, o, odt, (gf * sig) * uf);
    }
  }
  return 0;
}

/* ------------------------------------------ W8A16 weight-only int8 linear */

enum { ORACLE_W8_KERNEL = 0, ORACLE_W8_DEQUANT = 1 };
/* planted mistakes, W8A16 linear */
enum {
  ORACLE_MUT_W8_TRANSPOSE = 1,   /* read q as [k, n] instead of [n, k] */
  ORACLE_MUT_W8_UNSIGNED = 2,    /* read the int8 weights as unsigned bytes */
  ORACLE_MUT_W8_BIAS_FIRST = 3,  /* (acc + bias) * scale */
  ORACLE_MUT_W8_NO_BIAS = 4,     /* drop the bias */
  ORACLE_MUT_W8_SCALE_SHIFT = 5  /* scale of output feature (j + 1) % n */
};

/*
 * out[m, j] for x [rows, k] (xdt), q [n, k] int8, scale [n] (sdt), bias [n]
 * (bdt, or bdt < 0 for none).  The exact dot product of x with the integer
 * weights is formed in fp64 (every product of a 16-bit float and an int8 is
 * exact there) and:
 *   KERNEL  (the Triton kernel, src/kernels/w8a16_matmul_triton.py:64-86):
 *           acc = (float)sum_c x*q  -- fp32 accumulation, order-free --
 *           out = round_odt(fmaf(acc, scale, bias))  or  round_odt(acc * scale)
 *           (the scale is applied once to the accumulator, then the bias).
 *   DEQUANT (w8a16_reference, :137-149): wf = (float)q * scale (fp32, one
 *           rounding per weight), out = round_odt((float)sum_c x*wf + bias):
 *           the fp32 linear of the dequantised matrix, order-free.
 * Optional fp64 outputs (NULL to skip): out64 = sum x*q*scale + bias,
 * absacc = sum |x*q| (scale of the fp32 accumulation error).
 * Returns 0, or -1 on a bad argument.
 */
int oracle_w8a16_linear(const void* x, const int8_t* q, const void* scale, const void* bias, void* out,
                        double* out64, double* absacc, int64_t rows, int64_t k, int64_t n, int xdt, int sdt,
                        int bdt, int odt, int mode, int mutate) {
  if (!valid_dt(xdt) || !valid_dt(sdt) || !valid_dt(odt) || (bdt >= 0 && !valid_dt(bdt)) || rows < 0 || k < 1 ||
      n < 1)
    return -1;
  const int has_bias = bdt >= 0 && bias != NULL && mutate != ORACLE_MUT_W8_NO_BIAS;
  for (int64_t m = 0; m < rows; ++m) {
    for (int64_t j = 0; j < n; ++j) {
      const int64_t js = (mutate == ORACLE_MUT_W8_SCALE_SHIFT) ? (j + 1) % n : j;
      const float sc = load_f(scale, js, sdt);
      const float bs = has_bias ? load_f(bias, j, bdt) : 0.0f;
      double acc = 0.0, aabs = 0.0, deq = 0.0;
      for (int64_t c = 0; c < k; ++c) {
        const int64_t wi = (mutate == ORACLE_MUT_W8_TRANSPOSE) ? c * n + j : j * k + c;
        const double qv = (mutate == ORACLE_MUT_W8_UNSIGNED) ? (double)(uint8_t)q[wi] : (double)q[wi];
        const double xv = (double)load_f(x, m * k + c, xdt);
        acc += xv * qv;
        aabs += fabs(xv * qv);
        deq += xv * (double)((float)qv * sc);
      }
      const int64_t o = m * n + j;
      if (out64) out64[o] = acc * (double)sc + (double)bs;
      if (absacc) absacc[o] = aabs;
      float v;
      if (mode == ORACLE_W8_DEQUANT) {
        v = (float)deq + bs;
      } else if (mutate == ORACLE_MUT_W8_BIAS_FIRST) {
        v = ((float)acc + bs) * sc;
      } else {
        v = has_bias ? fmaf((float)acc, sc, bs) : (float)acc * sc;
      }
      store_f(out, o, odt, v);
    }
  }
  return 0;
}

/* ------------------------------------------------------- 16-bit linear */

/* planted mistakes, 16-bit linear */
enum {
  ORACLE_MUT_L16_TRANSPOSE = 1, /* read w as [k, n] instead of [n, k] */
  ORACLE_MUT_L16_NO_BIAS = 2,   /* drop the bias */
  ORACLE_MUT_L16_DROP_TAIL = 3, /* skip the last 8 columns of k */
  ORACLE_MUT_L16_ROW_SHIFT = 4, /* pair output row m with x row (m + 1) % rows */
  ORACLE_MUT_L16_BIAS_LATE = 5  /* round the dot product to odt before adding the bias */
};

/*
 * out[m, j] for x [rows, k] and w [n, k] (both dt storage), bias [n] (bdt, or
 * bdt < 0 for none):
 *   acc = (float)sum_c x[m,c] * w[j,c]   (exact fp64 sum of exact products,
 *                                         rounded once: order-free fp32)
 *   out = round_odt(acc + bias)           (fp32 add)  or  round_odt(acc)
 * Optional fp64 outputs (NULL to skip): out64 = sum x*w + bias,
 * absacc = sum |x*w| (scale of the fp32 accumulation error).
 * Returns 0, or -1 on a bad argument.
 */
int oracle_linear16(const void* x, const void* w, const void* bias, void* out, double* out64, double* absacc,
                    int64_t rows, int64_t k, int64_t n, int dt, int bdt, int odt, int mutate) {
  if (!valid_dt(dt) || !valid_dt(odt) || (bdt >= 0 && !valid_dt(bdt)) || rows < 0 || k < 1 || n < 1) return -1;
  const int has_bias = bdt >= 0 && bias != NULL && mutate != ORACLE_MUT_L16_NO_BIAS;
  const int64_t kk = (mutate == ORACLE_MUT_L16_DROP_TAIL && k > 8) ? k - 8 : k;
  for (int64_t m = 0; m < rows; ++m) {
    const int64_t xm = (mutate == ORACLE_MUT_L16_ROW_SHIFT) ? (m + 1) % rows : m;
    for (int64_t j = 0; j < n; ++j) {
      const float bs = has_bias ? load_f(bias, j, bdt) : 0.0f;
      double acc = 0.0, aabs = 0.0;
      for (int64_t c = 0; c < kk; ++c) {
        const int64_t wi = (mutate == ORACLE_MUT_L16_TRANSPOSE) ? c * n + j : j * k + c;
        const double p = (double)load_f(x, xm * k + c, dt) * (double)load_f(w, wi, dt);
        acc += p;
        aabs += fabs(p);
      }
      const int64_t o = m * n + j;
      if (out64) out64[o] = acc + (double)bs;
      if (absacc) absacc[o] = aabs;
      float v = (float)acc;
      if (mutate == ORACLE_MUT_L16_BIAS_LATE) v = round_to(v, odt);
      if (has_bias) v = v + bs;
      store_f(out, o, odt, v);
    }
  }
  return 0;
}

/* planted mistakes, int8 quantizer */
enum {
  ORACLE_MUT_Q8_TRUNC = 1,   /* truncate toward zero instead of rounding */
  ORACLE_MUT_Q8_HALF_UP = 2, /* round halves away from zero */
  ORACLE_MUT_Q8_BY_128 = 3,  /* scale = amax / 128 */
  ORACLE_MUT_Q8_NO_CLAMP = 4 /* no 1e-8 floor on the scale */
};

/*
 * Per-output-channel symmetric int8 quantisation of w [n, k] (wdt), the
 * reference's QuantizedLinearInt8.from_linear (src/quantization/int8.py:45-50):
 *   wf = (float)w;  amax = max_c |wf|;  scale = max(amax / 127, 1e-8)   (fp32)
 *   q  = clamp(round_half_even(wf / scale), -127, 127)                  (fp32 divide)
 * Rows of finite weights only (NaN / Inf propagate as the arithmetic gives).
 * Returns 0, or -1 on a bad argument.
 */
int oracle_quantize_int8(const void* w, int8_t* q, float* scale, int64_t n, int64_t k, int wdt, int mutate) {
  if (!valid_dt(wdt) || n < 0 || k < 1) return -1;
  const float floor_ = 1e-8f;
  for (int64_t j = 0; j < n; ++j) {
    float amax = 0.0f;
    for (int64_t c = 0; c < k; ++c) {
      const float a = fabsf(load_f(w, j * k + c, wdt));
      if (a > amax) amax = a;
    }
    float sc = amax / ((mutate == ORACLE_MUT_Q8_BY_128) ? 128.0f : 127.0f);
    if (mutate != ORACLE_MUT_Q8_NO_CLAMP && sc < floor_) sc = floor_; /* torch.clamp keeps NaN */
    scale[j] = sc;
    for (int64_t c = 0; c < k; ++c) {
      const float t = load_f(w, j * k + c, wdt) / sc;
      float r;
      if (mutate == ORACLE_MUT_Q8_TRUNC) r = truncf(t);
      else if (mutate == ORACLE_MUT_Q8_HALF_UP) r = roundf(t);
      else r = rintf(t);
      if (r > 127.0f) r = 127.0f;
      if (r < -127.0f) r = -127.0f;
      q[j * k + c] = (int8_t)r;
    }
  }
  return 0;
}

/* ------------------------------------------------- bulk conversion helpers */

void oracle_f32_to_f16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}
void oracle_f16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}
void oracle_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(in[i]);
}
void oracle_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_to_f32(in[i]);
}
