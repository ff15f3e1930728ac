"""CPU oracle for the fused RMSNorm / SiLU-and-mul path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker (or the timed CPU baseline).
The product package never imports it.

Contents
--------
* numpy front end for ``fused_oracle.c`` (built by :func:`build` into
  ``oracle/liboracle_fused.so`` with gcc):
    - :func:`rmsnorm` / :func:`silu_mul` in ``mode="triton"`` restate the
      reference's fused Triton kernels (one rounding,
      src/kernels/fused_rmsnorm_triton.py:41-49,
      src/kernels/fused_swiglu_triton.py:30-36);
    - ``mode="hf"`` restates the naive/HF formulas
      (src/kernels/fused_rmsnorm_triton.py:74-82,
      src/kernels/fused_swiglu_triton.py:56-59);
    - :func:`rmsnorm_f64` / :func:`silu_mul_f64` are fp64 brute force.
* :func:`add_rmsnorm`: the residual add + RMSNorm fusion (beyond the
  reference): h = round(x + residual), then RMSNorm(h) in either mode;
* :func:`gate_up_silu`: the MLP's gate / up projections followed by
  SiLU-and-mul, fused (no rounding between projection and activation) or as
  the reference's FusedMLP chain (projections rounded to x's type,
  src/engine/fused_norm_activation_patch.py:60-64), with the fp64 values and
  the |x|.|w| scales that bound fp32 accumulation error;
* :func:`w8a16_linear`: the weight-only int8 linear -- the Triton kernel's
  order (integer dot product, then the per-channel scale, then the bias,
  src/kernels/w8a16_matmul_triton.py:64-86) or its dequantise-first
  reference (:137-149) -- with the fp64 value and sum |x * q|;
* :func:`quantize_int8`: the per-output-channel int8 quantiser
  (src/quantization/int8.py:45-50);
* :func:`linear16`: the MLP's down projection, nn.Linear with 16-bit weights
  (src/engine/fused_norm_activation_patch.py:64): fp32 dot product (the
  order-free fp32 value of the exact sum), the bias in fp32, one rounding,
  with the fp64 value and sum |x * w|;
* :func:`naive_rmsnorm_torch` / :func:`naive_silu_mul_torch`: the reference's
  naive PyTorch path restated as the same torch op sequence, which bench.py
  times on the host cores as the CPU baseline.
* ULP helpers for comparing fp16 / bf16 outputs.

16-bit arrays are passed as ``np.uint16`` bit patterns together with a dtype
name ("f16", "bf16"); fp32 arrays as ``np.float32`` with "f32".

Parity status: every function is pinned by tests/test_oracle.py (numpy /
torch conversions, transformers' Qwen2RMSNorm, torch.nn.functional.silu,
closed forms, fp64 brute force, planted mistakes).  Bitwise equality with the
reference's Triton kernels themselves is unpinned (they need an NVIDIA GPU and
Triton's backend math); the oracle stands in for them at <= 1 output ulp.
"""
from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
SRC = ORACLE_DIR / "fused_oracle.c"
LIB = ORACLE_DIR / "liboracle_fused.so"

DT_CODE = {"f32": 0, "f16": 1, "bf16": 2}
MODE_CODE = {"triton": 0, "hf": 1}

# planted-mistake codes (see fused_oracle.c)
MUT_RMS = {"n_minus_1": 1, "no_eps": 2, "sqrt": 3, "no_weight": 4, "w_reversed": 5}
MUT_SILU = {"sign": 1, "swap": 2, "no_up": 3, "round2": 4}
MUT_GU = {"transpose": 1, "swap": 2, "drop_tail": 3, "row_shift": 4}
GU_MODE = {"fused": 0, "unfused": 1}
W8_MODE = {"kernel": 0, "dequant": 1}
MUT_W8 = {"transpose": 1, "unsigned": 2, "bias_first": 3, "no_bias": 4, "scale_shift": 5}
MUT_Q8 = {"trunc": 1, "half_up": 2, "by_128": 3, "no_clamp": 4}
MUT_L16 = {"transpose": 1, "no_bias": 2, "drop_tail": 3, "row_shift": 4, "bias_late": 5}

_lib = None


def build(force: bool = True) -> Path:
    """Compile fused_oracle.c with gcc (no FMA contraction, no fast-math)."""
    if LIB.exists() and not force:
        return LIB
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("gcc not found; cannot build the oracle")
    tmp = LIB.with_name(LIB.name + ".tmp")
    cmd = [cc, "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-Werror", str(SRC), "-o", str(tmp), "-lm"]
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_rmsnorm.argtypes = [vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, i32, i32, i32, i32, i32]
        L.oracle_rmsnorm.restype = i32
        L.oracle_add_rmsnorm.argtypes = [vp, vp, vp, vp, vp, i64, i64, ctypes.c_float, i32, i32, i32, i32, i32]
        L.oracle_add_rmsnorm.restype = i32
        L.oracle_rmsnorm_f64.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_double, i32, i32]
        L.oracle_rmsnorm_f64.restype = i32
        L.oracle_silu_mul.argtypes = [vp, vp, vp, i64, i32, i32, i32, i32]
        L.oracle_silu_mul.restype = i32
        L.oracle_silu_mul_f64.argtypes = [vp, vp, vp, i64, i32]
        L.oracle_silu_mul_f64.restype = i32
        L.oracle_gate_up_silu.argtypes = [vp] * 9 + [i64, i64, i64, i32, i32, i32, i32]
        L.oracle_gate_up_silu.restype = i32
        L.oracle_w8a16_linear.argtypes = [vp] * 7 + [i64, i64, i64, i32, i32, i32, i32, i32, i32]
        L.oracle_w8a16_linear.restype = i32
        L.oracle_quantize_int8.argtypes = [vp, vp, vp, i64, i64, i32, i32]
        L.oracle_quantize_int8.restype = i32
        L.oracle_linear16.argtypes = [vp] * 6 + [i64, i64, i64, i32, i32, i32, i32]
        L.oracle_linear16.restype = i32
        for name in ("oracle_f32_to_f16_n", "oracle_f16_to_f32_n", "oracle_f32_to_bf16_n", "oracle_bf16_to_f32_n"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        _lib = L
    return _lib


def _np_dtype(dt: str):
    return np.float32 if dt == "f32" else np.uint16


def _arr(a: np.ndarray, dt: str) -> np.ndarray:
    a = np.ascontiguousarray(a)
    want = _np_dtype(dt)
    if a.dtype != want:
        raise TypeError(f"expected {want} storage for {dt}, got {a.dtype}")
    return a


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ----------------------------------------------------------------- RMSNorm

def hf_out_dtype(xdt: str, wdt: str) -> str:
    """torch's promotion of ``weight * h.to(x.dtype)`` (src/kernels/fused_rmsnorm_triton.py:82)."""
    if xdt == wdt:
        return xdt
    return "f32"


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, *, xdt: str, wdt: str,
            ydt: str | None = None, mode: str = "triton", mutate: str | None = None) -> np.ndarray:
    """x: [rows, n] storage array; w: [n].  Returns y [rows, n] in ydt storage."""
    x = _arr(x, xdt)
    w = _arr(w, wdt)
    if x.ndim != 2 or w.shape != (x.shape[1],):
        raise ValueError(f"bad shapes x={x.shape} w={w.shape}")
    if ydt is None:
        ydt = xdt if mode == "triton" else hf_out_dtype(xdt, wdt)
    rows, n = x.shape
    y = np.empty((rows, n), dtype=_np_dtype(ydt))
    mut = 0 if mutate is None else MUT_RMS[mutate]
    st = lib().oracle_rmsnorm(_ptr(x), _ptr(w), _ptr(y), rows, n, n, n, float(np.float32(eps)),
                              DT_CODE[xdt], DT_CODE[wdt], DT_CODE[ydt], MODE_CODE[mode], mut)
    if st != 0:
        raise ValueError("oracle_rmsnorm rejected its arguments")
    return y


def add_rmsnorm(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float = 1e-6, *, xdt: str, wdt: str,
                ydt: str | None = None, mode: str = "triton", mutate: str | None = None):
    """Residual add + RMSNorm: returns (y, h), h = round_xdt(x + r), y = RMSNorm(h)."""
    x = _arr(x, xdt)
    r = _arr(r, xdt)
    w = _arr(w, wdt)
    if x.ndim != 2 or r.shape != x.shape or w.shape != (x.shape[1],):
        raise ValueError(f"bad shapes x={x.shape} r={r.shape} w={w.shape}")
    if ydt is None:
        ydt = xdt if mode == "triton" else hf_out_dtype(xdt, wdt)
    rows, n = x.shape
    y = np.empty((rows, n), dtype=_np_dtype(ydt))
    h = np.empty((rows, n), dtype=_np_dtype(xdt))
    mut = {None: 0, "no_round": 1, "subtract": 2}[mutate]
    st = lib().oracle_add_rmsnorm(_ptr(x), _ptr(r), _ptr(w), _ptr(y), _ptr(h), rows, n, float(np.float32(eps)),
                                  DT_CODE[xdt], DT_CODE[wdt], DT_CODE[ydt], MODE_CODE[mode], mut)
    if st != 0:
        raise ValueError("oracle_add_rmsnorm rejected its arguments")
    return y, h


def rmsnorm_f64(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, *, xdt: str, wdt: str) -> np.ndarray:
    x = _arr(x, xdt)
    w = _arr(w, wdt)
    rows, n = x.shape
    y = np.empty((rows, n), dtype=np.float64)
    st = lib().oracle_rmsnorm_f64(_ptr(x), _ptr(w), _ptr(y), rows, n, n, float(eps), DT_CODE[xdt], DT_CODE[wdt])
    if st != 0:
        raise ValueError("oracle_rmsnorm_f64 rejected its arguments")
    return y


# ------------------------------------------------------------- SiLU-and-mul

def silu_mul(gate: np.ndarray, up: np.ndarray, *, idt: str, odt: str | None = None,
             mode: str = "triton", mutate: str | None = None) -> np.ndarray:
    gate = _arr(gate, idt)
    up = _arr(up, idt)
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    odt = odt or idt
    out = np.empty(gate.shape, dtype=_np_dtype(odt))
    mut = 0 if mutate is None else MUT_SILU[mutate]
    st = lib().oracle_silu_mul(_ptr(gate), _ptr(up), _ptr(out), gate.size, DT_CODE[idt], DT_CODE[odt],
                               MODE_CODE[mode], mut)
    if st != 0:
        raise ValueError("oracle_silu_mul rejected its arguments")
    return out


def silu_mul_f64(gate: np.ndarray, up: np.ndarray, *, idt: str) -> np.ndarray:
    gate = _arr(gate, idt)
    up = _arr(up, idt)
    out = np.empty(gate.shape, dtype=np.float64)
    st = lib().oracle_silu_mul_f64(_ptr(gate), _ptr(up), _ptr(out), gate.size, DT_CODE[idt])
    if st != 0:
        raise ValueError("oracle_silu_mul_f64 rejected its arguments")
    return out


# -------------------------------------------------------------- conversions

# --------------------------------------------------- gate/up + SiLU-and-mul

def gate_up_silu(x: np.ndarray, wg: np.ndarray, wu: np.ndarray, *, dt: str, odt: str | None = None,
                 mode: str = "fused", mutate: str | None = None) -> dict:
    """x: [rows, k], wg / wu: [n, k] in dt storage.  Returns a dict with
    ``out`` ([rows, n], odt storage, the ``mode`` formula), ``out64``, ``g``,
    ``u`` (fp64) and ``gabs`` / ``uabs`` (sum_k |x * w|, fp64)."""
    x = _arr(x, dt)
    wg = _arr(wg, dt)
    wu = _arr(wu, dt)
    if x.ndim != 2 or wg.ndim != 2 or wg.shape != wu.shape or wg.shape[1] != x.shape[1]:
        raise ValueError(f"bad shapes x={x.shape} wg={wg.shape} wu={wu.shape}")
    odt = odt or dt
    rows, k = x.shape
    n = wg.shape[0]
    res = {"out": np.empty((rows, n), dtype=_np_dtype(odt))}
    for key in ("g", "u", "out64", "gabs", "uabs"):
        res[key] = np.empty((rows, n), dtype=np.float64)
    mut = 0 if mutate is None else MUT_GU[mutate]
    st = lib().oracle_gate_up_silu(_ptr(x), _ptr(wg), _ptr(wu), _ptr(res["out"]), _ptr(res["g"]), _ptr(res["u"]),
                                   _ptr(res["out64"]), _ptr(res["gabs"]), _ptr(res["uabs"]), rows, k, n,
                                   DT_CODE[dt], DT_CODE[odt], GU_MODE[mode], mut)
    if st != 0:
        raise ValueError("oracle_gate_up_silu rejected its arguments")
    return res


# ------------------------------------------- W8A16 weight-only int8 linear

def w8a16_linear(x: np.ndarray, q: np.ndarray, scale: np.ndarray, bias: np.ndarray | None = None, *, xdt: str,
                 sdt: str = "f32", bdt: str | None = None, odt: str | None = None, mode: str = "kernel",
                 mutate: str | None = None) -> dict:
    """x: [rows, k] (xdt storage), q: [n, k] int8, scale: [n] (sdt storage),
    bias: [n] (bdt storage) or None.  Returns a dict with ``out`` ([rows, n],
    odt storage, the ``mode`` formula), ``out64`` (fp64 exact) and ``absacc``
    (sum_k |x * q|, fp64)."""
    x = _arr(x, xdt)
    q = np.ascontiguousarray(q)
    if q.dtype != np.int8:
        raise TypeError(f"q must be int8, got {q.dtype}")
    scale = _arr(scale, sdt)
    if x.ndim != 2 or q.ndim != 2 or q.shape[1] != x.shape[1] or scale.shape != (q.shape[0],):
        raise ValueError(f"bad shapes x={x.shape} q={q.shape} scale={scale.shape}")
    rows, k = x.shape
    n = q.shape[0]
    if bias is not None:
        bdt = bdt or xdt
        bias = _arr(bias, bdt)
        if bias.shape != (n,):
            raise ValueError(f"bias must be [{n}], got {bias.shape}")
    odt = odt or xdt
    res = {"out": np.empty((rows, n), dtype=_np_dtype(odt)), "out64": np.empty((rows, n), np.float64),
           "absacc": np.empty((rows, n), np.float64)}
    mut = 0 if mutate is None else MUT_W8[mutate]
    st = lib().oracle_w8a16_linear(_ptr(x), _ptr(q), _ptr(scale), _ptr(bias) if bias is not None else None,
                                   _ptr(res["out"]), _ptr(res["out64"]), _ptr(res["absacc"]), rows, k, n,
                                   DT_CODE[xdt], DT_CODE[sdt], DT_CODE[bdt] if bias is not None else -1,
                                   DT_CODE[odt], W8_MODE[mode], mut)
    if st != 0:
        raise ValueError("oracle_w8a16_linear rejected its arguments")
    return res


def gate_up_silu_w8a16(x: np.ndarray, qg: np.ndarray, sg: np.ndarray, qu: np.ndarray, su: np.ndarray, *,
                       xdt: str, sdt: str = "f32", odt: str | None = None, mutate: str | None = None) -> dict:
    """Int8 gate/up projections + SiLU-and-mul without intermediate rounding
    (the quantised MLP's gate_proj / up_proj, src/quantization/int8.py:62-63,
    and its activation, src/engine/fused_norm_activation_patch.py:60-64, as
    one computation).  Composes the pinned pieces: ``w8a16_linear`` in its
    kernel mode with an fp32 result (the order-free fp32 sum times the
    scale, unrounded) for each projection, then ``silu_mul`` on those fp32
    values with one rounding to ``odt``.  Returns ``out`` (odt storage),
    ``out64`` = silu(g) * u of the exact scaled projections, ``g`` / ``u``
    (fp64) and ``gabs`` / ``uabs`` = |scale| * sum_k |x * q|.

    ``mutate`` plants a mistake for the tests: "swap_scales" (each projection
    takes the other's scale), "swap_gate_up" (silu(u) * g) or
    "round_projections" (g and u rounded to xdt first, as the unfused chain)."""
    if mutate == "swap_scales":
        sg, su = su, sg
    g = w8a16_linear(x, qg, sg, xdt=xdt, sdt=sdt, odt="f32")
    u = w8a16_linear(x, qu, su, xdt=xdt, sdt=sdt, odt="f32")
    if mutate == "swap_gate_up":
        g, u = u, g
    odt = odt or xdt
    g32, u32 = g["out"], u["out"]
    if mutate == "round_projections":
        g32 = to_f32(from_f32(g32, xdt), xdt)
        u32 = to_f32(from_f32(u32, xdt), xdt)
    out = silu_mul(g32, u32, idt="f32", odt=odt)
    g64, u64 = g["out64"], u["out64"]
    sgv = np.abs(to_f32(_arr(sg, sdt), sdt).astype(np.float64))
    suv = np.abs(to_f32(_arr(su, sdt), sdt).astype(np.float64))
    return {"out": out, "out64": g64 / (1.0 + np.exp(-g64)) * u64, "g": g64, "u": u64,
            "gabs": g["absacc"] * sgv[None, :], "uabs": u["absacc"] * suv[None, :]}


def linear16(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None, *, dt: str, bdt: str | None = None,
             odt: str | None = None, mutate: str | None = None) -> dict:
    """x: [rows, k], w: [n, k] (dt storage), bias: [n] (bdt storage) or None.
    Returns a dict with ``out`` ([rows, n], odt storage), ``out64`` (fp64) and
    ``absacc`` (sum_k |x * w|, fp64)."""
    x = _arr(x, dt)
    w = _arr(w, dt)
    if x.ndim != 2 or w.ndim != 2 or w.shape[1] != x.shape[1]:
        raise ValueError(f"bad shapes x={x.shape} w={w.shape}")
    rows, k = x.shape
    n = w.shape[0]
    if bias is not None:
        bdt = bdt or dt
        bias = _arr(bias, bdt)
        if bias.shape != (n,):
            raise ValueError(f"bias must be [{n}], got {bias.shape}")
    odt = odt or dt
    res = {"out": np.empty((rows, n), dtype=_np_dtype(odt)), "out64": np.empty((rows, n), np.float64),
           "absacc": np.empty((rows, n), np.float64)}
    mut = 0 if mutate is None else MUT_L16[mutate]
    st = lib().oracle_linear16(_ptr(x), _ptr(w), _ptr(bias) if bias is not None else None, _ptr(res["out"]),
                               _ptr(res["out64"]), _ptr(res["absacc"]), rows, k, n, DT_CODE[dt],
                               DT_CODE[bdt] if bias is not None else -1, DT_CODE[odt], mut)
    if st != 0:
        raise ValueError("oracle_linear16 rejected its arguments")
    return res


def quantize_int8(w: np.ndarray, *, wdt: str, mutate: str | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric int8 quantisation of w [n, k] (wdt
    storage), as QuantizedLinearInt8.from_linear (src/quantization/int8.py:45-50).
    Returns (q int8 [n, k], scale float32 [n])."""
    w = _arr(w, wdt)
    if w.ndim != 2:
        raise ValueError(f"w must be 2-D, got {w.shape}")
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    scale = np.empty((n,), np.float32)
    mut = 0 if mutate is None else MUT_Q8[mutate]
    st = lib().oracle_quantize_int8(_ptr(w), _ptr(q), _ptr(scale), n, k, DT_CODE[wdt], mut)
    if st != 0:
        raise ValueError("oracle_quantize_int8 rejected its arguments")
    return q, scale


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    o = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_f16_n(_ptr(a), _ptr(o), a.size)
    return o


def f16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    o = np.empty(a.shape, np.float32)
    lib().oracle_f16_to_f32_n(_ptr(a), _ptr(o), a.size)
    return o


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    o = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_bf16_n(_ptr(a), _ptr(o), a.size)
    return o


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    o = np.empty(a.shape, np.float32)
    lib().oracle_bf16_to_f32_n(_ptr(a), _ptr(o), a.size)
    return o


def to_f32(a: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return np.asarray(a, np.float32)
    return f16_to_f32(a) if dt == "f16" else bf16_to_f32(a)


def from_f32(a: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return np.ascontiguousarray(a, np.float32)
    return f32_to_f16(a) if dt == "f16" else f32_to_bf16(a)


# ------------------------------------------------------------- ULP helpers

def ordered16(bits: np.ndarray) -> np.ndarray:
    """Map sign-magnitude 16-bit float patterns onto a monotone integer line
    (+0 and -0 both map to 0), so |a - b| counts representable steps."""
    b = bits.astype(np.int32)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def ulp_diff16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    return np.abs(ordered16(a_bits) - ordered16(b_bits))


# ---------------------------------------------- naive torch path (CPU baseline)

def naive_rmsnorm_torch(x, weight, eps: float = 1e-6):
    """The reference's unfused RMSNorm op sequence
    (src/kernels/fused_rmsnorm_triton.py:74-82): fp32 upcast, pow, mean,
    rsqrt, multiply, downcast, weight multiply."""
    import torch

    input_dtype = x.dtype
    h = x.to(torch.float32)
    variance = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(variance + eps)
    return weight * h.to(input_dtype)


def naive_silu_mul_torch(gate, up):
    """The reference's unfused SiLU-and-mul (src/kernels/fused_swiglu_triton.py:56-59)."""
    import torch

    return torch.nn.functional.silu(gate) * up
