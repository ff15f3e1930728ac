"""CPU pins of the 16-bit linear oracle (``oracle.linear16``), the restatement
of FusedMLP's down projection (nn.Linear with fp16 / bf16 weights,
src/engine/fused_norm_activation_patch.py:64):

* its fp64 value equals numpy's float64 GEMM of the same 16-bit data (plus
  the bias), and its |x|.|w| scale equals numpy's GEMM of the magnitudes;
* its fp32 output is the order-free fp32 accumulator plus the bias in fp32
  (one fp32 add), and its 16-bit output is that fp32 value rounded once;
* it agrees with torch's own fp32 ``F.linear`` of the same 16-bit data cast to
  the output type, up to fp32 summation order (<= 1 output ulp on < 1% of
  elements);
* closed forms: an identity weight returns x (+ bias) exactly, a zero weight
  returns the bias;
* each planted mistake (transposed weight, dropped bias, dropped K tail,
  shifted x row, dot product rounded before the bias) fails one of these
  checks.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _storage(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.double().numpy()


def _case(rows, k, n, dt, seed, bias_dt=None):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(rows, k, generator=g).to(DT[dt])
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(DT[dt])
    b = None if bias_dt is None else (0.5 * torch.randn(n, generator=g)).to(DT[bias_dt])
    return x, w, b


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("rows,k,n,bias", [(7, 100, 37, True), (16, 256, 96, False), (3, 1536, 64, True),
                                           (1, 8, 1, False), (2, 8960, 24, True)])
def test_linear16_fp64_value_equals_numpy_gemm(dt, rows, k, n, bias):
    x, w, b = _case(rows, k, n, dt, seed=rows * 13 + k, bias_dt=dt if bias else None)
    r = orc.linear16(_storage(x), _storage(w), None if b is None else _storage(b), dt=dt)
    want = _f64(x) @ _f64(w).T
    if b is not None:
        want = want + _f64(b)
    assert np.allclose(r["out64"], want, rtol=1e-12, atol=1e-12)
    assert np.allclose(r["absacc"], np.abs(_f64(x)) @ np.abs(_f64(w)).T, rtol=1e-12)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("bias_dt", [None, "f32", "same"])
def test_linear16_is_fp32_sum_plus_bias_rounded_once(dt, bias_dt):
    rows, k, n = 9, 640, 48
    bdt = dt if bias_dt == "same" else bias_dt
    x, w, b = _case(rows, k, n, dt, seed=31, bias_dt=bdt)
    bs = None if b is None else _storage(b)
    r32 = orc.linear16(_storage(x), _storage(w), bs, dt=dt, bdt=bdt, odt="f32")
    r16 = orc.linear16(_storage(x), _storage(w), bs, dt=dt, bdt=bdt)
    acc = np.float32(_f64(x) @ _f64(w).T)  # order-free fp32 accumulator
    want = acc if b is None else (acc + b.float().numpy()[None, :]).astype(np.float32)
    # numpy's fp64 sum may differ from the exact sum in its last fp32 bit (rarely)
    diff = np.abs(r32["out"].view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert diff.max() <= 1 and (diff > 0).mean() < 0.01
    assert np.array_equal(r16["out"], orc.from_f32(r32["out"], dt))


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_linear16_matches_torch_fp32_linear(dt):
    """nn.Linear's arithmetic: fp32 sums of the 16-bit products, fp32 bias, one rounding."""
    rows, k, n = 12, 1536, 80
    x, w, b = _case(rows, k, n, dt, seed=5, bias_dt=dt)
    r = orc.linear16(_storage(x), _storage(w), _storage(b), dt=dt)
    want = torch.nn.functional.linear(x.float(), w.float(), b.float()).to(DT[dt])
    d = orc.ulp_diff16(r["out"], _storage(want))
    assert d.max() <= 1 and (d > 0).mean() < 0.01


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_linear16_closed_forms(dt):
    rows, k = 5, 64
    x, _, b = _case(rows, k, k, dt, seed=3, bias_dt=dt)
    eye = torch.eye(k).to(DT[dt])
    r = orc.linear16(_storage(x), _storage(eye), dt=dt)
    assert np.array_equal(r["out"], _storage(x))
    zero = torch.zeros(k, k).to(DT[dt])
    r = orc.linear16(_storage(x), _storage(zero), _storage(b), dt=dt)
    assert np.array_equal(r["out"], np.broadcast_to(_storage(b), (rows, k)))


@pytest.mark.parametrize("mutate", ["transpose", "no_bias", "drop_tail", "row_shift"])
def test_linear16_planted_mistakes_are_caught(mutate):
    rows, k, n = 6, 96, 96
    x, w, b = _case(rows, k, n, "f16", seed=17, bias_dt="f32")
    want = _f64(x) @ _f64(w).T + _f64(b)
    good = orc.linear16(_storage(x), _storage(w), _storage(b), dt="f16", bdt="f32", odt="f32")["out"]
    bad = orc.linear16(_storage(x), _storage(w), _storage(b), dt="f16", bdt="f32", odt="f32", mutate=mutate)["out"]
    tol = 1e-5 * (np.abs(want) + 1e-2)
    assert np.all(np.abs(good - want) <= tol)
    assert not np.all(np.abs(bad - want) <= tol), f"planted mistake {mutate} not caught"


def test_linear16_double_rounding_is_caught():
    """Rounding the dot product to the output type before the bias (two
    roundings) moves many outputs off the correctly rounded exact value."""
    rows, k, n = 16, 256, 128
    x, w, b = _case(rows, k, n, "f16", seed=19, bias_dt="f32")
    exact16 = orc.from_f32((_f64(x) @ _f64(w).T + _f64(b)).astype(np.float32), "f16")
    good = orc.linear16(_storage(x), _storage(w), _storage(b), dt="f16", bdt="f32")["out"]
    bad = orc.linear16(_storage(x), _storage(w), _storage(b), dt="f16", bdt="f32", mutate="bias_late")["out"]
    dg, db = orc.ulp_diff16(good, exact16), orc.ulp_diff16(bad, exact16)
    assert dg.max() <= 1 and (dg > 0).mean() < 0.01
    assert (db > 0).mean() > 0.05, "planted double rounding not caught"
