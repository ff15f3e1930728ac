"""CPU pins of the W8A16 oracle (``oracle.w8a16_linear``) and the int8
quantiser oracle (``oracle.quantize_int8``):

* the quantiser equals, bit for bit, torch's evaluation of the reference's
  expression (src/quantization/int8.py:46-48) on fp32 / fp16 / bf16 weights,
  zero rows, rows whose scale hits the 1e-8 floor, and exact ties (which
  torch.round sends to even); it keeps the reference's own guarantees (every
  dequantised weight within scale / 2, tests/test_w8a16_kernel.py:103-113;
  the largest |q| of a row is 127);
* the linear's fp64 value equals numpy's float64 GEMM of the same int8
  weights; KERNEL mode is that value through one fp32 fma and one rounding
  (within one fp32 ulp of the accumulator before the last step); DEQUANT mode
  agrees with torch's fp32 ``F.linear`` of the dequantised matrix (the
  reference's ``w8a16_reference``, :137-149) up to fp32 summation order;
* each planted mistake (transposed weights, bytes read unsigned, bias before
  scale, dropped bias, scale of the wrong feature; truncation, half-up
  rounding, /128, no scale floor) fails one of these checks.
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


def _from_storage(a: np.ndarray, dt: str) -> torch.Tensor:
    if dt == "f32":
        return torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(DT[dt])


def _torch_quantize(w: torch.Tensor):
    """The reference's quantiser expression evaluated by torch on the CPU."""
    wf = w.detach().float()
    scale = (wf.abs().amax(dim=1) / 127.0).clamp(min=1e-8)
    q = torch.round(wf / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return q.numpy(), scale.numpy()


def _weights(n, k, dt, seed, std=0.05):
    g = torch.Generator()
    g.manual_seed(seed)
    return (torch.randn(n, k, generator=g) * std).to(DT[dt])


# ------------------------------------------------------------- quantiser

@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n,k", [(37, 100), (64, 1536), (3, 1), (5, 8960)])
def test_quantizer_matches_torch_bitwise(dt, n, k):
    w = _weights(n, k, dt, seed=n + k)
    q, s = orc.quantize_int8(_storage(w), wdt=dt)
    tq, ts = _torch_quantize(w)
    assert np.array_equal(s.view(np.uint32), ts.view(np.uint32))
    assert np.array_equal(q, tq)


def test_quantizer_special_rows_match_torch():
    rows = [
        np.zeros(16, np.float32),                                   # scale floor 1e-8, q = 0
        np.full(16, 1e-12, np.float32),                             # amax / 127 below the floor
        np.array([127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5] * 2, np.float32),  # scale 1: ties
        np.array([-127.0, 126.5, -126.5, 0.0] * 4, np.float32),
        np.linspace(-3, 3, 16, dtype=np.float32),
        np.array([1e30, -1e30] + [1.0] * 14, np.float32),
    ]
    w = torch.from_numpy(np.stack(rows))
    q, s = orc.quantize_int8(w.numpy(), wdt="f32")
    tq, ts = _torch_quantize(w)
    assert np.array_equal(s.view(np.uint32), ts.view(np.uint32))
    assert np.array_equal(q, tq)
    assert s[0] == np.float32(1e-8) and not q[0].any()
    assert list(q[2][:8]) == [127, 2, -2, 4, -4, 0, 0, 2]           # ties to even


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_quantizer_invariants(dt):
    w = _weights(96, 1536, dt, seed=3)
    q, s = orc.quantize_int8(_storage(w), wdt=dt)
    wf = w.float().numpy().astype(np.float64)
    deq = q.astype(np.float64) * s.astype(np.float64)[:, None]
    assert np.all(np.abs(wf - deq) <= s[:, None] / 2 * 1.001 + 1e-6)
    assert np.all(np.abs(q).max(axis=1) == 127)
    assert np.all(np.sign(q) * np.sign(wf) >= 0)


@pytest.mark.parametrize("mutate", ["trunc", "half_up", "by_128", "no_clamp"])
def test_quantizer_planted_mistakes_are_caught(mutate):
    rows = np.stack([np.array([127.0, 2.5, -2.5, 3.5, 0.4, 0.6, -1.5, 9.75], np.float32),
                     np.zeros(8, np.float32)])
    w = torch.from_numpy(np.concatenate([rows, _weights(6, 8, "f32", seed=9).numpy()]))
    tq, ts = _torch_quantize(w)
    with np.errstate(invalid="ignore"):
        q, s = orc.quantize_int8(w.numpy(), wdt="f32", mutate=mutate)
    same = np.array_equal(q, tq) and np.array_equal(s.view(np.uint32), ts.view(np.uint32))
    assert not same, f"planted mistake {mutate} not caught"


# ---------------------------------------------------------------- linear

def _case(rows, k, n, xdt, seed, bias_dt=None):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(rows, k, generator=g).to(DT[xdt])
    w = (torch.randn(n, k, generator=g) * 0.05).to(DT[xdt])
    q, s = _torch_quantize(w)
    b = None if bias_dt is None else (torch.randn(n, generator=g) * 0.1).to(DT[bias_dt])
    return x, q, s, b


def _f64(x: torch.Tensor) -> np.ndarray:
    return x.double().numpy()


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("rows,k,n,bias", [(7, 100, 37, True), (16, 256, 96, False), (3, 1536, 64, True),
                                           (1, 1, 1, False)])
def test_linear_fp64_value_equals_numpy_gemm(xdt, rows, k, n, bias):
    x, q, s, b = _case(rows, k, n, xdt, seed=rows * 7 + k, bias_dt=xdt if bias else None)
    r = orc.w8a16_linear(_storage(x), q, s, None if b is None else _storage(b), xdt=xdt)
    want = (_f64(x) @ q.astype(np.float64).T) * s.astype(np.float64)
    if b is not None:
        want = want + _f64(b)
    assert np.allclose(r["out64"], want, rtol=1e-12, atol=1e-12)
    assert np.allclose(r["absacc"], np.abs(_f64(x)) @ np.abs(q.astype(np.float64)).T, rtol=1e-12)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_kernel_mode_is_one_fma_and_one_rounding(xdt):
    rows, k, n = 9, 640, 48
    x, q, s, b = _case(rows, k, n, xdt, seed=21, bias_dt="f32")
    r32 = orc.w8a16_linear(_storage(x), q, s, _storage(b), xdt=xdt, bdt="f32", odt="f32")
    r16 = orc.w8a16_linear(_storage(x), q, s, _storage(b), xdt=xdt, bdt="f32")
    acc = np.float32(_f64(x) @ q.astype(np.float64).T)           # order-free fp32 accumulator
    fma = (acc.astype(np.float64) * s.astype(np.float64) + _f64(b)).astype(np.float32)
    # numpy's fp64 sum may differ from the exact sum in its last fp32 bit (rarely)
    diff = np.abs(r32["out"].view(np.int32).astype(np.int64) - fma.view(np.int32).astype(np.int64))
    assert diff.max() <= 1 and (diff > 0).mean() < 0.01
    assert np.array_equal(r16["out"], orc.from_f32(r32["out"], xdt))


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_dequant_mode_matches_torch_reference_formula(xdt):
    """w8a16_reference: dequantise to fp32, fp32 F.linear, cast to x's dtype."""
    rows, k, n = 12, 896, 80
    x, q, s, b = _case(rows, k, n, xdt, seed=5, bias_dt=xdt)
    r = orc.w8a16_linear(_storage(x), q, s, _storage(b), xdt=xdt, mode="dequant", odt="f32")
    w = torch.from_numpy(q).float() * torch.from_numpy(s)[:, None]
    want = torch.nn.functional.linear(x.float(), w, b.float()).numpy()
    assert np.allclose(r["out"], want, rtol=2e-6, atol=2e-6)
    r16 = orc.w8a16_linear(_storage(x), q, s, _storage(b), xdt=xdt, mode="dequant")
    want16 = _storage(torch.from_numpy(want).to(DT[xdt]))
    d = orc.ulp_diff16(r16["out"], want16)
    assert d.max() <= 1 and (d > 0).mean() < 0.01


@pytest.mark.parametrize("mutate", ["transpose", "unsigned", "bias_first", "no_bias", "scale_shift"])
def test_linear_planted_mistakes_are_caught(mutate):
    rows, k, n = 6, 96, 40
    x, q, s, b = _case(rows, k, n, "f16", seed=13, bias_dt="f16")
    want = (_f64(x) @ q.astype(np.float64).T) * s.astype(np.float64) + _f64(b)
    good = orc.w8a16_linear(_storage(x), q, s, _storage(b), xdt="f16", odt="f32")["out"]
    bad = orc.w8a16_linear(_storage(x), q, s, _storage(b), xdt="f16", odt="f32", mutate=mutate)["out"]
    tol = 1e-4 * (np.abs(want) + 1e-2)
    assert np.all(np.abs(good - want) <= tol)
    assert not np.all(np.abs(bad - want) <= tol), f"planted mistake {mutate} not caught"


# ------------------------------------------ int8 gate/up + SiLU-and-mul

def _gu_case(rows, k, n, xdt, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    x = torch.randn(rows, k, generator=g).to(DT[xdt])
    qg, sg = _torch_quantize((torch.randn(n, k, generator=g) * (2.0 * k ** -0.5)).to(DT[xdt]))
    qu, su = _torch_quantize((torch.randn(n, k, generator=g) * k ** -0.5).to(DT[xdt]))
    return x, qg, sg, qu, su


def _gu_closed_form(x, qg, sg, qu, su):
    g = (_f64(x) @ qg.astype(np.float64).T) * sg.astype(np.float64)
    u = (_f64(x) @ qu.astype(np.float64).T) * su.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("rows,k,n", [(8, 1536, 96), (3, 100, 37), (33, 256, 64)])
def test_gate_up_w8a16_exact_value_is_the_closed_form(xdt, rows, k, n):
    x, qg, sg, qu, su = _gu_case(rows, k, n, xdt, seed=rows + k)
    r = orc.gate_up_silu_w8a16(_storage(x), qg, sg, qu, su, xdt=xdt)
    assert np.allclose(r["out64"], _gu_closed_form(x, qg, sg, qu, su), rtol=1e-12, atol=1e-14)
    assert np.allclose(r["gabs"], (np.abs(_f64(x)) @ np.abs(qg.astype(np.float64)).T) * sg, rtol=1e-12)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_gate_up_w8a16_single_rounding_matches_torch_fp32(xdt):
    """torch's fp32 evaluation of the fused formula: the order-free fp32
    projection sums times their scales, F.silu(g) * u in fp32, one cast."""
    rows, k, n = 16, 896, 160
    x, qg, sg, qu, su = _gu_case(rows, k, n, xdt, seed=3)
    r = orc.gate_up_silu_w8a16(_storage(x), qg, sg, qu, su, xdt=xdt)
    g32 = torch.from_numpy(np.float32(_f64(x) @ qg.astype(np.float64).T)) * torch.from_numpy(sg)
    u32 = torch.from_numpy(np.float32(_f64(x) @ qu.astype(np.float64).T)) * torch.from_numpy(su)
    want = _storage((torch.nn.functional.silu(g32) * u32).to(DT[xdt]))
    d = orc.ulp_diff16(r["out"], want)
    assert d.max() <= 1 and (d > 0).mean() < 0.01


@pytest.mark.parametrize("mutate", ["swap_scales", "swap_gate_up", "round_projections"])
def test_gate_up_w8a16_planted_mistakes_are_caught(mutate):
    rows, k, n = 12, 512, 96
    x, qg, sg, qu, su = _gu_case(rows, k, n, "f16", seed=11)
    sg = sg * np.float32(1.7)  # distinct scale magnitudes, so a swap shows
    exact = _gu_closed_form(x, qg, sg, qu, su)

    def ok(out):
        v = orc.to_f32(out, "f16").astype(np.float64)
        ulp = np.maximum(np.abs(exact), 2.0 ** -14) * 2.0 ** -10
        return np.mean(np.abs(v - exact) <= 0.5 * ulp + 1e-6 * np.abs(exact)) >= 0.99

    good = orc.gate_up_silu_w8a16(_storage(x), qg, sg, qu, su, xdt="f16")["out"]
    bad = orc.gate_up_silu_w8a16(_storage(x), qg, sg, qu, su, xdt="f16", mutate=mutate)["out"]
    assert ok(good)
    assert not ok(bad), f"planted mistake {mutate} not caught"
