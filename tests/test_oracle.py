"""Pins the CPU oracle (oracle/fused_oracle.c) before it is trusted as the
parity checker.  Nothing here retypes the oracle's formulas; each check is
against something independent of it:

* storage conversions -- numpy's float16 casts (exhaustive for fp16 -> fp32)
  and torch's bfloat16 casts;
* the HF / naive formulation -- transformers' installed ``Qwen2RMSNorm`` and
  ``torch.nn.functional.silu`` run on the CPU (the same math as the
  reference's naive references, src/kernels/fused_rmsnorm_triton.py:74-82 and
  src/kernels/fused_swiglu_triton.py:56-59);
* the Triton formulation -- an fp64 brute force (within half an output ulp
  plus fp32 noise) and closed forms: zero rows, constant rows, exact
  power-of-two scale invariance, unit RMS with a unit weight, silu special
  values;
* the gate/up projections -- numpy's float64 GEMM, torch's float64 silu and
  torch's own 16-bit casts composed with the pinned SiLU-and-mul oracle;
* planted mistakes -- each deliberate error the oracle can be built with
  (``mutate``) fails at least one of the checks above.
"""
import numpy as np
import pytest
import torch

from parity_utils import randn, storage

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


# ----------------------------------------------------------------- conversions

def test_f16_to_f32_exhaustive(orc):
    allh = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(allh)
    want = allh.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _edge_floats():
    rng = np.random.default_rng(0)
    parts = [
        rng.standard_normal(200_000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(50_000) * 1e-5).astype(np.float32),          # fp16 subnormal range
        (rng.standard_normal(50_000) * 3e4).astype(np.float32),           # near fp16 overflow
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65519.99, 65520.0, -65520.0, 1e-8, 2.0**-24,
                  2.0**-25, 3 * 2.0**-26, 2.0**-14, 2.0**-14 - 2.0**-25, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11,
                  3.0e38, 1e-45], dtype=np.float32),
    ]
    # exact ties between consecutive fp16 values, both parities
    h = np.arange(0x0400, 0x7BFF, 7, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    parts.append(((lo + hi) / 2).astype(np.float32))
    return np.concatenate(parts)


def test_f32_to_f16_matches_numpy(orc):
    a = _edge_floats()
    got = orc.f32_to_f16(a)
    want = a.astype(np.float16).view(np.uint16)
    nan = np.isnan(a)
    assert np.array_equal(got[~nan], want[~nan])
    assert (np.isnan(got[nan].view(np.float16))).all()


def test_f32_to_bf16_matches_torch(orc):
    a = _edge_floats()
    got = orc.f32_to_bf16(a)
    want = torch.from_numpy(a).to(BF16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(a)
    assert np.array_equal(got[~nan], want[~nan])
    allb = np.arange(65536, dtype=np.uint16)
    back = orc.bf16_to_f32(allb)
    tb = torch.from_numpy(allb.view(np.int16)).view(BF16).float().numpy()
    ok = ~np.isnan(tb)
    assert np.array_equal(back[ok].view(np.uint32), tb[ok].view(np.uint32))


# ----------------------------------------------------- HF formulation pins

def _hf_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm
    m = Qwen2RMSNorm(x.shape[-1], eps=eps)
    m.weight = torch.nn.Parameter(w.clone())
    with torch.no_grad():
        return m(x)


def _check_rms_vs_hf(orc, xdt, wdt, n, mutate=None, rows=32, seed=0):
    x = randn((rows, n), seed, xdt)
    w = randn((n,), seed + 1, wdt, mean=1.0, std=0.1)
    y = _hf_rmsnorm(x, w, 1e-6)
    name = {F16: "f16", BF16: "bf16", F32: "f32"}
    got = orc.rmsnorm(storage(x), storage(w), 1e-6, xdt=name[xdt], wdt=name[wdt], mode="hf", mutate=mutate)
    if y.dtype == F32:
        return float(np.max(np.abs(got - y.numpy()) / (np.abs(y.numpy()) + 1e-30))), 0.0
    d = orc.ulp_diff16(got, storage(y))
    return int(d.max()), float((d > 0).mean())


@pytest.mark.parametrize("xdt,wdt,n", [(F16, F16, 1536), (BF16, BF16, 3584), (F16, F16, 100),
                                       (F16, F32, 896), (BF16, F32, 2048)])
def test_oracle_hf_rmsnorm_matches_transformers(orc, xdt, wdt, n):
    mx, frac = _check_rms_vs_hf(orc, xdt, wdt, n)
    if isinstance(mx, float):
        assert mx <= 1e-6
    else:
        # Only the fp32 summation order of the variance differs (torch's mean
        # vs the oracle's fp64 sum rounded once).
        assert mx <= 1 and frac < 1e-3


@pytest.mark.parametrize("dt,name", [(F16, "f16"), (BF16, "bf16")])
def test_oracle_hf_silu_mul_matches_torch(orc, dt, name):
    g = randn((64, 8960), 2, dt, std=2.0)
    u = randn((64, 8960), 3, dt)
    want = torch.nn.functional.silu(g) * u
    got = orc.silu_mul(storage(g), storage(u), idt=name, mode="hf")
    d = orc.ulp_diff16(got, storage(want))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


# ------------------------------------------------- Triton formulation pins

def _ulp16(vals: np.ndarray, dt: str) -> np.ndarray:
    """Spacing of the 16-bit grid at |vals| (for normal numbers)."""
    mant = 10 if dt == "f16" else 7
    e = np.floor(np.log2(np.maximum(np.abs(vals), 1e-30)))
    e = np.maximum(e, -14 if dt == "f16" else -126)
    return 2.0 ** (e - mant)


def _rms_triton_vs_f64(orc, dt, n, mutate=None, seed=0):
    tdt = {"f16": F16, "bf16": BF16}[dt]
    x = randn((16, n), seed, tdt)
    w = randn((n,), seed + 1, tdt, mean=1.0, std=0.1)
    got = orc.rmsnorm(storage(x), storage(w), 1e-6, xdt=dt, wdt=dt, mutate=mutate)
    got32 = orc.rmsnorm(storage(x), storage(w), 1e-6, xdt=dt, wdt=dt, ydt="f32", mutate=mutate)
    ref = orc.rmsnorm_f64(storage(x), storage(w), 1e-6, xdt=dt, wdt=dt)
    err16 = np.abs(orc.to_f32(got, dt).astype(np.float64) - ref) / _ulp16(ref, dt)
    err32 = np.abs(got32.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)
    return float(err16.max()), float(err32.max())


@pytest.mark.parametrize("dt,n", [("f16", 1536), ("bf16", 3584), ("f16", 100), ("bf16", 1)])
def test_oracle_triton_rmsnorm_vs_fp64(orc, dt, n):
    e16, e32 = _rms_triton_vs_f64(orc, dt, n)
    assert e32 < 2e-6          # the fp32 pipeline: a few fp32 ulp
    assert e16 <= 0.5 + 1e-3   # one rounding: half an output ulp (plus fp32 noise)


def _silu_triton_vs_f64(orc, dt, mutate=None):
    tdt = {"f16": F16, "bf16": BF16}[dt]
    g = randn((200_000,), 4, tdt, std=3.0)
    u = randn((200_000,), 5, tdt)
    got = orc.silu_mul(storage(g), storage(u), idt=dt, mutate=mutate)
    got32 = orc.silu_mul(storage(g), storage(u), idt=dt, odt="f32", mutate=mutate)
    ref = orc.silu_mul_f64(storage(g), storage(u), idt=dt)
    big = np.abs(ref) > 1e-3  # keep the check in the normal range of both formats
    err16 = np.abs(orc.to_f32(got, dt).astype(np.float64) - ref)[big] / _ulp16(ref[big], dt)
    err32 = (np.abs(got32.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30))[big]
    return float(err16.max()), float(err32.max())


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_oracle_triton_silu_mul_vs_fp64(orc, dt):
    e16, e32 = _silu_triton_vs_f64(orc, dt)
    assert e32 < 2e-6
    assert e16 <= 0.5 + 1e-3


def test_oracle_rmsnorm_closed_forms(orc):
    n = 1536
    x = np.zeros((3, n), np.float32)
    x[1] = 3.0
    x[2] = np.linspace(-2, 2, n, dtype=np.float32)
    w = (1 + 0.1 * np.random.default_rng(1).standard_normal(n)).astype(np.float32)
    y = orc.rmsnorm(x, w, 1e-6, xdt="f32", wdt="f32")
    assert (y[0] == 0).all()
    np.testing.assert_allclose(y[1], 3.0 / np.sqrt(9.0 + 1e-6) * w, rtol=1e-6)
    # unit weight: each row has RMS 1 (eps negligible)
    ones = np.ones(n, np.float32)
    y1 = orc.rmsnorm(x[2:], ones, 1e-12, xdt="f32", wdt="f32")
    assert abs(float(np.sqrt(np.mean(y1.astype(np.float64) ** 2))) - 1.0) < 1e-6


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_oracle_rmsnorm_power_of_two_scale_invariance(orc, dt):
    """With eps = 0, scaling x by 2^k scales the sum of squares by 4^k, the
    variance by 4^k and rstd by 2^-k, all exactly, so y is bit-identical."""
    tdt = {"f16": F16, "bf16": BF16}[dt]
    x = randn((16, 1536), 7, tdt)
    w = randn((1536,), 8, tdt, mean=1.0, std=0.1)
    y = orc.rmsnorm(storage(x), storage(w), 0.0, xdt=dt, wdt=dt)
    for k in (1, 2, 3):  # upward scaling stays exact (downward would hit fp16 subnormals)
        xs = (x.float() * 2.0 ** k).to(tdt)
        assert torch.equal(xs.float(), x.float() * 2.0 ** k)  # exact scaling in storage
        ys = orc.rmsnorm(storage(xs), storage(w), 0.0, xdt=dt, wdt=dt)
        assert np.array_equal(ys, y)


def test_oracle_silu_special_values(orc):
    g = np.array([0.0, -0.0, 30.0, 100.0, -100.0, np.inf, np.nan, 1.0], np.float32)
    u = np.array([5.0, 5.0, 2.0, 3.0, 3.0, 1.0, 1.0, 0.0], np.float32)
    o = orc.silu_mul(g, u, idt="f32")
    assert o[0] == 0 and o[1] == 0
    assert o[2] == np.float32(30.0 / (1 + np.exp(-30.0))) * 2.0
    assert o[3] == 300.0
    assert o[4] == 0 and np.signbit(o[4])
    assert o[5] == np.inf and np.isnan(o[6]) and o[7] == 0


# --------------------------------------------------------- planted mistakes

@pytest.mark.parametrize("mutate", ["n_minus_1", "no_eps", "sqrt", "no_weight", "w_reversed"])
def test_planted_rmsnorm_mistake_is_caught(orc, mutate):
    """Each mistake must fail the HF pin or the fp64 pin (eps is only visible
    on small-norm rows, so the fp64 pin also runs on a row scaled to ~1e-3)."""
    caught = []
    mx, frac = _check_rms_vs_hf(orc, F16, F16, 1536, mutate=mutate)
    caught.append(mx > 1 or frac >= 1e-3)
    e16, e32 = _rms_triton_vs_f64(orc, "f16", 1536, mutate=mutate)
    caught.append(e16 > 0.5 + 1e-3 or e32 >= 2e-6)
    x = (randn((4, 1536), 9, F32) * 1e-3)
    w = randn((1536,), 10, F32, mean=1.0, std=0.1)
    got = orc.rmsnorm(storage(x), storage(w), 1e-6, xdt="f32", wdt="f32", mutate=mutate)
    ref = orc.rmsnorm_f64(storage(x), storage(w), 1e-6, xdt="f32", wdt="f32")
    caught.append(np.max(np.abs(got - ref) / np.abs(ref)) > 1e-5)
    assert any(caught), f"planted mistake {mutate} was not caught"
    # and the faithful oracle passes the same checks
    assert _check_rms_vs_hf(orc, F16, F16, 1536)[0] <= 1


@pytest.mark.parametrize("mutate", ["sign", "swap", "no_up", "round2"])
def test_planted_silu_mistake_is_caught(orc, mutate):
    e16, e32 = _silu_triton_vs_f64(orc, "f16", mutate=mutate)
    g = randn((64, 8960), 2, F16, std=2.0)
    u = randn((64, 8960), 3, F16)
    want = torch.nn.functional.silu(g) * u
    hf = orc.silu_mul(storage(g), storage(u), idt="f16", mode="hf", mutate=mutate)
    d = orc.ulp_diff16(hf, storage(want))
    assert e16 > 0.5 + 1e-3 or e32 >= 2e-6 or d.max() > 1, f"planted mistake {mutate} was not caught"


# --------------------------------------------- residual add + RMSNorm (fused)

def _add_rms_vs_torch(orc, dt, n, mutate=None, rows=16, seed=40):
    x = randn((rows, n), seed, dt)
    r = randn((rows, n), seed + 1, dt, std=4.0)
    w = randn((n,), seed + 2, dt, mean=1.0, std=0.1)
    h_t = r + x                               # torch's CPU add, rounded to dt
    y_t = _hf_rmsnorm(h_t, w, 1e-6)           # transformers' norm of the rounded sum
    name = {F16: "f16", BF16: "bf16"}[dt]
    y, h = orc.add_rmsnorm(storage(x), storage(r), storage(w), 1e-6, xdt=name, wdt=name, mode="hf", mutate=mutate)
    dh = orc.ulp_diff16(h, storage(h_t))
    dy = orc.ulp_diff16(y, storage(y_t))
    yt, _ = orc.add_rmsnorm(storage(x), storage(r), storage(w), 1e-6, xdt=name, wdt=name, ydt="f32", mutate=mutate)
    ref = orc.rmsnorm_f64(storage(h_t), storage(w), 1e-6, xdt=name, wdt=name)
    rel = float(np.max(np.abs(yt.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)))
    return int(dh.max()), int(dy.max()), float((dy > 0).mean()), rel


@pytest.mark.parametrize("dt,n", [(F16, 1536), (BF16, 3584), (F16, 100)])
def test_oracle_add_rmsnorm_matches_torch_and_transformers(orc, dt, n):
    """h equals torch's own fp16/bf16 add bit for bit; y equals transformers'
    Qwen2RMSNorm of that sum (HF mode) to <= 1 ulp; the Triton-mode fp32 value
    is within fp32 noise of fp64 on the rounded sum."""
    dh, dy, frac, rel = _add_rms_vs_torch(orc, dt, n)
    assert dh == 0
    assert dy <= 1 and frac < 1e-3
    assert rel < 2e-6


@pytest.mark.parametrize("mutate", ["no_round", "subtract"])
def test_planted_add_rmsnorm_mistake_is_caught(orc, mutate):
    dh, dy, frac, rel = _add_rms_vs_torch(orc, F16, 1536, mutate=mutate)
    assert dh > 0 or dy > 1 or frac >= 1e-3 or rel >= 2e-6, f"planted mistake {mutate} was not caught"


# ------------------------------------------- gate/up projections + SiLU-and-mul

def _gate_up_inputs(dt, rows, k, n, seed):
    x = randn((rows, k), seed, dt)
    wg = randn((n, k), seed + 1, dt, std=k ** -0.5 * 2.0)
    wu = randn((n, k), seed + 2, dt, std=k ** -0.5)
    return x, wg, wu


def _gate_up_pins(orc, dt, rows, k, n, mutate=None, seed=50):
    """Errors of the oracle's gate/up path against independent computations:
    numpy's float64 GEMM for the projections, torch's float64 silu for the
    activation, and (unfused mode) torch's own fp32 -> 16-bit casts followed
    by the separately pinned SiLU-and-mul oracle."""
    name = {F16: "f16", BF16: "bf16"}[dt]
    x, wg, wu = _gate_up_inputs(dt, rows, k, n, seed)
    x64, wg64, wu64 = (t.to(torch.float64).numpy() for t in (x, wg, wu))
    g_np, u_np = x64 @ wg64.T, x64 @ wu64.T
    act = (torch.nn.functional.silu(torch.from_numpy(g_np)) * torch.from_numpy(u_np)).numpy()
    r = orc.gate_up_silu(storage(x), storage(wg), storage(wu), dt=name, mutate=mutate)
    r32 = orc.gate_up_silu(storage(x), storage(wg), storage(wu), dt=name, odt="f32", mutate=mutate)
    scale_g = np.abs(x64) @ np.abs(wg64).T
    scale_u = np.abs(x64) @ np.abs(wu64).T
    e_proj = max(float(np.max(np.abs(r["g"] - g_np) / scale_g)), float(np.max(np.abs(r["u"] - u_np) / scale_u)))
    e_act = float(np.max(np.abs(r["out64"] - act) / np.maximum(np.abs(act), 1e-30)))
    big = np.abs(act) > 1e-3
    e16 = float(np.max(np.abs(orc.to_f32(r["out"], name).astype(np.float64) - act)[big] / _ulp16(act[big], name)))
    e32 = float(np.max((np.abs(r32["out"].astype(np.float64) - act) / np.maximum(np.abs(act), 1e-30))[big]))
    # unfused chain: fp32 projections rounded by torch to the 16-bit type, then SiLU-and-mul
    gate16 = torch.from_numpy(g_np.astype(np.float32)).to(dt)
    up16 = torch.from_numpy(u_np.astype(np.float32)).to(dt)
    chain = orc.silu_mul(storage(gate16), storage(up16), idt=name)
    unf = orc.gate_up_silu(storage(x), storage(wg), storage(wu), dt=name, mode="unfused", mutate=mutate)["out"]
    chain_diff = int(orc.ulp_diff16(unf, chain).max())
    return e_proj, e_act, e16, e32, chain_diff


@pytest.mark.parametrize("dt,rows,k,n", [(F16, 8, 1536, 256), (BF16, 8, 1536, 256), (F16, 5, 72, 40),
                                         (BF16, 33, 40, 24), (F16, 1, 8, 7)])
def test_oracle_gate_up_silu_vs_numpy_and_torch(orc, dt, rows, k, n):
    e_proj, e_act, e16, e32, chain_diff = _gate_up_pins(orc, dt, rows, k, n)
    assert e_proj < 1e-13       # fp64 sums of exact products: rounding noise only
    assert e_act < 1e-12
    assert e32 < 2e-6           # fp32 activation of the fp64 projections
    assert e16 <= 0.5 + 1e-3    # one rounding to the output type
    assert chain_diff == 0      # unfused mode = torch's roundings + the SiLU-and-mul oracle


@pytest.mark.parametrize("mutate", ["transpose", "swap", "drop_tail", "row_shift"])
def test_planted_gate_up_mistake_is_caught(orc, mutate):
    e_proj, e_act, e16, e32, chain_diff = _gate_up_pins(orc, F16, 5, 72, 40, mutate=mutate)
    assert e_proj >= 1e-13 or e_act >= 1e-12 or e32 >= 2e-6 or e16 > 0.5 + 1e-3 or chain_diff != 0, (
        f"planted mistake {mutate} was not caught")
