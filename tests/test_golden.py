"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from transformers' Qwen2RMSNorm / torch's F.silu on the CPU plus a numpy
fp64 evaluation).  On the CPU they pin the oracle; on the GPU the HIP
kernels are held to them through the C ABI, on machines where neither
transformers' outputs nor the oracle are recomputed."""
import importlib
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
RMS = sorted(GOLDEN.glob("rmsnorm_*.npz"))
SILU = sorted(GOLDEN.glob("silu_mul_*.npz"))
DT = {"float16": "f16", "bfloat16": "bf16", "float32": "f32"}
TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _load(p):
    return dict(np.load(p, allow_pickle=False))


def _ulp_bound(ref, dt):
    mant = 10 if dt == "f16" else 7
    e = np.floor(np.log2(np.maximum(np.abs(ref.astype(np.float64)), 1e-30)))
    e = np.maximum(e, -14 if dt == "f16" else -126)
    return 2.0 ** (e - mant)


def _to_torch(a, dt):
    if dt == "f32":
        return torch.from_numpy(a.copy())
    return torch.from_numpy(a.view(np.int16).copy()).view(TORCH_DT[dt])


def test_fixtures_present():
    assert len(RMS) >= 4 and len(SILU) >= 3


@pytest.mark.parametrize("path", RMS, ids=lambda p: p.stem)
def test_oracle_reproduces_rmsnorm_fixture(orc, path):
    f = _load(path)
    xdt, wdt, hdt = DT[str(f["xdt"])], DT[str(f["wdt"])], DT[str(f["hf_dt"])]
    eps = float(f["eps"])
    hf = orc.rmsnorm(f["x"], f["w"], eps, xdt=xdt, wdt=wdt, mode="hf")
    if hdt == "f32":
        np.testing.assert_allclose(hf, f["y_hf"], rtol=1e-6)
    else:
        d = orc.ulp_diff16(hf, f["y_hf"])
        assert d.max() <= 1 and (d > 0).mean() < 2e-3
    tri = orc.rmsnorm(f["x"], f["w"], eps, xdt=xdt, wdt=wdt, ydt=xdt)
    if xdt != "f32":
        err = np.abs(orc.to_f32(tri, xdt).astype(np.float64) - f["y_exact"]) / _ulp_bound(f["y_exact"], xdt)
        assert err.max() <= 0.5 + 1e-2


@pytest.mark.parametrize("path", SILU, ids=lambda p: p.stem)
def test_oracle_reproduces_silu_fixture(orc, path):
    f = _load(path)
    dt = DT[str(f["dt"])]
    hf = orc.silu_mul(f["gate"], f["up"], idt=dt, mode="hf")
    d = orc.ulp_diff16(hf, f["y_hf"])
    assert d.max() <= 1 and (d > 0).mean() < 2e-3
    tri = orc.silu_mul(f["gate"], f["up"], idt=dt)
    big = np.abs(f["y_exact"]) > 1e-3
    err = np.abs(orc.to_f32(tri, dt).astype(np.float64) - f["y_exact"])[big] / _ulp_bound(f["y_exact"][big], dt)
    assert err.max() <= 0.5 + 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("path", RMS, ids=lambda p: p.stem)
def test_kernel_matches_rmsnorm_fixture(pkg, cuda, path):
    f = _load(path)
    xdt, wdt = DT[str(f["xdt"])], DT[str(f["wdt"])]
    x = _to_torch(f["x"], xdt).to(cuda)
    w = _to_torch(f["w"], wdt).to(cuda)
    y = pkg.fused_rmsnorm(x, w, float(f["eps"])).cpu()
    assert y.dtype == TORCH_DT[xdt]
    yf = y.float().numpy().astype(np.float64)
    # one rounding of a value within a few fp32 ulp of exact: <= 0.5 ulp + noise
    err = np.abs(yf - f["y_exact"]) / _ulp_bound(f["y_exact"], xdt)
    assert err.max() <= 0.5 + 1e-2, err.max()
    # and within 1 ulp of HF's double-rounded value where HF kept x's dtype
    if DT[str(f["hf_dt"])] == xdt:
        L = importlib.import_module("oracle.oracle")
        d = L.ulp_diff16(y.contiguous().view(torch.int16).numpy().view(np.uint16), f["y_hf"])
        assert d.max() <= 1


@pytest.mark.gpu
@pytest.mark.parametrize("path", SILU, ids=lambda p: p.stem)
def test_kernel_matches_silu_fixture(pkg, cuda, path):
    f = _load(path)
    dt = DT[str(f["dt"])]
    g = _to_torch(f["gate"], dt).to(cuda)
    u = _to_torch(f["up"], dt).to(cuda)
    out = pkg.fused_silu_mul(g, u).cpu().float().numpy().astype(np.float64)
    big = np.abs(f["y_exact"]) > 1e-3
    err = np.abs(out - f["y_exact"])[big] / _ulp_bound(f["y_exact"][big], dt)
    assert err.max() <= 0.5 + 1e-2, err.max()


# ---- the package's naive references (the reference's naive_rmsnorm_reference /
# naive_silu_mul_reference, src/kernels/fused_rmsnorm_triton.py:74-82 and
# fused_swiglu_triton.py:56-59) on CPU tensors: HF's two-rounding formula, so
# they must reproduce the fixtures' y_hf -- written from transformers'
# Qwen2RMSNorm and torch's F.silu -- bit for bit, and the oracle's HF mode.

@pytest.mark.parametrize("path", RMS, ids=lambda p: p.stem)
def test_naive_rmsnorm_reference_reproduces_hf(pkg, orc, path):
    g = _load(path)
    xdt, wdt, hdt = DT[str(g["xdt"])], DT[str(g["wdt"])], DT[str(g["hf_dt"])]
    x, w = _to_torch(g["x"], xdt), _to_torch(g["w"], wdt)
    y = pkg.naive_rmsnorm_reference(x, w, float(g["eps"]))
    assert y.dtype == TORCH_DT[hdt]
    got = y.numpy() if hdt == "f32" else y.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, g["y_hf"]), path.stem
    hf = orc.rmsnorm(g["x"], g["w"], float(g["eps"]), xdt=xdt, wdt=wdt, mode="hf")
    assert np.array_equal(got, hf), path.stem


@pytest.mark.parametrize("path", SILU, ids=lambda p: p.stem)
def test_naive_silu_mul_reference_reproduces_hf(pkg, orc, path):
    g = _load(path)
    dt = DT[str(g["dt"])]
    gate, up = _to_torch(g["gate"], dt), _to_torch(g["up"], dt)
    y = pkg.naive_silu_mul_reference(gate, up)
    got = y.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, g["y_hf"]), path.stem
    assert np.array_equal(got, orc.silu_mul(g["gate"], g["up"], idt=dt, mode="hf")), path.stem
