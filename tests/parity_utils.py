"""Shared helpers for the parity tests: seeded CPU inputs, storage views and
ULP comparisons."""
from __future__ import annotations

import numpy as np
import torch

DT_NAME = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, seed: int, dtype, mean: float = 0.0, std: float = 1.0) -> torch.Tensor:
    """N(mean, std) drawn in fp32 from a seeded CPU generator, then cast; the
    same values on every machine."""
    t = torch.randn(*shape, generator=gen(seed), dtype=torch.float32)
    return (mean + std * t).to(dtype)


def storage(t: torch.Tensor) -> np.ndarray:
    """CPU tensor -> numpy storage (uint16 bit patterns for fp16/bf16)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def ulp_report(got: np.ndarray, want: np.ndarray, orc) -> tuple[int, float]:
    d = orc.ulp_diff16(got, want)
    return int(d.max()) if d.size else 0, float((d > 0).mean()) if d.size else 0.0


def ulp16(v: np.ndarray, dt) -> np.ndarray:
    """One ulp of fp16 / bf16 at the magnitude of each (fp64) value."""
    mant, emin = (10, -14) if dt == torch.float16 else (7, -126)
    e = np.maximum(np.floor(np.log2(np.maximum(np.abs(v), 1e-300))), emin)
    return 2.0 ** (e - mant)


def act_error_bound(g, u, gabs, uabs, k):
    """Worst-case effect of fp32 summation (any order) of the gate / up
    projections on silu(g) * u: gamma_k * sum|x w| per projection (gabs,
    uabs; scaled by the quantisation scale where there is one), carried
    through the activation's derivatives."""
    gam = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    eg, eu = gam * gabs, gam * uabs
    sig = 1.0 / (1.0 + np.exp(-g))
    dsilu = sig * (1.0 + g * (1.0 - sig))
    # second-order slack: |silu''| <= 0.5
    return np.abs(dsilu * u) * eg + np.abs(g * sig) * eu + eg * eu + 0.5 * eg * eg * np.abs(u)
