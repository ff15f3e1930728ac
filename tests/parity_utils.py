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
