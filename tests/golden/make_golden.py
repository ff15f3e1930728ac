"""Writes the golden fixtures in this directory.

Inputs come from seeded CPU torch generators.  Expected outputs come from
code that is independent of this repository's oracle and kernels:

* ``y_hf`` -- transformers' installed ``Qwen2RMSNorm.forward`` (the naive
  formula the reference's fused kernel replaces,
  src/kernels/fused_rmsnorm_triton.py:74-82) and ``F.silu(g) * u``
  (src/kernels/fused_swiglu_triton.py:56-59), run on the CPU;
* ``y_exact`` -- the same mathematics in numpy float64 (stored as float32,
  whose rounding is far below one fp16/bf16 ulp).

Run from the repository root:  python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
import torch
from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

OUT = Path(__file__).resolve().parent


def gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def bits(t):
    t = t.contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def rms_case(name, rows, n, xdt, wdt, eps, seed):
    x = torch.randn(rows, n, generator=gen(seed)).to(xdt)
    w = (1 + 0.1 * torch.randn(n, generator=gen(seed + 1))).to(wdt)
    m = Qwen2RMSNorm(n, eps=eps)
    m.weight = torch.nn.Parameter(w.clone())
    with torch.no_grad():
        y_hf = m(x)
    x64 = x.double().numpy()
    y64 = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps) * w.double().numpy()
    np.savez_compressed(OUT / f"{name}.npz", x=bits(x), w=bits(w), y_hf=bits(y_hf),
                        y_exact=y64.astype(np.float32), eps=np.float64(eps),
                        xdt=str(xdt).split(".")[-1], wdt=str(wdt).split(".")[-1],
                        hf_dt=str(y_hf.dtype).split(".")[-1])


def silu_case(name, shape, dt, seed):
    g = torch.randn(*shape, generator=gen(seed)).mul(2.0).to(dt)
    u = torch.randn(*shape, generator=gen(seed + 1)).to(dt)
    y_hf = torch.nn.functional.silu(g) * u
    g64, u64 = g.double().numpy(), u.double().numpy()
    y64 = g64 / (1.0 + np.exp(-g64)) * u64
    np.savez_compressed(OUT / f"{name}.npz", gate=bits(g), up=bits(u), y_hf=bits(y_hf),
                        y_exact=y64.astype(np.float32), dt=str(dt).split(".")[-1])


if __name__ == "__main__":
    rms_case("rmsnorm_f16_4x1536", 4, 1536, torch.float16, torch.float16, 1e-6, 100)
    rms_case("rmsnorm_f16_8x100", 8, 100, torch.float16, torch.float16, 1e-6, 110)
    rms_case("rmsnorm_bf16_4x3584", 4, 3584, torch.bfloat16, torch.bfloat16, 1e-6, 120)
    rms_case("rmsnorm_f16_w32_4x896", 4, 896, torch.float16, torch.float32, 1e-5, 130)
    silu_case("silu_mul_f16_1x8960", (1, 8960), torch.float16, 200)
    silu_case("silu_mul_f16_8x37", (8, 37), torch.float16, 210)
    silu_case("silu_mul_bf16_2x2048", (2, 2048), torch.bfloat16, 220)
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
