"""Fused SiLU-and-mul (the SwiGLU activation) on MI355X: drop-in for the
reference's ``src/kernels/fused_swiglu_triton.py``.

``fused_silu_mul(gate, up)`` keeps the reference launcher's contract
(:39-53): shapes must match, any shape is accepted because memory is treated
as flat, inputs are made contiguous, and the output has gate's dtype and
shape.  The computation runs in the gfx950 HIP kernels of
``libmi355_fused.so`` (C ABI ``mi355_silu_mul_fwd``) on torch's current
stream; there is no Triton and no CPU fallback.

Semantics are the reference Triton kernel's (:30-36): out = (g * sigmoid(g))
* u in fp32, rounded once to gate's dtype.

``naive_silu_mul_reference`` is the reference's unfused formula (:56-59).
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["fused_silu_mul", "naive_silu_mul_reference"]


def fused_silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Fused silu(gate) * up.  Purely elementwise -- shapes must match
    exactly, any shape is fine since the kernel treats memory as flat.
    Inputs are made contiguous; with different gate / up dtypes both are
    widened to fp32 and the result is rounded once to gate's dtype.  Launched
    by the C++ launcher ``_mi355_torch.silu_mul``."""
    return _lib.ext().silu_mul(gate, up)


def naive_silu_mul_reference(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Unfused reference: two separate PyTorch ops, exactly what HF does by
    default."""
    return torch.nn.functional.silu(gate) * up
