"""Fused RMSNorm on MI355X: drop-in for the reference's
``src/kernels/fused_rmsnorm_triton.py``.

``fused_rmsnorm`` keeps the reference launcher's signature, preconditions and
output convention (:52-71): it normalises the last dimension, the output has
x's dtype and shape, and a failed precondition raises ``AssertionError``.
The computation runs in the gfx950 HIP kernels of ``libmi355_fused.so``
(C ABI ``mi355_rmsnorm_fwd``) on torch's current stream; there is no
Triton and no CPU fallback.

Semantics are the reference Triton kernel's (:35-49): fp32 sum of squares,
rstd = 1/sqrt(sum/n + eps), y = (x * rstd) * w in fp32, rounded once.

``naive_rmsnorm_reference`` is the reference's unfused HF formula (:74-82),
kept for callers that compare against it.

``fused_add_rmsnorm`` goes one step past the reference: the residual add that
precedes the norm in a decoder layer (``hidden = residual + attn_out`` then
``post_attention_layernorm(hidden)``) in the same pass, which the reference
plans as "fused RMSNorm + residual" (docs/architecture-cuda.md:94).
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["fused_rmsnorm", "fused_add_rmsnorm", "naive_rmsnorm_reference"]


def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Drop-in replacement for HF's RMSNorm.forward.  x: (..., hidden_size),
    weight: (hidden_size,).  Normalizes over the last dimension.

    Preconditions (AssertionError, as the reference's launcher): x and weight
    on the GPU, weight of shape (hidden_size,), fp16 / bf16 / fp32 storage,
    one device.  A row-strided x is read in place (rows only need to be
    contiguous along the hidden dimension); the output has x's dtype and
    shape.  The checks, the output allocation and the launch run in the C++
    launcher ``_mi355_torch.rmsnorm`` (csrc/torch_launchers.cpp)."""
    return _lib.ext().rmsnorm(x, weight, eps)


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6):
    """Residual add fused with RMSNorm: returns ``(rmsnorm(h), h)`` with
    ``h = residual + x`` rounded to x's dtype -- exactly what
    ``h = residual + x; y = fused_rmsnorm(h, weight, eps)`` returns, in one
    pass (read x and residual, write h and y).  x and residual have the same
    shape and dtype; normalises over the last dimension.  Launched by the C++
    launcher ``_mi355_torch.add_rmsnorm``."""
    return _lib.ext().add_rmsnorm(x, residual, weight, eps)


def naive_rmsnorm_reference(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Unfused reference matching HF's RMSNorm formula: compute in fp32, cast
    back to x's dtype, then multiply by the weight."""
    input_dtype = x.dtype
    hidden_states = x.to(torch.float32)
    variance = hidden_states.pow(2).mean(-1, keepdim=True)
    hidden_states = hidden_states * torch.rsqrt(variance + eps)
    return weight * hidden_states.to(input_dtype)
