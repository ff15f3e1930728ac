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


_CODE = _lib.DTYPE_CODE


def _rows(t: torch.Tensor, N: int):
    """(rows view, row count, row stride) of t with contiguous rows, copying
    only when the last dimension itself is strided."""
    if t.is_contiguous():
        return t, (t.numel() // N if N else 0), N
    t2 = t.reshape(-1, N)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < N):
        t2 = t2.contiguous()
    M = t2.shape[0]
    # Rows only need to be contiguous along the hidden dimension: a row-strided
    # view is passed with its stride instead of being copied.
    return t2, M, (t2.stride(0) if M > 1 else N)


def _empty_like_rows(x: torch.Tensor) -> torch.Tensor:
    return torch.empty_like(x) if x.is_contiguous() else torch.empty(x.shape, dtype=x.dtype, device=x.device)


def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Drop-in replacement for HF's RMSNorm.forward.  x: (..., hidden_size),
    weight: (hidden_size,).  Normalizes over the last dimension."""
    assert x.is_cuda and weight.is_cuda, "x and weight must be ROCm GPU tensors"
    N = x.shape[-1]
    assert weight.shape == (N,), f"weight shape {tuple(weight.shape)} != ({N},)"
    code, wcode = _CODE.get(x.dtype), _CODE.get(weight.dtype)
    assert code is not None and wcode is not None, (
        f"unsupported dtypes x={x.dtype} weight={weight.dtype} (fp16, bf16, fp32)")
    dev = x.get_device()
    assert weight.get_device() == dev, "x and weight must be on the same device"
    x2, M, xs = _rows(x, N)
    if weight.stride(0) != 1:
        weight = weight.contiguous()
    out = _empty_like_rows(x)
    if M and N:
        _lib.launch("mi355_rmsnorm_fwd", dev, x2.data_ptr(), weight.data_ptr(), out.data_ptr(), M, N, xs, N,
                    eps, code, wcode, code)
    return out


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6):
    """Residual add fused with RMSNorm: returns ``(rmsnorm(h), h)`` with
    ``h = residual + x`` rounded to x's dtype -- exactly what
    ``h = residual + x; y = fused_rmsnorm(h, weight, eps)`` returns, in one
    pass (read x and residual, write h and y).  x and residual have the same
    shape and dtype; normalises over the last dimension."""
    assert x.is_cuda and residual.is_cuda and weight.is_cuda, "x, residual and weight must be ROCm GPU tensors"
    assert x.shape == residual.shape, f"shape mismatch {tuple(x.shape)} vs {tuple(residual.shape)}"
    assert x.dtype == residual.dtype, f"dtype mismatch {x.dtype} vs {residual.dtype}"
    N = x.shape[-1]
    assert weight.shape == (N,), f"weight shape {tuple(weight.shape)} != ({N},)"
    code, wcode = _CODE.get(x.dtype), _CODE.get(weight.dtype)
    assert code is not None and wcode is not None, (
        f"unsupported dtypes x={x.dtype} weight={weight.dtype} (fp16, bf16, fp32)")
    dev = x.get_device()
    assert residual.get_device() == dev and weight.get_device() == dev, (
        "x, residual and weight must be on the same device")
    x2, M, xs = _rows(x, N)
    r2, _, rs = _rows(residual, N)
    if weight.stride(0) != 1:
        weight = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    h = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if M and N:
        _lib.launch("mi355_add_rmsnorm_fwd", dev, x2.data_ptr(), r2.data_ptr(), weight.data_ptr(), out.data_ptr(),
                    h.data_ptr(), M, N, xs, rs, N, N, eps, code, wcode, code)
    return out, h


def naive_rmsnorm_reference(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Unfused reference matching HF's RMSNorm formula: compute in fp32, cast
    back to x's dtype, then multiply by the weight."""
    input_dtype = x.dtype
    hidden_states = x.to(torch.float32)
    variance = hidden_states.pow(2).mean(-1, keepdim=True)
    hidden_states = hidden_states * torch.rsqrt(variance + eps)
    return weight * hidden_states.to(input_dtype)
