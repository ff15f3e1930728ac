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


_CODE = _lib.DTYPE_CODE


def fused_silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Fused silu(gate) * up.  Purely elementwise -- shapes must match
    exactly, any shape is fine since the kernel treats memory as flat."""
    assert gate.shape == up.shape, f"shape mismatch {tuple(gate.shape)} vs {tuple(up.shape)}"
    assert gate.is_cuda and up.is_cuda, "gate and up must be ROCm GPU tensors"
    code, ucode = _CODE.get(gate.dtype), _CODE.get(up.dtype)
    assert code is not None and ucode is not None, (
        f"unsupported dtypes gate={gate.dtype} up={up.dtype} (fp16, bf16, fp32)")
    dev = gate.get_device()
    assert up.get_device() == dev, "gate and up must be on the same device"

    if code != ucode:
        # The reference widens each input to fp32 separately; widening both
        # here is exact, and the fp32 result is rounded once below.
        gate_c = gate.contiguous().to(torch.float32)
        up_c = up.contiguous().to(torch.float32)
        code = _CODE[torch.float32]
    else:
        gate_c = gate if gate.is_contiguous() else gate.contiguous()
        up_c = up if up.is_contiguous() else up.contiguous()
    out = torch.empty_like(gate_c)
    n = gate_c.numel()
    if n:
        _lib.launch("mi355_silu_mul_fwd", dev, gate_c.data_ptr(), up_c.data_ptr(), out.data_ptr(), n, code, code)
    if out.dtype != gate.dtype:
        out = out.to(gate.dtype)
    return out.view(gate.shape)


def naive_silu_mul_reference(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Unfused reference: two separate PyTorch ops, exactly what HF does by
    default."""
    return torch.nn.functional.silu(gate) * up
