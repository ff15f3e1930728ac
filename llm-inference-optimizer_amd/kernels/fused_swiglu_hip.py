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
    exactly, any shape is fine since the kernel treats memory as flat."""
    assert gate.shape == up.shape, f"shape mismatch {tuple(gate.shape)} vs {tuple(up.shape)}"
    assert gate.is_cuda and up.is_cuda, "gate and up must be ROCm GPU tensors"
    assert gate.dtype in _lib.DTYPE_CODE and up.dtype in _lib.DTYPE_CODE, (
        f"unsupported dtypes gate={gate.dtype} up={up.dtype} (fp16, bf16, fp32)")
    assert gate.device == up.device, "gate and up must be on the same device"

    out_dtype = gate.dtype
    if up.dtype != gate.dtype:
        # The reference widens each input to fp32 separately; widening both
        # here is exact, and the fp32 result is rounded once below.
        gate_c = gate.contiguous().to(torch.float32)
        up_c = up.contiguous().to(torch.float32)
    else:
        gate_c = gate.contiguous()
        up_c = up.contiguous()
    out = torch.empty(gate_c.shape, dtype=gate_c.dtype, device=gate.device)
    n = gate_c.numel()
    if n:
        dev = gate.device
        code = _lib.DTYPE_CODE[gate_c.dtype]
        if dev.index is not None and dev.index != torch.cuda.current_device():
            with torch.cuda.device(dev):
                _lib.silu_mul_fwd(gate_c.data_ptr(), up_c.data_ptr(), out.data_ptr(), n, code, code,
                                  _lib.stream_handle(dev))
        else:
            _lib.silu_mul_fwd(gate_c.data_ptr(), up_c.data_ptr(), out.data_ptr(), n, code, code,
                              _lib.stream_handle(dev))
    if out.dtype != out_dtype:
        out = out.to(out_dtype)
    return out.reshape(gate.shape)


def naive_silu_mul_reference(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Unfused reference: two separate PyTorch ops, exactly what HF does by
    default."""
    return torch.nn.functional.silu(gate) * up
