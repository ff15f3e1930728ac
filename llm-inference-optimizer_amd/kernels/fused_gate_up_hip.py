"""Gate/up projections fused with SiLU-and-mul.

``fused_gate_up_silu(x, w_gate, w_up)`` returns ``silu(x @ w_gate.T) *
(x @ w_up.T)`` in one gfx950 kernel (C ABI ``mi355_gate_up_silu_fwd``): the
two projections accumulate in fp32 on MFMA and feed the activation without
leaving registers, so the [rows, n_out] gate and up tensors of the
reference's FusedMLP chain (src/engine/fused_norm_activation_patch.py:60-64:
two GEMMs, each rounded to x's dtype, then ``fused_silu_mul``) are never
written or read.  This is the fusion the reference's design lists next
(docs/architecture-cuda.md:94).

At decode sizes (rows <= 32) the call streams both weight matrices once, at
HBM bandwidth; larger batches run an LDS-tiled MFMA GEMM over both weight
matrices with SiLU-and-mul in its epilogue.  Because g and u are not rounded
to x's dtype before the activation, results differ from the unfused chain by
that rounding (they are closer to the exact value), so FusedMLP uses it only
on request (``fuse_gate_up=True``).
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["fused_gate_up_silu", "naive_gate_up_silu_reference", "GATE_UP_MAX_ROWS"]

# Rows up to which the fused kernel streams the weights once (one 32-row
# tile); more rows take the tiled GEMM.
GATE_UP_MAX_ROWS = 32

_CODE = _lib.DTYPE_CODE


def fused_gate_up_silu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                       out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """silu(x @ w_gate.T) * (x @ w_up.T) for x [..., k] and nn.Linear weights
    [n_out, k] (fp16 or bf16, one dtype).  Output [..., n_out] in x's dtype
    (or ``out_dtype=torch.float32`` for the value before the final rounding).
    k and the row strides must be multiples of 8 elements."""
    assert x.is_cuda and w_gate.is_cuda and w_up.is_cuda, "x and the weights must be ROCm GPU tensors"
    assert x.dtype in (torch.float16, torch.bfloat16), f"x must be fp16 or bf16, got {x.dtype}"
    assert w_gate.dtype == x.dtype and w_up.dtype == x.dtype, (
        f"dtype mismatch x={x.dtype} w_gate={w_gate.dtype} w_up={w_up.dtype}")
    k = x.shape[-1]
    assert w_gate.dim() == 2 and w_gate.shape == w_up.shape and w_gate.shape[1] == k, (
        f"weights must be [n_out, {k}], got {tuple(w_gate.shape)} and {tuple(w_up.shape)}")
    dev = x.get_device()
    assert w_gate.get_device() == dev and w_up.get_device() == dev, "x and the weights must share a device"
    out_dtype = x.dtype if out_dtype is None else out_dtype
    assert out_dtype in (x.dtype, torch.float32), f"out_dtype must be {x.dtype} or float32"

    n_out = w_gate.shape[0]
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if w_gate.stride(-1) != 1 or w_up.stride(-1) != 1 or w_gate.stride(0) != w_up.stride(0):
        w_gate, w_up = w_gate.contiguous(), w_up.contiguous()
    rows = x2.shape[0]
    out = torch.empty((rows, n_out), dtype=out_dtype, device=x.device)
    if rows and n_out:
        # a single row's stride is arbitrary in torch (even 0); the kernel reads one row then
        xs = x2.stride(0) if rows > 1 else k
        ws = w_gate.stride(0) if n_out > 1 else k
        _lib.launch("mi355_gate_up_silu_fwd", dev, x2.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(),
                    out.data_ptr(), rows, k, n_out, xs, ws, n_out,
                    _CODE[x.dtype], _CODE[out_dtype])
    return out.view(*x.shape[:-1], n_out)


def naive_gate_up_silu_reference(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """The unfused formula with PyTorch ops: two projections, SiLU, multiply."""
    return torch.nn.functional.silu(x @ w_gate.T) * (x @ w_up.T)
