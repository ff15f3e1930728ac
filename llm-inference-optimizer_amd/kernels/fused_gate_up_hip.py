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

def fused_gate_up_silu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                       out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """silu(x @ w_gate.T) * (x @ w_up.T) for x [..., k] and nn.Linear weights
    [n_out, k] (fp16 or bf16, one dtype).  Output [..., n_out] in x's dtype
    (or ``out_dtype=torch.float32`` for the value before the final rounding).
    k and the row strides must be multiples of 8 elements.  Launched by the
    C++ launcher ``_mi355_torch.gate_up_silu``."""
    out_f32 = out_dtype is not None and out_dtype != x.dtype
    assert not out_f32 or out_dtype == torch.float32, f"out_dtype must be {x.dtype} or float32"
    return _lib.ext().gate_up_silu(x, w_gate, w_up, out_f32)


def naive_gate_up_silu_reference(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """The unfused formula with PyTorch ops: two projections, SiLU, multiply."""
    return torch.nn.functional.silu(x @ w_gate.T) * (x @ w_up.T)
