"""16-bit linear on gfx950: the down projection of FusedMLP.

``linear16(x, weight, bias=None)`` computes ``x @ weight.T + bias`` (nn.Linear's
forward with fp16 / bf16 weights) through the C ABI ``mi355_linear16_fwd``.
The reference's FusedMLP ends with ``self.down_proj(activated)``
(src/engine/fused_norm_activation_patch.py:64), an nn.Linear that torch runs on
hipBLASLt; at decode batch sizes that call streams the whole weight matrix for
a handful of rows and hipBLASLt runs it well below HBM bandwidth.  Here up to
32 rows (64 on narrow outputs) read every weight byte once, at HBM
bandwidth, on MFMA; more rows run an LDS-tiled MFMA GEMM.  Sums are fp32 in this library's own order and the
bias is added in fp32 before the one rounding to x's dtype, so results may
differ from torch's linear in the last output bit.  FusedMLP uses it only on
request (``hip_down=True``) and only for inputs of at most ``LINEAR16_MAX_ROWS``
rows, where it is faster than hipBLASLt.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["linear16", "LINEAR16_MAX_ROWS"]

# Rows up to which FusedMLP's down projection takes this kernel (one 32-row
# weight-streaming tile); larger inputs stay on torch's linear.
LINEAR16_MAX_ROWS = 32


def linear16(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x: (..., K) fp16/bf16.  weight: (N, K) of x's dtype.  bias: optional (N,)
    float tensor.  Returns (..., N) in x's dtype (or ``out_dtype=torch.float32``:
    the value before the final rounding).  Launched by the C++ launcher
    ``_mi355_torch.linear16``."""
    out_f32 = out_dtype is not None and out_dtype != x.dtype
    assert not out_f32 or out_dtype == torch.float32, f"out_dtype must be {x.dtype} or float32"
    return _lib.ext().linear16(x, weight, bias, out_f32)
