"""16-bit linear on gfx950: the down projection of FusedMLP.

``linear16(x, weight, bias=None)`` computes ``x @ weight.T + bias`` (nn.Linear's
forward with fp16 / bf16 weights) through the C ABI ``mi355_linear16_fwd``.
The reference's FusedMLP ends with ``self.down_proj(activated)``
(src/engine/fused_norm_activation_patch.py:64), an nn.Linear that torch runs on
hipBLASLt; at decode batch sizes that call streams the whole weight matrix for
a handful of rows and hipBLASLt runs it well below HBM bandwidth.  Here up to
32 rows read every weight byte once, at HBM bandwidth, on MFMA; more rows run
an LDS-tiled MFMA GEMM.  Sums are fp32 in this library's own order and the
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

_CODE = _lib.DTYPE_CODE


def linear16(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x: (..., K) fp16/bf16.  weight: (N, K) of x's dtype.  bias: optional (N,)
    float tensor.  Returns (..., N) in x's dtype (or ``out_dtype=torch.float32``:
    the value before the final rounding)."""
    assert x.is_cuda and weight.is_cuda, "x and weight must be ROCm GPU tensors"
    assert x.dtype in (torch.float16, torch.bfloat16), f"x must be fp16 or bf16, got {x.dtype}"
    assert weight.dtype == x.dtype, f"dtype mismatch x={x.dtype} weight={weight.dtype}"
    assert weight.dim() == 2, f"weight must be (N, K), got {tuple(weight.shape)}"
    N, K = weight.shape
    assert x.shape[-1] == K, f"x last dim {x.shape[-1]} != weight in_features {K}"
    if bias is not None:
        assert bias.is_cuda and bias.shape == (N,) and bias.dtype in _CODE, (
            f"bias must be a ({N},) float GPU tensor, got {tuple(bias.shape)} {bias.dtype}")
    dev = x.get_device()
    assert weight.get_device() == dev and (bias is None or bias.get_device() == dev), (
        "x, weight and bias must share a device")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    assert out_dtype in (x.dtype, torch.float32), f"out_dtype must be {x.dtype} or float32"

    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if weight.stride(-1) != 1:
        weight = weight.contiguous()
    if bias is not None:
        bias = bias.contiguous()
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if M and N:
        # a single row's stride is arbitrary in torch (even 0); the kernels read one row then
        xs = x2.stride(0) if M > 1 else K
        ws = weight.stride(0) if N > 1 else K
        _lib.launch("mi355_linear16_fwd", dev, x2.data_ptr(), weight.data_ptr(),
                    bias.data_ptr() if bias is not None else None, out.data_ptr(), M, K, N, xs, ws, N,
                    _CODE[x.dtype], _CODE[bias.dtype] if bias is not None else 0, _CODE[out_dtype])
    return out.reshape(*x.shape[:-1], N)
