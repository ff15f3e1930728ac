"""Weight-only int8 linear (W8A16) on gfx950 behind the reference's launcher API.

``w8a16_linear(x, w_q, scale, bias=None)`` keeps the signature, assertions,
output dtype and shapes of the reference's launcher
(src/kernels/w8a16_matmul_triton.py:102-134); the Triton kernel it launched is
replaced by hand-written HIP kernels behind the C ABI
``mi355_w8a16_linear_fwd``: a weight-streaming MFMA kernel for decode batches
(<= 32 rows), an LDS-tiled MFMA GEMM for larger ones.  Arithmetic as there:
``out = (sum_k x * w_q) * scale + bias`` with the integer dot product in fp32,
the scale applied once, one rounding to x's dtype.

``quantize_int8_weight(w)`` is the quantiser of
``QuantizedLinearInt8.from_linear`` (src/quantization/int8.py:45-50) as one
HIP kernel (C ABI ``mi355_quantize_int8_fwd``), bit-identical to the
reference's torch expression.

``w8a16_reference`` is the reference's dequantise-then-fp32-linear check
(:137-149), kept for API parity.

``fused_gate_up_silu_w8a16(x, wq_gate, scale_gate, wq_up, scale_up)`` is the
int8 form of ``fused_gate_up_silu``: the quantised model's gate_proj and
up_proj (two W8A16 linears) and SiLU-and-mul as one kernel (C ABI
``mi355_gate_up_silu_w8a16_fwd``), without rounding the projections.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["w8a16_linear", "w8a16_reference", "quantize_int8_weight", "fused_gate_up_silu_w8a16"]

_CODE = _lib.DTYPE_CODE


def w8a16_linear(x: torch.Tensor, w_q: torch.Tensor, scale: torch.Tensor,
                 bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x: (..., K) fp16/bf16.  w_q: (N, K) int8.  scale: (N,) float32 (fp16 /
    bf16 accepted).  bias: optional (N,).  Returns (..., N) in x's dtype (or
    ``out_dtype=torch.float32``: the value before the final rounding)."""
    assert x.is_cuda and w_q.is_cuda, "x and w_q must be ROCm GPU tensors"
    assert w_q.dtype == torch.int8, f"w_q must be int8, got {w_q.dtype}"
    N, K = w_q.shape
    assert x.shape[-1] == K, f"x last dim {x.shape[-1]} != weight in_features {K}"
    assert x.dtype in (torch.float16, torch.bfloat16), f"x must be fp16 or bf16, got {x.dtype}"
    assert scale.is_cuda and scale.shape == (N,) and scale.dtype in _CODE, (
        f"scale must be a ({N},) float GPU tensor, got {tuple(scale.shape)} {scale.dtype}")
    if bias is not None:
        assert bias.is_cuda and bias.shape == (N,) and bias.dtype in _CODE, (
            f"bias must be a ({N},) float GPU tensor, got {tuple(bias.shape)} {bias.dtype}")
    dev = x.get_device()
    assert w_q.get_device() == dev and scale.get_device() == dev, "x, w_q and scale must share a device"
    out_dtype = x.dtype if out_dtype is None else out_dtype
    assert out_dtype in (x.dtype, torch.float32), f"out_dtype must be {x.dtype} or float32"

    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if w_q.stride(-1) != 1:
        w_q = w_q.contiguous()
    scale = scale.contiguous()
    if bias is not None:
        bias = bias.contiguous()
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if M and N:
        # a single row's stride is arbitrary in torch (even 0); the kernels read one row then
        xs = x2.stride(0) if M > 1 else K
        ws = w_q.stride(0) if N > 1 else K
        _lib.launch("mi355_w8a16_linear_fwd", dev, x2.data_ptr(), w_q.data_ptr(), scale.data_ptr(),
                    bias.data_ptr() if bias is not None else None, out.data_ptr(), M, K, N,
                    xs, ws, N, _CODE[x.dtype], _CODE[scale.dtype],
                    _CODE[bias.dtype] if bias is not None else 0, _CODE[out_dtype])
    return out.reshape(*x.shape[:-1], N)


def fused_gate_up_silu_w8a16(x: torch.Tensor, wq_gate: torch.Tensor, scale_gate: torch.Tensor,
                             wq_up: torch.Tensor, scale_up: torch.Tensor,
                             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """silu((x @ wq_gate.T) * scale_gate) * ((x @ wq_up.T) * scale_up) for x
    (..., K) fp16/bf16 and int8 weights (N, K) with (N,) scales (one float
    dtype).  Output (..., N) in x's dtype (or ``out_dtype=torch.float32``)."""
    assert x.is_cuda and wq_gate.is_cuda and wq_up.is_cuda, "x and the weights must be ROCm GPU tensors"
    assert wq_gate.dtype == torch.int8 and wq_up.dtype == torch.int8, "weights must be int8"
    assert wq_gate.shape == wq_up.shape, f"weight shapes differ: {tuple(wq_gate.shape)} vs {tuple(wq_up.shape)}"
    N, K = wq_gate.shape
    assert x.shape[-1] == K, f"x last dim {x.shape[-1]} != weight in_features {K}"
    assert x.dtype in (torch.float16, torch.bfloat16), f"x must be fp16 or bf16, got {x.dtype}"
    for sc in (scale_gate, scale_up):
        assert sc.is_cuda and sc.shape == (N,) and sc.dtype in _CODE, (
            f"scales must be ({N},) float GPU tensors, got {tuple(sc.shape)} {sc.dtype}")
    assert scale_gate.dtype == scale_up.dtype, "the two scales must share a dtype"
    dev = x.get_device()
    assert all(t.get_device() == dev for t in (wq_gate, wq_up, scale_gate, scale_up)), "all inputs must share a device"
    out_dtype = x.dtype if out_dtype is None else out_dtype
    assert out_dtype in (x.dtype, torch.float32), f"out_dtype must be {x.dtype} or float32"

    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if wq_gate.stride(-1) != 1 or wq_up.stride(-1) != 1 or wq_gate.stride(0) != wq_up.stride(0):
        wq_gate, wq_up = wq_gate.contiguous(), wq_up.contiguous()
    scale_gate, scale_up = scale_gate.contiguous(), scale_up.contiguous()
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if M and N:
        xs = x2.stride(0) if M > 1 else K
        ws = wq_gate.stride(0) if N > 1 else K
        _lib.launch("mi355_gate_up_silu_w8a16_fwd", dev, x2.data_ptr(), wq_gate.data_ptr(), wq_up.data_ptr(),
                    scale_gate.data_ptr(), scale_up.data_ptr(), out.data_ptr(), M, K, N, xs, ws, N,
                    _CODE[x.dtype], _CODE[scale_gate.dtype], _CODE[out_dtype])
    return out.reshape(*x.shape[:-1], N)


def w8a16_reference(x: torch.Tensor, w_q: torch.Tensor, scale: torch.Tensor,
                    bias: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's check (src/kernels/w8a16_matmul_triton.py:137-149):
    dequantise the whole matrix to fp32, then an fp32 linear."""
    w = w_q.float() * scale.float()[:, None]
    b = bias.float() if bias is not None else None
    return torch.nn.functional.linear(x.float(), w, b).to(x.dtype)


def quantize_int8_weight(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel symmetric int8 quantisation of an (N, K) weight on the
    GPU: returns (w_q int8 (N, K), scale float32 (N,)) with
    ``scale = max(max|w_row| / 127, 1e-8)`` and ``w_q = clamp(round(w / scale),
    -127, 127)`` (ties to even), as src/quantization/int8.py:46-48 computes it."""
    assert weight.is_cuda, "weight must be a ROCm GPU tensor"
    assert weight.dim() == 2, f"weight must be 2-D, got {tuple(weight.shape)}"
    assert weight.dtype in _CODE, f"weight must be fp32, fp16 or bf16, got {weight.dtype}"
    w = weight.detach()
    if w.stride(-1) != 1:
        w = w.contiguous()
    N, K = w.shape
    w_q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    scale = torch.empty((N,), dtype=torch.float32, device=w.device)
    if N and K:
        _lib.launch("mi355_quantize_int8_fwd", w.get_device(), w.data_ptr(), w_q.data_ptr(), scale.data_ptr(),
                    N, K, w.stride(0) if N > 1 else K, K, _CODE[w.dtype])
    return w_q, scale
