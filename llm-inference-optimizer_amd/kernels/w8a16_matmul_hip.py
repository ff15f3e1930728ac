"""Weight-only int8 linear (W8A16) on gfx950 behind the reference's launcher API.

``w8a16_linear(x, w_q, scale, bias=None)`` keeps the signature, assertions,
output dtype and shapes of the reference's launcher
(src/kernels/w8a16_matmul_triton.py:102-134); the Triton kernel it launched is
replaced by hand-written HIP kernels behind the C ABI
``mi355_w8a16_linear_fwd``: a weight-streaming MFMA kernel for decode batches
(<= 16 rows; up to 48 -- 64 for matrices of at most 8 MB -- where the
small tiles do not pay), an LDS-tiled MFMA GEMM for larger ones.  Arithmetic as there:
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
    ``out_dtype=torch.float32``: the value before the final rounding).
    Preconditions as the reference's launcher (:108-111) plus dtype checks.
    Launched by the C++ launcher ``_mi355_torch.w8a16_linear``."""
    out_f32 = out_dtype is not None and out_dtype != x.dtype
    assert not out_f32 or out_dtype == torch.float32, f"out_dtype must be {x.dtype} or float32"
    return _lib.ext().w8a16_linear(x, w_q, scale, bias, out_f32)


def fused_gate_up_silu_w8a16(x: torch.Tensor, wq_gate: torch.Tensor, scale_gate: torch.Tensor,
                             wq_up: torch.Tensor, scale_up: torch.Tensor,
                             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """silu((x @ wq_gate.T) * scale_gate) * ((x @ wq_up.T) * scale_up) for x
    (..., K) fp16/bf16 and int8 weights (N, K) with (N,) scales (one float
    dtype).  Output (..., N) in x's dtype (or ``out_dtype=torch.float32``).
    Launched by the C++ launcher ``_mi355_torch.gate_up_silu_w8a16``."""
    out_f32 = out_dtype is not None and out_dtype != x.dtype
    assert not out_f32 or out_dtype == torch.float32, f"out_dtype must be {x.dtype} or float32"
    return _lib.ext().gate_up_silu_w8a16(x, wq_gate, scale_gate, wq_up, scale_up, out_f32)


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
