"""MI355X-native fused RMSNorm + SwiGLU path for Qwen2-style decoders.

The package directory name contains hyphens, so import it by name with
importlib after putting the repository root on ``sys.path``::

    import importlib, sys
    sys.path.insert(0, "/path/to/repo")
    fk = importlib.import_module("llm-inference-optimizer_amd")
    fk.patch_model_with_fused_kernels(model)

Public surface (the reference's Stage 3 plugin API):

* ``fused_rmsnorm(x, weight, eps=1e-6)``, ``naive_rmsnorm_reference``
* ``fused_silu_mul(gate, up)``, ``naive_silu_mul_reference``
* ``FusedRMSNorm``, ``FusedMLP``, ``patch_model_with_fused_kernels``,
  ``RMSNORM_CLASS_NAMES``, ``MLP_CLASS_NAMES``

and, beyond it, ``fused_add_rmsnorm`` (residual add + RMSNorm in one pass)
with ``FusedDecoderLayer`` / ``DECODER_LAYER_CLASS_NAMES``, which
``patch_model_with_fused_kernels(..., fuse_residual=True)`` installs, and
``GraphedGreedyDecoder``, greedy decoding whose per-token step replays one
captured HIP graph, and ``fused_gate_up_silu`` (gate / up projections +
SiLU-and-mul in one kernel for decode batches), which
``patch_model_with_fused_kernels(..., fuse_gate_up=True)`` lets FusedMLP use,
and ``linear16`` (a 16-bit linear that streams the weights at HBM bandwidth
for decode batches), which ``patch_model_with_fused_kernels(...,
hip_down=True)`` lets FusedMLP use for its down projection.

The reference's weight-only int8 stage sits beside it: ``w8a16_linear`` /
``w8a16_reference``, ``QuantizedLinearInt8`` and ``quantize_model_int8``
(int8 weights with per-output-channel scales, HIP quantiser and W8A16
kernels), composable with the fused-kernel patch.

The kernels live in ``libmi355_fused.so`` (gfx950 HIP, C ABI in
``include/mi355_fused.h``), built by ``build.py``.
"""
from .engine.fused_norm_activation_patch import (DECODER_LAYER_CLASS_NAMES, MLP_CLASS_NAMES, RMSNORM_CLASS_NAMES,
                                                 FusedDecoderLayer, FusedMLP, FusedRMSNorm,
                                                 patch_model_with_fused_kernels)
from .engine.graphed_decode import GraphedGreedyDecoder
from .kernels.fused_rmsnorm_hip import fused_add_rmsnorm, fused_rmsnorm, naive_rmsnorm_reference
from .kernels.fused_gate_up_hip import GATE_UP_MAX_ROWS, fused_gate_up_silu, naive_gate_up_silu_reference
from .kernels.fused_swiglu_hip import fused_silu_mul, naive_silu_mul_reference
from .kernels.linear16_hip import LINEAR16_MAX_ROWS, linear16
from .kernels.w8a16_matmul_hip import fused_gate_up_silu_w8a16, quantize_int8_weight, w8a16_linear, w8a16_reference
from .quantization.int8 import QuantizedLinearInt8, quantize_model_int8

__all__ = [
    "fused_rmsnorm", "naive_rmsnorm_reference", "fused_silu_mul", "naive_silu_mul_reference",
    "FusedRMSNorm", "FusedMLP", "patch_model_with_fused_kernels", "RMSNORM_CLASS_NAMES", "MLP_CLASS_NAMES",
    "fused_add_rmsnorm", "FusedDecoderLayer", "DECODER_LAYER_CLASS_NAMES", "GraphedGreedyDecoder",
    "fused_gate_up_silu", "naive_gate_up_silu_reference", "GATE_UP_MAX_ROWS",
    "w8a16_linear", "w8a16_reference", "quantize_int8_weight", "QuantizedLinearInt8", "quantize_model_int8",
    "fused_gate_up_silu_w8a16", "linear16", "LINEAR16_MAX_ROWS",
]
