"""Module-replacement plugin that installs the fused kernels into a model."""
from .graphed_decode import GraphedGreedyDecoder
from .fused_norm_activation_patch import (DECODER_LAYER_CLASS_NAMES, MLP_CLASS_NAMES, RMSNORM_CLASS_NAMES,
                                          FusedDecoderLayer, FusedMLP, FusedRMSNorm, patch_model_with_fused_kernels)

__all__ = ["RMSNORM_CLASS_NAMES", "MLP_CLASS_NAMES", "DECODER_LAYER_CLASS_NAMES", "FusedRMSNorm", "FusedMLP",
           "FusedDecoderLayer", "patch_model_with_fused_kernels", "GraphedGreedyDecoder"]
