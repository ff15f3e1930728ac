"""Weight-only int8 quantisation of a model's linear layers (module replacement)."""
from .int8 import QuantizedLinearInt8, quantize_model_int8

__all__ = ["QuantizedLinearInt8", "quantize_model_int8"]
