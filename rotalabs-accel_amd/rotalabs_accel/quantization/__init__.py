"""Quantization utilities (re-export names as src/rotalabs_accel/quantization/__init__.py:6-12),
plus ``quantize_model`` (the whole-model conversion recipe of the reference's docs)."""
from rotalabs_accel.quantization.convert import quantize_model
from rotalabs_accel.quantization.symmetric import (
    QuantizedLinear,
    calculate_quantization_error,
    dequantize,
    quantize_symmetric,
    quantize_weight_per_channel,
)

__all__ = [
    "quantize_symmetric",
    "dequantize",
    "quantize_weight_per_channel",
    "calculate_quantization_error",
    "QuantizedLinear",
    "quantize_model",
]
