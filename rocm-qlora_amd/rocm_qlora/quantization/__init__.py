"""Quantization module (quantization/__init__.py:5-23 of the reference)."""
from rocm_qlora.quantization.quant_ops import (
    NF4_VALUES, quantize_int8, dequantize_int8, quantize_int4, dequantize_int4,
)
from rocm_qlora.quantization.double_quant import (
    double_quantize, double_dequantize, DoubleQuantState, estimate_double_quant_savings,
    patch_quant_linear_for_double_quant,
)

__all__ = [
    "quantize_int8", "dequantize_int8",
    "NF4_VALUES", "quantize_int4", "dequantize_int4",
    "QuantLinear", "W8A8Linear",
    "double_quantize", "double_dequantize",
    "DoubleQuantState", "estimate_double_quant_savings",
    "patch_quant_linear_for_double_quant",
]

from rocm_qlora.quantization.quant_linear import QuantLinear  # noqa: E402
from rocm_qlora.quantization.w8a8_linear import W8A8Linear  # noqa: E402
