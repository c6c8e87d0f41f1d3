"""Model-level quantization (model/__init__.py of the reference)."""
from rocm_qlora.model.quantize_model import quantize_model, enable_all_kernels

__all__ = ["quantize_model", "enable_all_kernels"]
