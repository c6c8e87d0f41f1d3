"""FP8 compute (fp8/__init__.py of the reference): per-tensor e4m3fnuz
linears on the gfx950 FP8 kernels."""
from rocm_qlora.fp8.fp8_config import detect_fp8_support, FP8Config, get_fp8_dtype, get_fp8_recipe
from rocm_qlora.fp8.fp8_linear import FP8LinearWrapper, wrap_model_for_fp8, enable_fp8_autocast

__all__ = [
    "detect_fp8_support", "FP8Config", "get_fp8_dtype", "get_fp8_recipe",
    "FP8LinearWrapper", "wrap_model_for_fp8", "enable_fp8_autocast",
]
