"""GPU kernels of the quantized-linear path (kernels/__init__.py:5-23 of the
reference): fused dequantize + matmul for NF4 and INT8 weights, standalone
NF4 dequantization, device and tile information.  All run as hand-written
HIP kernels for gfx950."""
from rocm_qlora.kernels.kernel_config import (
    get_kernel_config,
    get_device_info,
    is_triton_available,
)
from rocm_qlora.kernels.dequant_matmul import (
    fused_dequant_int8_matmul,
    fused_dequant_nf4_matmul,
)
from rocm_qlora.kernels.nf4_dequant import dequantize_nf4_triton

__all__ = [
    "get_kernel_config",
    "get_device_info",
    "is_triton_available",
    "fused_dequant_int8_matmul",
    "fused_dequant_nf4_matmul",
    "dequantize_nf4_triton",
]
