"""HIP kernels for the quantized linears (hip_kernels/__init__.py:22-36 of
the reference), built ahead of time for gfx950 (CDNA4).

    from rocm_qlora.hip_kernels import (
        is_hip_kernel_available, enable_hip_kernels,
        hip_dequant_int4_matmul, hip_dequant_int8_matmul, benchmark_hip_vs_triton)
"""
from rocm_qlora.hip_kernels.int4_matmul import (
    is_hip_kernel_available,
    enable_hip_kernels,
    hip_dequant_int4_matmul,
    hip_dequant_int8_matmul,
    benchmark_hip_vs_triton,
)

__all__ = [
    "is_hip_kernel_available",
    "enable_hip_kernels",
    "hip_dequant_int4_matmul",
    "hip_dequant_int8_matmul",
    "benchmark_hip_vs_triton",
]
