"""GPU architecture detection and kernel tile configuration
(kernels/kernel_config.py:1-127 of the reference).

The reference picks Triton tile sizes per AMD family.  Here the kernels are
hand-written HIP for gfx950 (CDNA4), so the configuration reports the tiles
those kernels use; the other families keep their entries for callers that
inspect them, but no kernel of this package runs on them.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict

import torch


@dataclass
class KernelConfig:
    """Tile shape of the NF4 GEMM (same fields as the reference's
    TritonKernelConfig, kernel_config.py:9-16)."""
    BLOCK_M: int
    BLOCK_N: int
    BLOCK_K: int
    num_warps: int       # wavefronts per workgroup
    num_stages: int      # weight-tile pipeline depth
    wavefront_size: int  # 64 on CDNA, 32 on RDNA


# The name callers of the reference import.
TritonKernelConfig = KernelConfig

# gfx950 = MI355X / MI350X (CDNA4): the MFMA GEMM's 256x128 workgroup tiles,
# 64 k per step, eight wavefronts (two per SIMD), activation ring and weight
# tile double buffered in LDS -- the values rq_gemm_tile_config reports
CDNA4_CONFIG = KernelConfig(BLOCK_M=256, BLOCK_N=128, BLOCK_K=64, num_warps=8, num_stages=2, wavefront_size=64)
CDNA3_CONFIG = KernelConfig(BLOCK_M=64, BLOCK_N=64, BLOCK_K=32, num_warps=4, num_stages=2, wavefront_size=64)
CDNA2_CONFIG = KernelConfig(BLOCK_M=128, BLOCK_N=64, BLOCK_K=32, num_warps=8, num_stages=2, wavefront_size=64)
RDNA3_CONFIG = KernelConfig(BLOCK_M=64, BLOCK_N=64, BLOCK_K=64, num_warps=4, num_stages=2, wavefront_size=32)
RDNA2_CONFIG = KernelConfig(BLOCK_M=64, BLOCK_N=64, BLOCK_K=32, num_warps=4, num_stages=2, wavefront_size=32)
GENERIC_AMD_CONFIG = KernelConfig(BLOCK_M=64, BLOCK_N=64, BLOCK_K=32, num_warps=4, num_stages=2,
                                  wavefront_size=32)

_FAMILIES = (
    ("cdna4", ("gfx950", "mi355", "mi350")),
    ("cdna3", ("gfx942", "gfx941", "gfx940", "mi300")),
    ("cdna2", ("gfx90a", "mi250", "mi210")),
    ("rdna3", ("gfx1100", "gfx1101", "gfx1102", "7900", "7800")),
    ("rdna2", ("gfx1030", "gfx1031", "6900", "6800")),
)
_CONFIGS = {"cdna4": CDNA4_CONFIG, "cdna3": CDNA3_CONFIG, "cdna2": CDNA2_CONFIG,
            "rdna3": RDNA3_CONFIG, "rdna2": RDNA2_CONFIG}


def detect_gpu_arch() -> str:
    """'cdna4', 'cdna3', 'cdna2', 'rdna3', 'rdna2' or 'unknown'
    (kernel_config.py:50-78, with gfx950 added).  The device name and the
    gcnArchName are both consulted."""
    if not torch.cuda.is_available():
        return "unknown"
    props = torch.cuda.get_device_properties(0)
    text = (props.name + " " + getattr(props, "gcnArchName", "")).lower()
    for family, keys in _FAMILIES:
        if any(k in text for k in keys):
            return family
    return "unknown"


def get_kernel_config() -> KernelConfig:
    """Tile configuration for the detected architecture (kernel_config.py:80-93)."""
    return _CONFIGS.get(detect_gpu_arch(), GENERIC_AMD_CONFIG)


def is_triton_available() -> bool:
    """Always False: this package has no Triton kernels.  The name is kept for
    callers of the reference (kernel_config.py:95-104); the HIP kernels run
    whether or not a triton module is importable."""
    return False


def get_device_info() -> Dict[str, Any]:
    """Device summary with the reference's keys (kernel_config.py:106-127):
    arch, compute_units, vram_gb, wavefront_size, triton_available; plus
    gcn_arch and hip_kernels_available."""
    from rocm_qlora import _native
    if not torch.cuda.is_available():
        return {"arch": "unknown", "compute_units": 0, "vram_gb": 0.0, "wavefront_size": 32,
                "triton_available": False, "gcn_arch": "", "hip_kernels_available": False}
    props = torch.cuda.get_device_properties(0)
    return {
        "arch": detect_gpu_arch(),
        "compute_units": getattr(props, "multi_processor_count", 0),
        "vram_gb": props.total_memory / (1024 ** 3),
        "wavefront_size": get_kernel_config().wavefront_size,
        "triton_available": False,
        "gcn_arch": getattr(props, "gcnArchName", ""),
        "hip_kernels_available": _native.available(),
    }
