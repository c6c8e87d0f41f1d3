"""FP8 configuration and hardware detection (fp8/fp8_config.py of the reference)."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict

import torch

from rocm_qlora.quantization.double_quant import _has_fp8
from rocm_qlora.kernels import get_device_info


def detect_fp8_support() -> Dict[str, Any]:
    """FP8 support report with the reference's keys (fp8_config.py:11-56).
    Supported when torch has the fp8 dtypes, ROCm >= 6.2 and the GPU is CDNA4
    (gfx950, where this package's FP8 kernels run) or CDNA3 / CDNA2."""
    info = {"fp8_supported": False, "rocm_version": "not ROCm", "arch": "unknown",
            "fp8_dtypes_available": _has_fp8(), "transformer_engine_available": False, "reason": ""}
    rocm_ver = (0, 0)
    if getattr(torch.version, "hip", None):
        info["rocm_version"] = torch.version.hip
        try:
            parts = [int(p) for p in torch.version.hip.split(".")[:2]]
            rocm_ver = tuple(parts) if len(parts) == 2 else (0, 0)
        except ValueError:
            pass
    info["arch"] = get_device_info().get("arch", "unknown")
    # the FP8 linears run on this package's own kernels: TransformerEngine is
    # never imported or dispatched to, so it is reported as unavailable
    if not info["fp8_dtypes_available"]:
        info["reason"] = "FP8 dtypes unavailable in this PyTorch build"
    elif rocm_ver < (6, 2):
        info["reason"] = f"ROCm < 6.2 (found {info['rocm_version']})"
    elif info["arch"] not in ("cdna4", "cdna3", "cdna2"):
        info["reason"] = f"Unsupported GPU architecture ({info['arch']}) — CDNA GPU required"
    else:
        info["fp8_supported"] = True
        info["reason"] = "Supported"
    return info


@dataclass
class FP8Config:
    """FP8 training configuration (fp8_config.py:58-69)."""
    enabled: bool = True
    forward_dtype: str = "e4m3"
    backward_dtype: str = "e5m2"
    use_transformer_engine: bool = True  # kept for interface; TransformerEngine is never used
    fallback_dtype: torch.dtype = torch.bfloat16
    amax_history_len: int = 16
    amax_compute_algo: str = "max"


def get_fp8_dtype(format_str: str) -> torch.dtype:
    """'e4m3' -> float8_e4m3fnuz (else e4m3fn); 'e5m2' -> float8_e5m2fnuz
    (else e5m2) (fp8_config.py:72-89)."""
    if format_str == "e4m3":
        for name in ("float8_e4m3fnuz", "float8_e4m3fn"):
            if hasattr(torch, name):
                return getattr(torch, name)
        raise RuntimeError("No FP8 E4M3 dtype available. Check PyTorch version.")
    if format_str == "e5m2":
        for name in ("float8_e5m2fnuz", "float8_e5m2"):
            if hasattr(torch, name):
                return getattr(torch, name)
        raise RuntimeError("No FP8 E5M2 dtype available. Check PyTorch version.")
    raise ValueError(f"Unknown FP8 format: {format_str}")


def get_fp8_recipe(config: FP8Config):
    """The reference returns a TransformerEngine DelayedScaling recipe when TE
    is importable (fp8_config.py:91-101).  This package's FP8 linears use the
    per-tensor current-scaling recipe of fp8_linear.py:33-42 on its own
    kernels and never dispatch to TransformerEngine, so there is no recipe
    object: always None."""
    return None
