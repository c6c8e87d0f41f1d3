"""HIP dequant-matmul entry points (hip_kernels/int4_matmul.py:306-498 of the
reference): ctypes dispatch into librocm_qlora_amd.so, enabling on a model,
and a micro-benchmark.  The kernels are gfx950 (CDNA4) code."""
from __future__ import annotations

import logging
import math
import time
from typing import Dict, Optional

import torch
import torch.nn as nn

from rocm_qlora import _native
from rocm_qlora.kernels.dequant_matmul import fused_dequant_nf4_matmul, fused_dequant_int8_matmul

logger = logging.getLogger("rocm_qlora.hip_kernels")


def is_hip_kernel_available() -> bool:
    """True when the library loads and a GPU is visible."""
    return torch.cuda.is_available() and _native.available()


def hip_dequant_int4_matmul(x: torch.Tensor, w_packed: torch.Tensor, scales: torch.Tensor,
                            bias: Optional[torch.Tensor] = None, block_size: int = 64) -> torch.Tensor:
    """NF4 dequantize + matmul, output in x's dtype with x's leading dims
    (int4_matmul.py:310-343).  Differentiable in x."""
    return fused_dequant_nf4_matmul(x, w_packed, scales, bias, block_size)


def hip_dequant_int8_matmul(x: torch.Tensor, w_int8: torch.Tensor, scales: torch.Tensor,
                            bias: Optional[torch.Tensor] = None, block_size: int = 64) -> torch.Tensor:
    """INT8 dequantize + matmul (int4_matmul.py:346-370); w_int8 [N, K]."""
    if w_int8.dim() == 1:
        w_int8 = w_int8.view(-1, x.shape[-1])
    return fused_dequant_int8_matmul(x, w_int8, scales, bias, block_size)


def enable_hip_kernels(model: nn.Module) -> int:
    """Set use_hip_kernel on every QuantLinear (int4_matmul.py:372-418);
    returns how many now run the HIP kernels (0 without a GPU or library)."""
    available = is_hip_kernel_available()
    count = 0
    for module in model.modules():
        if module.__class__.__name__ == "QuantLinear":
            module.use_hip_kernel = available
            if available:
                count += 1
    if not available:
        logger.info("HIP kernels not available: no GPU or librocm_qlora_amd.so not built")
    return count


def benchmark_hip_vs_triton(size: tuple = (4096, 4096), n_runs: int = 100, block_size: int = 64
                            ) -> Dict[str, float]:
    """Time the fused NF4 linear against the unfused path (HIP dequantize to
    fp16, then the library GEMM) on x [M, K] fp16 and a [4096, K] weight
    (int4_matmul.py:421-498).  Keys as the reference: hip_ms (fused),
    triton_ms (unfused -- there is no Triton here), speedup_x =
    triton_ms / hip_ms, winner, hip_available."""
    from rocm_qlora.quantization.quant_ops import quantize_int4, nf4_dequantize_to
    M, K = size
    N = 4096
    available = is_hip_kernel_available()
    if not available:
        return {"hip_ms": float("nan"), "triton_ms": float("nan"), "speedup_x": 0.0,
                "winner": "triton", "hip_available": False}
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(M, K, generator=g).to(dev, torch.float16)
    w_packed, scales = quantize_int4(torch.randn(N, K, generator=g).to(dev).flatten(), block_size=block_size)

    def fused():
        return fused_dequant_nf4_matmul(x, w_packed, scales, None, block_size)

    def unfused():
        w = nf4_dequantize_to(w_packed, scales, block_size, torch.float16, N * K).view(N, K)
        return torch.nn.functional.linear(x, w)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_runs):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n_runs * 1e3

    hip_ms = timed(fused)
    ref_ms = timed(unfused)
    speedup = ref_ms / hip_ms if hip_ms > 0 else 0.0
    return {"hip_ms": hip_ms, "triton_ms": ref_ms, "speedup_x": round(speedup, 2),
            "winner": "hip" if speedup > 1.0 else "triton", "hip_available": True}
