"""Double quantization of the NF4 absmax (QLoRA): c1 -> (c2, c2_scales).

Same API and state layout as the reference's quantization/double_quant.py:
c2 holds torch.float8_e4m3fnuz codes (or int8 when no fp8 dtype exists),
c2_scales one absmax per `blocksize_2` c1 values, in c1's dtype.  The
arithmetic runs in csrc/codec.hip (rq_dq_quantize / rq_dq_dequantize).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict

import torch
import torch.nn as nn

from rocm_qlora import _native as nat
from rocm_qlora._device import on, to_gpu
from rocm_qlora.quantization.quant_ops import _squeeze_scales, quantize_int4, nf4_dequantize_to


def _has_fp8() -> bool:
    """True when torch has an fp8 e4m3 dtype (double_quant.py:20-25)."""
    return hasattr(torch, "float8_e4m3fnuz") or hasattr(torch, "float8_e4m3fn")


def _get_fp8_dtype() -> torch.dtype:
    """float8_e4m3fnuz when available, else float8_e4m3fn (double_quant.py:28-33).
    The kernels encode fnuz; an e4m3fn-only torch is rejected at quantize time."""
    if hasattr(torch, "float8_e4m3fnuz"):
        return torch.float8_e4m3fnuz
    return torch.float8_e4m3fn


@dataclass
class DoubleQuantState:
    """Complete state for double-quantized weights (double_quant.py:35-44)."""
    W_quant: torch.Tensor
    c2: torch.Tensor
    c2_scales: torch.Tensor
    blocksize_1: int = 64
    blocksize_2: int = 256
    original_shape: tuple = None
    use_fp8_c2: bool = False


def _c2_format(use_fp8: bool) -> int:
    return nat.C2_FP8_E4M3FNUZ if use_fp8 else nat.C2_INT8


def dq_quantize_absmax(c1: torch.Tensor, blocksize_2: int, use_fp8: bool):
    """Second quantization stage on GPU c1 values: returns (c2 [padded],
    c2_scales [nb2] unsqueezed), c2 as fnuz (use_fp8) or int8."""
    dev = nat.require_gpu(c1)
    with on(dev):
        c1f = c1.contiguous().view(-1)
        n = c1f.numel()
        nb2 = -(-n // blocksize_2)
        c2 = torch.empty((nb2 * blocksize_2,), dtype=torch.uint8, device=dev)
        c2s = torch.empty((nb2,), dtype=c1f.dtype, device=dev)
        if n:
            nat.call("rq_dq_quantize", c1f.data_ptr(), nat.dtype_code(c1f.dtype), n, blocksize_2,
                     _c2_format(use_fp8), c2.data_ptr(), c2s.data_ptr(), nat.stream_handle(dev))
    if use_fp8:
        if _get_fp8_dtype() != getattr(torch, "float8_e4m3fnuz", None):
            raise RuntimeError("double quantization encodes float8_e4m3fnuz; this torch lacks it")
        return c2.view(torch.float8_e4m3fnuz), c2s
    return c2.view(torch.int8), c2s


def double_quantize(tensor: torch.Tensor, blocksize_1: int = 64, blocksize_2: int = 256
                    ) -> DoubleQuantState:
    """NF4 quantization, then quantization of its absmax (double_quant.py:46-97).
    No mean offset is subtracted from c1 (the reference subtracts none)."""
    original_shape = tensor.shape
    src, home = to_gpu(tensor)
    packed, c1 = quantize_int4(src, block_size=blocksize_1)
    use_fp8 = _has_fp8()
    c2, c2s = dq_quantize_absmax(c1, blocksize_2, use_fp8)
    return DoubleQuantState(
        W_quant=packed.to(home),
        c2=c2.to(home),
        c2_scales=_squeeze_scales(c2s).to(home),
        blocksize_1=blocksize_1,
        blocksize_2=blocksize_2,
        original_shape=original_shape,
        use_fp8_c2=use_fp8,
    )


def dq_dequantize_to(packed: torch.Tensor, c2: torch.Tensor, c2_scales: torch.Tensor,
                     blocksize_1: int, blocksize_2: int, use_fp8_c2: bool,
                     out_dtype: torch.dtype, n_out: int) -> torch.Tensor:
    """GPU-only: first n_out weights of double_dequantize, rounded to out_dtype."""
    dev = nat.require_gpu(packed, c2, c2_scales)
    with on(dev):
        p = packed.contiguous().view(-1)
        codes = c2.contiguous().view(-1).view(torch.uint8)
        s2 = c2_scales.contiguous().view(-1)
        if 2 * p.numel() % blocksize_1:
            raise RuntimeError("packed size is not a whole number of blocks")
        nb1 = 2 * p.numel() // blocksize_1
        if codes.numel() < nb1 or s2.numel() * blocksize_2 < nb1:
            raise RuntimeError("c2 / c2_scales too short for the packed weights")
        out = torch.empty((n_out,), dtype=out_dtype, device=dev)
        if n_out:
            nat.call("rq_dq_dequantize", p.data_ptr(), codes.data_ptr(), _c2_format(use_fp8_c2),
                     s2.data_ptr(), nat.dtype_code(s2.dtype), p.numel(), blocksize_1, blocksize_2,
                     out.data_ptr(), nat.dtype_code(out_dtype), n_out, nat.stream_handle(dev))
    return out


def double_dequantize(state: DoubleQuantState) -> torch.Tensor:
    """fp32 weights reshaped to original_shape (double_quant.py:99-122)."""
    p, home = to_gpu(state.W_quant)
    numel = 1
    for d in state.original_shape:
        numel *= int(d)
    out = dq_dequantize_to(p, state.c2.to(p.device), state.c2_scales.to(p.device),
                           state.blocksize_1, state.blocksize_2, state.use_fp8_c2,
                           torch.float32, numel)
    return out.reshape(state.original_shape).to(home)


def estimate_double_quant_savings(tensor: torch.Tensor, blocksize_1: int = 64,
                                  blocksize_2: int = 256) -> Dict[str, Any]:
    """Byte accounting of NF4 with and without double quantization
    (double_quant.py:124-158): fp32 c1 vs 1-byte c2 + fp32 c2_scales."""
    n = tensor.numel()
    nb1 = -(-n // blocksize_1)
    nb2 = -(-nb1 // blocksize_2)
    nf4_bytes = (n + 1) // 2
    naive = nf4_bytes + 4 * nb1
    dq = nf4_bytes + nb1 + 4 * nb2
    saved = naive - dq
    return {
        "without_dq_bytes": naive,
        "with_dq_bytes": dq,
        "saved_bytes": saved,
        "saved_pct": saved / naive * 100,
        "bits_saved_per_param": (naive - dq) * 8 / n,
    }


def patch_quant_linear_for_double_quant(model: nn.Module) -> int:
    """Upgrade every 4-bit QuantLinear to double quantization
    (double_quant.py:160-200): dequantize to fp32, re-run double_quantize,
    register c2 / c2_scales, empty weight_scales."""
    from rocm_qlora.quantization.quant_linear import QuantLinear

    targets = [m for _, m in model.named_modules() if isinstance(m, QuantLinear) and m.bits == 4]
    for m in targets:
        p, home = to_gpu(m.weight_quant)
        n = m.out_features * m.in_features
        w = nf4_dequantize_to(p, m.weight_scales.to(p.device), m.block_size, torch.float32, n)
        state = double_quantize(w.reshape(m.original_shape), blocksize_1=m.block_size, blocksize_2=256)
        m.register_buffer("c2", state.c2.to(home))
        m.register_buffer("c2_scales", state.c2_scales.to(home))
        m.blocksize_2 = state.blocksize_2
        m.use_fp8_c2 = state.use_fp8_c2
        m.use_double_quant = True
        # weight_quant keeps the original codes (re-quantizing dequantized NF4
        # weights reproduces them); weight_scales becomes an empty dummy
        del m.weight_scales
        m.register_buffer("weight_scales", torch.empty(0))
    return len(targets)
