"""Standalone NF4 dequantization to bf16 (kernels/nf4_dequant.py:80-115 of
the reference), run by the HIP codec kernel."""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from rocm_qlora.quantization.quant_ops import NF4_VALUES, dequantize_int4, nf4_dequantize_to

NF4_TABLE = torch.tensor(NF4_VALUES, dtype=torch.float32)


def dequantize_nf4_triton(packed: torch.Tensor, scales: torch.Tensor, block_size: int = 64,
                          original_shape: Optional[Tuple[int, ...]] = None) -> torch.Tensor:
    """GPU tensors: every packed code dequantized and rounded to bf16
    (RNE of T[code] * scale), viewed as original_shape when given.  CPU
    tensors: the fp32 result of dequantize_int4, as the reference returns
    for them.  The name is the reference's; no Triton is involved."""
    if packed.device.type != "cuda":
        return dequantize_int4(packed, scales, block_size)
    out = nf4_dequantize_to(packed, scales.to(packed.device), block_size, torch.bfloat16)
    return out.view(original_shape) if original_shape else out
