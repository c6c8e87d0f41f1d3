"""LoRALinear: trainable low-rank adapters on a QuantLinear
(lora/lora_layer.py:16-132 of the reference).

y = base(x) + ((drop(x) @ A^T) @ B^T * s).to(base dtype), s = alpha / r,
A [r, in] Kaiming-uniform(a=sqrt 5), B [out, r] zeros.  With an NF4 base on
the GPU, the adapter term runs inside the quantized linear's kernel sequence
(the LoRA epilogue of the GEMV / GEMM) -- with active dropout, on drop(x),
whose mask the dX kernel applies in the backward pass -- and the backward
pass runs the fused NF4 dX kernel plus two small library GEMMs for dA and
dB.  Otherwise the base layer and the adapter are composed as in the
reference.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from rocm_qlora.quantization.quant_linear import QuantLinear


class LoRALinear(nn.Module):
    """Wraps a QuantLinear with LoRA adapters; merge_lora folds them into an
    fp16 copy of the weight for inference."""

    def __init__(self, quant_linear: QuantLinear, r: int = 8, lora_alpha: int = 16, lora_dropout: float = 0.0):
        super().__init__()
        self.base_layer = quant_linear
        self.r = r
        self.lora_alpha = lora_alpha
        self.merged = False
        for p in self.base_layer.parameters():
            p.requires_grad_(False)
        # initialised on the CPU generator (as the reference does), then placed
        # beside the quantized weight
        dev = quant_linear.weight_quant.device
        a = torch.empty(r, quant_linear.in_features)
        nn.init.kaiming_uniform_(a, a=math.sqrt(5))
        self.lora_A = nn.Parameter(a.to(dev))
        self.lora_B = nn.Parameter(torch.zeros(quant_linear.out_features, r, device=dev))
        self.scaling = lora_alpha / r
        self.lora_dropout = nn.Dropout(p=lora_dropout) if lora_dropout > 0.0 else nn.Identity()

    def _dropout_active(self) -> bool:
        return isinstance(self.lora_dropout, nn.Dropout) and self.training and self.lora_dropout.p > 0.0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """base_output + (x @ A^T @ B^T * scaling), lora_layer.py:51-70."""
        if self.merged:
            return self.base_layer(x)
        base = self.base_layer
        if isinstance(base, QuantLinear) and not base.merged_mode:
            p = self.lora_dropout.p if self._dropout_active() else 0.0
            return base.fused_forward(x, self.lora_A, self.lora_B, self.scaling, p)
        if hasattr(base, "weight"):
            base_out = base(x.to(base.weight.dtype))
        else:
            base_out = base(x)
        lora_out = self.lora_dropout(x) @ self.lora_A.to(x.dtype).T @ self.lora_B.to(x.dtype).T * self.scaling
        return base_out + lora_out.to(base_out.dtype)

    @torch.no_grad()
    def merge_lora(self) -> None:
        """Store fp16(W_deq + B @ A * s) as the base layer's merged weight
        (lora_layer.py:72-113).  No re-quantization.  Unlike the reference,
        the dequantization honours double quantization and the adapters are
        kept (the reference zeroes A and B, lora_layer.py:111-113, so its
        unmerge_lora cannot restore the adapted layer; here it does)."""
        if self.merged:
            raise RuntimeError("LoRA already merged")
        # one kernel: RND_fp16(W_deq + RND(RND(B @ A) * s)) from the quantized
        # buffers (double quantization included)
        merged = self.base_layer.merged_weight(self.lora_A, self.lora_B, self.scaling, "sum_then_round",
                                               torch.float16)
        self.base_layer.merged_fp16_weight = merged
        self.base_layer.merged_mode = True
        self.merged = True

    def unmerge_lora(self) -> None:
        """Drop the merged fp16 weight (lora_layer.py:115-128); the adapters,
        kept by merge_lora, apply again."""
        if not self.merged:
            raise RuntimeError("LoRA is not merged — nothing to unmerge")
        self.base_layer.merged_fp16_weight = None
        self.base_layer.merged_mode = False
        self.merged = False

    def get_trainable_params(self) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad)

    def extra_repr(self) -> str:
        return f"r={self.r}, alpha={self.lora_alpha}, scaling={self.scaling:.4f}, merged={self.merged}"
