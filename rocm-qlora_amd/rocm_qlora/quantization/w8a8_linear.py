"""W8A8Linear: the INT8 linear with int8 activations too.

No counterpart in the reference, whose INT8 QuantLinear multiplies 16-bit
activations by dequantized int8 weights (quant_linear.py:193-197).  Here the
weight is quantized once per row with quantize_int8(w, per_channel=True)
(quant_ops.py:29-35), each activation row is quantized the same way (in
fp32) on every call, and the int8 products are summed exactly in int32 by
gfx950's int8 matrix cores:

    y = RND(RND(float(sum_k xq wq) * x_scale[m] * w_scale[n]) + RND(bias))

It trades the activation rounding for twice the matrix-core rate of the
16-bit path; results are close to, not equal to, QuantLinear(bits=8).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from rocm_qlora import torch_ops
from rocm_qlora.quantization.quant_ops import quantize_int8


class W8A8Linear(nn.Module):
    """Linear layer with per-row int8 weights and per-row int8 activations."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight_quant", torch.empty(0, dtype=torch.int8))
        self.register_buffer("weight_scales", torch.empty(0, dtype=torch.float32))
        self.bias = nn.Parameter(torch.zeros(out_features), requires_grad=False) if bias else None

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "W8A8Linear":
        """Quantize an nn.Linear's weight per row (its fp32 values: scales are
        fp32 whatever the layer's dtype)."""
        m = cls(linear.in_features, linear.out_features, linear.bias is not None)
        q, s = quantize_int8(linear.weight.detach().float(), per_channel=True)
        m.weight_quant = q.reshape(linear.out_features, linear.in_features)
        m.weight_scales = s.reshape(-1).float()
        if linear.bias is not None:
            m.bias = nn.Parameter(linear.bias.detach().clone(), requires_grad=False)
        return m

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch_ops.call_int8_linear_w8a8(x, self.weight_quant, self.weight_scales, self.bias)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"
