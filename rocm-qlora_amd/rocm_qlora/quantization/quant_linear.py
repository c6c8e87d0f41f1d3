"""QuantLinear: a linear layer whose weight is stored quantized
(quantization/quant_linear.py:16-200 of the reference).

Same constructor, buffers (weight_quant, weight_scales, weight_zeros, bias,
merged_fp16_weight), flat layouts, flags and state_dict keys as the
reference, so checkpoints and model surgery carry over unchanged.  The
forward pass is the HIP kernels': the weight is never materialised for bf16 /
fp16 activations with K % 64 == 0 -- it is dequantized inside the GEMV / GEMM
-- and the shapes the specialized kernels do not take (any K and block
size, fp32 activations) run the generic HIP dequantize-and-multiply kernel.
Inputs must be on the GPU.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from rocm_qlora.quantization.quant_ops import quantize_int8, quantize_int4


class QuantLinear(nn.Module):
    """Linear layer with an INT8 (blockwise absmax) or NF4 (blockwise absmax,
    optionally double-quantized) weight held in buffers."""

    def __init__(self, in_features: int, out_features: int, bits: int = 8, bias: bool = True,
                 block_size: int = 64):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.block_size = block_size
        self.original_shape: Optional[Tuple[int, ...]] = (out_features, in_features)
        # buffers, not parameters: the optimizer never sees them, .to() moves them
        self.register_buffer("weight_quant", torch.empty(0, dtype=torch.int8 if bits == 8 else torch.uint8))
        self.register_buffer("weight_scales", torch.empty(0))
        self.register_buffer("weight_zeros", torch.zeros(1))  # reserved (asymmetric schemes)
        if bias:
            self.register_buffer("bias", torch.zeros(out_features))
        else:
            self.bias = None
        # Compatibility flags of the reference (quant_linear.py:46-50).  The
        # HIP kernels are the only execution path; the flags record whether
        # enable_kernel() / enable_hip_kernels() were called.
        self.use_triton_kernel: bool = False
        self.use_hip_kernel: bool = False
        self.use_double_quant: bool = False
        self.register_buffer("merged_fp16_weight", None)
        self.merged_mode: bool = False

    @classmethod
    def from_linear(cls, linear: nn.Linear, bits: int = 8, block_size: int = 64) -> "QuantLinear":
        """Quantize an nn.Linear (quant_linear.py:56-98): the flattened weight
        goes through quantize_int8 (blockwise) or quantize_int4; the source
        layer's weight and bias are deleted to free memory."""
        if bits not in (4, 8):
            raise ValueError(f"Unsupported bit depth: {bits}")
        inst = cls(linear.in_features, linear.out_features, bits=bits, bias=linear.bias is not None,
                   block_size=block_size)
        inst.original_shape = tuple(linear.weight.shape)
        flat = linear.weight.data.flatten()
        if bits == 8:
            q, s = quantize_int8(flat, block_size=block_size)
        else:
            q, s = quantize_int4(flat, block_size=block_size)
        inst.weight_quant = q
        inst.weight_scales = s
        if linear.bias is not None:
            inst.bias = linear.bias.data.clone()
        del linear.weight
        if linear.bias is not None:
            del linear.bias
        return inst

    @classmethod
    def empty_quantized(cls, in_features: int, out_features: int, bits: int = 8, bias: bool = True,
                        block_size: int = 64, dtype: torch.dtype = torch.float32,
                        device: Optional[torch.device] = None) -> "QuantLinear":
        """A layer whose buffers have the shapes and dtypes from_linear gives
        a `dtype` weight (codes [numel_padded] int8 or [numel_padded / 2]
        uint8, squeezed absmax in `dtype`, bias in `dtype`), uninitialised:
        the target of a state_dict saved after quantization."""
        if bits not in (4, 8):
            raise ValueError(f"Unsupported bit depth: {bits}")
        if bits == 4 and (block_size < 2 or block_size % 2):
            raise ValueError(f"block_size must be even and >= 2, got {block_size}")
        if bits == 8 and block_size < 1:
            raise ValueError("block_size must be >= 1")
        inst = cls(in_features, out_features, bits=bits, bias=bias, block_size=block_size)
        nb = -(-in_features * out_features // block_size)
        n_codes = nb * block_size if bits == 8 else nb * block_size // 2
        inst.weight_quant = torch.empty((n_codes,), dtype=torch.int8 if bits == 8 else torch.uint8, device=device)
        inst.weight_scales = torch.empty((nb,), dtype=dtype, device=device).view(-1, 1).squeeze()
        inst.weight_zeros = torch.zeros(1, device=device)
        if bias:
            inst.bias = torch.zeros(out_features, dtype=dtype, device=device)
        return inst

    def enable_kernel(self) -> bool:
        """Mark the layer as running the fused HIP kernels (quant_linear.py:100-106).
        True when the native library is present."""
        from rocm_qlora import _native
        if _native.available():
            self.use_triton_kernel = True
            self.use_hip_kernel = True
            return True
        return False

    def enable_double_quant(self) -> bool:
        """Re-quantize the NF4 absmax (quant_linear.py:108-119)."""
        from rocm_qlora.quantization.double_quant import patch_quant_linear_for_double_quant

        class _Holder(nn.Module):
            def __init__(self, layer):
                super().__init__()
                self.layer = layer

        return patch_quant_linear_for_double_quant(_Holder(self)) > 0

    # -- kernels' view of the stored weight ---------------------------------
    def nf4_weight(self):
        from rocm_qlora.kernels.dequant_matmul import NF4Weight
        if self.use_double_quant:
            if not hasattr(self, "c2") or not hasattr(self, "c2_scales"):
                raise RuntimeError("Double quantization attributes not initialized. "
                                   "Call patch_quant_linear_for_double_quant() first.")
            return NF4Weight(self.weight_quant, None, self.out_features, self.in_features, self.block_size,
                             c2=self.c2, c2_scales=self.c2_scales, blocksize_2=self.blocksize_2,
                             use_fp8_c2=self.use_fp8_c2)
        return NF4Weight(self.weight_quant, self.weight_scales, self.out_features, self.in_features,
                         self.block_size)

    def int8_weight(self):
        from rocm_qlora.kernels.dequant_matmul import Int8Weight
        return Int8Weight(self.weight_quant, self.weight_scales, self.out_features, self.in_features,
                          self.block_size)

    def dequantized_weight(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """[out, in] weight as the reference's forward reconstructs it
        (quant_linear.py:168-193), rounded to `dtype`."""
        w = self.nf4_weight() if self.bits == 4 else self.int8_weight()
        return w.dense(dtype)

    def merged_weight(self, lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
                      scaling: float = 0.0, mode: str = "sum_then_round",
                      dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """[out, in] 16-bit weight of the dequantized weight plus (B @ A) *
        scaling, from the quantized buffers in one kernel (ops.merge_lora:
        "sum_then_round" as merge_lora rounds, "round_then_sum" as the export
        path does)."""
        from rocm_qlora import ops
        dq = self.bits == 4 and self.use_double_quant
        return ops.merge_lora(self.weight_quant, self.c2_scales if dq else self.weight_scales, self.out_features,
                              self.in_features, self.block_size, lora_a, lora_b, scaling, bits=self.bits,
                              c2=self.c2 if dq else None, use_fp8_c2=getattr(self, "use_fp8_c2", True),
                              blocksize_2=getattr(self, "blocksize_2", 256), mode=mode, out_dtype=dtype)

    def fused_forward(self, x: torch.Tensor, lora_a: Optional[torch.Tensor] = None,
                      lora_b: Optional[torch.Tensor] = None, scaling: float = 0.0,
                      dropout_p: float = 0.0) -> torch.Tensor:
        """Quantized linear with the LoRA term (its input through dropout of
        probability dropout_p when > 0) in the same kernel sequence (NF4);
        INT8 adds the LoRA term after the int8 kernel."""
        from rocm_qlora.kernels import dequant_matmul as dm
        if self.bits == 4:
            return dm.nf4_linear(x, self.nf4_weight(), self.bias, lora_a, lora_b, scaling, dropout_p)
        y = dm.int8_linear(x, self.int8_weight(), self.bias)
        if lora_a is not None and lora_b is not None and lora_a.shape[0] > 0:
            xl = torch.nn.functional.dropout(x, dropout_p, True) if dropout_p > 0.0 else x
            y = y + dm._lora_term(xl, lora_a, lora_b, scaling).to(y.dtype)
        return y

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """y = x . W^T + bias in x's dtype, any leading dims (quant_linear.py:121-197)."""
        if self.merged_mode and self.merged_fp16_weight is not None:
            weight = self.merged_fp16_weight.to(x.dtype)
            bias = self.bias.to(x.dtype) if self.bias is not None else None
            return F.linear(x, weight, bias)
        return self.fused_forward(x)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, bits={self.bits}, block_size={self.block_size}"
