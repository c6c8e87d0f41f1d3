"""Fused dequantize + matmul for NF4 and INT8 weights, with autograd
(kernels/dequant_matmul.py:214-376 of the reference).

Forward runs the HIP kernels of this package: a weight-streaming GEMV for up
to 16 activation rows, the MFMA GEMM above that, both with bias and the LoRA
term fused.  Backward returns dX only, as the reference does
(dequant_matmul.py:338-351), plus dA / dB when LoRA adapters are passed:
dX = dY . W_deq (+ ((dY * s) . B) . A) by the NF4 dX kernel.

Every shape, block size and activation dtype (fp32 included) runs on the
library's HIP kernels: shapes the specialized kernels do not take (K not a
multiple of 64, block sizes that are not powers of two >= 64 dividing K,
unaligned rows) run on its generic kernels, which decode the weight inside
the multiply with the same roundings as the reference's
dequantize-then-F.linear path.  INT8 backward is dX = dY . W_deq on those
kernels too.  Tensors on the CPU raise; there is no CPU or library path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from rocm_qlora import _native as nat
from rocm_qlora import torch_ops

# activation dtypes of the HIP linear kernels
_KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


@dataclass
class NF4Weight:
    """An NF4 weight as QuantLinear stores it: flat packed codes (byte j =
    element 2j low nibble, 2j+1 high nibble) and one absmax per block, or,
    with double quantization, c2 codes plus c2_scales per blocksize_2 blocks."""
    packed: torch.Tensor
    scales: Optional[torch.Tensor]
    N: int
    K: int
    block_size: int = 64
    c2: Optional[torch.Tensor] = None
    c2_scales: Optional[torch.Tensor] = None
    blocksize_2: int = 256
    use_fp8_c2: bool = True

    def kernel_ok(self, dtype: torch.dtype) -> bool:
        """The HIP kernels take this activation dtype (any shape)."""
        return dtype in _KERNEL_DTYPES

    def dq_kwargs(self) -> dict:
        if self.c2 is None:
            return {}
        return dict(c2=self.c2, c2_scales=self.c2_scales, blocksize_2=self.blocksize_2,
                    use_fp8_c2=self.use_fp8_c2)

    def dense(self, dtype: torch.dtype) -> torch.Tensor:
        """[N, K] dequantized weight in `dtype` (dequantize_int4 /
        double_dequantize, then `[:N*K].reshape(N, K).to(dtype)`,
        quant_linear.py:168-193), by the HIP codec kernels."""
        from rocm_qlora.quantization.quant_ops import nf4_dequantize_to
        from rocm_qlora.quantization.double_quant import dq_dequantize_to
        n = self.N * self.K
        if self.c2 is not None:
            w = dq_dequantize_to(self.packed, self.c2, self.c2_scales, self.block_size, self.blocksize_2,
                                 self.use_fp8_c2, dtype, n)
        else:
            w = nf4_dequantize_to(self.packed, self.scales, self.block_size, dtype, n)
        return w.view(self.N, self.K)


@dataclass
class Int8Weight:
    """An int8 weight: per-row scales (block_size 0, the row-absmax recipe,
    q [N, K] with [N] scales) or blockwise scales over the flat weight."""
    q: torch.Tensor
    scales: torch.Tensor
    N: int
    K: int
    block_size: int = 64

    def kernel_ok(self, dtype: torch.dtype) -> bool:
        """The HIP kernels take this activation dtype (any shape)."""
        return dtype in _KERNEL_DTYPES

    def dense(self, dtype: torch.dtype) -> torch.Tensor:
        """[N, K] dequantized weight (dequantize_int8, quant_ops.py:55-78), cast."""
        from rocm_qlora.quantization.quant_ops import dequantize_int8
        n = self.N * self.K
        if self.block_size == 0:
            w = dequantize_int8(self.q.reshape(self.N, self.K), self.scales.reshape(-1))
        else:
            w = dequantize_int8(self.q.reshape(-1), self.scales.reshape(-1), self.block_size)
        return w.reshape(-1)[:n].view(self.N, self.K).to(dtype)


def _lora_present(lora_a, lora_b) -> bool:
    return lora_a is not None and lora_b is not None and lora_a.shape[0] > 0


def _lora_term(x, lora_a, lora_b, scaling):
    """(x @ A^T @ B^T * s) in x's dtype (lora_layer.py:67)."""
    return x @ lora_a.to(x.dtype).T @ lora_b.to(x.dtype).T * scaling


class _FusedNF4LinearFunc(torch.autograd.Function):
    """y = x . W_deq^T + bias (+ LoRA) by the HIP kernels; backward gives dX
    (NF4 dX kernel, LoRA term fused) and the adapters' gradients.

    With LoRA dropout p > 0 the adapter reads drop(x) (lora_layer.py:67):
    the mask comes from torch's own dropout kernel (aten::native_dropout,
    the kernel nn.Dropout runs, so the random stream is the same), the
    forward passes drop(x) as the LoRA input of the fused kernels, and the
    dX kernel applies dropout's backward (mask / (1 - p)) to the adapter's
    input gradient in its epilogue."""

    @staticmethod
    def forward(ctx, x, lora_a, lora_b, bias, w: NF4Weight, scaling: float, dropout_p: float = 0.0):
        lora = _lora_present(lora_a, lora_b)
        xl = mask = None
        if lora and dropout_p > 0.0:
            xl, mask = torch.ops.aten.native_dropout(x, float(dropout_p), True)
        ctx.w = w
        ctx.scaling = float(scaling)
        ctx.lora = lora
        ctx.mask_scale = 1.0 / (1.0 - dropout_p) if mask is not None else 1.0
        ctx.save_for_backward(x if lora else None, lora_a if lora else None, lora_b if lora else None,
                              xl, mask)
        return torch_ops.call_nf4_linear(x, w.packed, w.scales, w.N, w.block_size, bias,
                                         lora_a=lora_a if lora else None, lora_b=lora_b if lora else None,
                                         scaling=scaling, lora_x=xl, **w.dq_kwargs())

    @staticmethod
    def backward(ctx, dy):
        x, A, B, xl, mask = ctx.saved_tensors
        w: NF4Weight = ctx.w
        s = ctx.scaling
        need_x, need_a, need_b = ctx.needs_input_grad[:3]
        dx = da = db = None
        if need_x:
            dx = torch_ops.call_nf4_linear_dx(dy, w.packed, w.scales, w.K, w.block_size,
                                              lora_a=A, lora_b=B, scaling=s, lora_mask=mask,
                                              mask_scale=ctx.mask_scale, **w.dq_kwargs())
        if ctx.lora and (need_a or need_b):
            # lora_out = ((xl A^T) B^T) * s in x's dtype, xl = drop(x) or x:
            # dv = dY * s, dB = dv^T (xl A^T), dA = (dv B)^T xl, cast to the
            # parameters' dtype
            dt = x.dtype
            x2 = (xl if xl is not None else x).reshape(-1, x.shape[-1])
            dv = dy.reshape(-1, dy.shape[-1]).to(dt) * s
            if need_b:
                u = x2 @ A.to(dt).T
                db = (dv.T @ u).to(B.dtype)
            if need_a:
                da = ((dv @ B.to(dt)).T @ x2).to(A.dtype)
        return dx, da, db, None, None, None, None


class _FusedInt8LinearFunc(torch.autograd.Function):
    """y = x . (q * s)^T + bias by the HIP int8 kernels; backward dX =
    dY . RND(W_deq) (dequant_matmul.py:308-324) by the HIP int8 dX kernel."""

    @staticmethod
    def forward(ctx, x, bias, w: Int8Weight):
        ctx.w = w
        return torch_ops.call_int8_linear(x, w.q, w.scales, w.N, w.block_size, bias)

    @staticmethod
    def backward(ctx, dy):
        if not ctx.needs_input_grad[0]:
            return None, None, None
        w: Int8Weight = ctx.w
        return torch_ops.call_int8_linear_dx(dy, w.q, w.scales, w.K, w.block_size), None, None


def nf4_linear(x: torch.Tensor, w: NF4Weight, bias: Optional[torch.Tensor] = None,
               lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
               scaling: float = 0.0, dropout_p: float = 0.0) -> torch.Tensor:
    """Autograd-aware NF4 linear (+ LoRA, its input through dropout of
    probability dropout_p when > 0) on the HIP kernels."""
    nat.require_gpu(x, w.packed)
    if not w.kernel_ok(x.dtype):
        raise TypeError(f"NF4 linear takes fp32/bf16/fp16 activations, got {x.dtype}")
    # the reference adds bias.to(x.dtype) (quant_linear.py:196)
    bias = bias.to(x.dtype) if bias is not None else None
    return _FusedNF4LinearFunc.apply(x, lora_a, lora_b, bias, w, scaling, float(dropout_p))


def int8_linear(x: torch.Tensor, w: Int8Weight, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Autograd-aware INT8 linear on the HIP kernels."""
    nat.require_gpu(x, w.q)
    if not w.kernel_ok(x.dtype):
        raise TypeError(f"INT8 linear takes fp32/bf16/fp16 activations, got {x.dtype}")
    bias = bias.to(x.dtype) if bias is not None else None
    return _FusedInt8LinearFunc.apply(x, bias, w)


def fused_dequant_nf4_matmul(x: torch.Tensor, w_packed: torch.Tensor, scales: torch.Tensor,
                             bias: Optional[torch.Tensor] = None, block_size: int = 64) -> torch.Tensor:
    """y = x . dequant_nf4(w)^T + bias (dequant_matmul.py:367-376).  w_packed
    is 1-D flat (N = numel * 2 // K) or 2-D [N, K // 2]; output has x's dtype
    and leading dims; differentiable in x (backward returns dX only)."""
    K = x.shape[-1]
    N = w_packed.numel() * 2 // K if w_packed.dim() == 1 else w_packed.shape[0]
    return nf4_linear(x, NF4Weight(w_packed.reshape(-1), scales, N, K, block_size), bias)


def fused_dequant_int8_matmul(x: torch.Tensor, w_int8: torch.Tensor, scales: torch.Tensor,
                              bias: Optional[torch.Tensor] = None, block_size: int = 64) -> torch.Tensor:
    """y = x . dequant_int8(w)^T + bias (dequant_matmul.py:356-365).  w_int8 is
    [N, K]; like dequantize_int8, one scale per row when scales.numel() == N,
    otherwise blockwise over the flat weight."""
    K = x.shape[-1]
    if w_int8.dim() != 2:
        raise ValueError(f"w_int8 must be [N, K], got shape {tuple(w_int8.shape)}")
    N = w_int8.shape[0]
    per_row = scales.numel() == N
    w = Int8Weight(w_int8, scales, N, K, 0 if per_row else block_size)
    return int8_linear(x, w, bias)
