"""FP8 compute for LoRA layers (fp8/fp8_linear.py of the reference).

Storage stays QuantLinear (NF4 / INT8); the base matmul runs in e4m3fnuz
with per-tensor scales on the gfx950 FP8 kernels: x and W are quantized
with scale = fp32(max|t| / 240) and codes = fnuz(RND(t / scale)), their
products are summed in fp32, scaled by x_scale * w_scale and rounded to x's
dtype, then the bias is added (fp8_linear.py:27-60).  Backward gives dX =
dY . W (the base weight is frozen) from the stored NF4 / INT8 codes by the
HIP dX kernels, whose weight operand is the dequantized weight rounded to
dY's dtype -- the reference's `grad_output @ w.to(grad_output.dtype)`.
The LoRA term stays in x's dtype.
"""
from __future__ import annotations

import contextlib
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from rocm_qlora import ops
from rocm_qlora import torch_ops
from rocm_qlora.fp8.fp8_config import detect_fp8_support, FP8Config
from rocm_qlora.lora.lora_layer import LoRALinear

_FNUZ_MAX = 240.0


def _fp8_forward(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor],
                 w_q: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> torch.Tensor:
    # 16-bit activations run on the fp8 matrix cores; fp32 activations on the
    # generic kernels, which decode both code matrices and sum the fp32
    # products (fp8_linear.py:44-52)
    wc, ws = w_q if w_q is not None else torch_ops.call_fp8_quantize(w)
    return torch_ops.call_fp8_linear(x, wc, ws, bias)


class _FP8LinearFunc(torch.autograd.Function):
    """FP8 forward, dX = dY . W backward (fp8_linear.py:19-67).  w_q: the
    weight's FP8 codes and scale (or None: w_fp16 is quantized here); qw: the
    layer's quantized weight (NF4Weight or Int8Weight) the FP8 codes were
    made from, which the backward multiplies by."""

    @staticmethod
    def forward(ctx, x, w_fp16, bias, w_q, qw):
        ctx.qw = qw
        ctx.has_bias = bias is not None
        ctx.fp8_used = True
        return _fp8_forward(x, w_fp16, bias, w_q)

    @staticmethod
    def backward(ctx, grad_output):
        from rocm_qlora.kernels.dequant_matmul import NF4Weight
        qw = ctx.qw
        if not qw.kernel_ok(grad_output.dtype):
            raise TypeError(f"FP8 backward takes fp32/bf16/fp16 gradients, got {grad_output.dtype}")
        if isinstance(qw, NF4Weight):
            dx = torch_ops.call_nf4_linear_dx(grad_output, qw.packed, qw.scales, qw.K, qw.block_size,
                                              **qw.dq_kwargs())
        else:
            dx = torch_ops.call_int8_linear_dx(grad_output, qw.q, qw.scales, qw.K, qw.block_size)
        return dx, None, None, None, None


class FP8LinearWrapper(nn.Module):
    """Runs a LoRALinear's base matmul in FP8 (fp8_linear.py:69-118).  Backend
    'native' (this package's FP8 kernels) when FP8 is supported and enabled,
    else 'bf16' (the wrapped layer unchanged).  The reference's third
    backend, TransformerEngine, is not dispatched to: there is one FP8 code
    path.  The FP8 weight codes are cached, in the matrix cores' e4m3fn
    encoding, until the stored weight changes; the dequantized 16-bit weight
    they come from is not kept (the backward multiplies by the stored codes)."""

    def __init__(self, base_lora_linear: nn.Module, config: Optional[FP8Config] = None):
        super().__init__()
        self.config = config if config is not None else FP8Config()
        self.base = base_lora_linear
        self.fp8_info = detect_fp8_support()
        if self.config.enabled and self.fp8_info["fp8_supported"] and self.fp8_info["fp8_dtypes_available"]:
            self.backend = "native"
        else:
            self.backend = "bf16"
        self._cache_key = None
        self._cache = None

    def _weight(self, dtype: torch.dtype):
        ql = self.base.base_layer
        key = (ql.weight_quant.data_ptr(), ql.weight_quant._version, dtype,
               getattr(ql, "c2", ql.weight_scales).data_ptr())
        if self._cache_key != key:
            codes, scale = ops.fp8_quantize(ql.dequantized_weight(dtype))
            self._cache = (ops.fp8_to_e4m3fn(codes), scale)
            self._cache_key = key
        return self._cache

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.backend == "native":
            ql = self.base.base_layer
            w_q = self._weight(x.dtype)
            bias = ql.bias.to(x.dtype) if ql.bias is not None else None
            qw = ql.nf4_weight() if ql.bits == 4 else ql.int8_weight()
            base_out = _FP8LinearFunc.apply(x, None, bias, w_q, qw)
            lora_out = (self.base.lora_dropout(x) @ self.base.lora_A.t().to(x.dtype)
                        @ self.base.lora_B.t().to(x.dtype) * self.base.scaling)
            return base_out + lora_out.to(base_out.dtype)
        return self.base(x)

    def extra_repr(self) -> str:
        return f"backend={self.backend}, fp8_supported={self.fp8_info['fp8_supported']}"


def wrap_model_for_fp8(model: nn.Module, config: Optional[FP8Config] = None) -> Tuple[nn.Module, Dict[str, Any]]:
    """Wrap every LoRALinear in an FP8LinearWrapper (fp8_linear.py:120-160).
    Unlike the reference, no environment variables are set: the FP8 kernels
    need no NCCL stream priority or hardware-queue settings."""
    config = config if config is not None else FP8Config()
    info = detect_fp8_support()
    status = {"enabled": False, "backend": "bf16", "layers_wrapped": 0, "reason": info["reason"]}
    if not info["fp8_supported"] and config.enabled:
        return model, status
    targets = [(n, m) for n, m in model.named_modules() if isinstance(m, LoRALinear)]
    for name, module in targets:
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        wrapped = FP8LinearWrapper(module, config)
        setattr(parent, child, wrapped)
        status["layers_wrapped"] += 1
        status["backend"] = wrapped.backend
        status["enabled"] = wrapped.backend != "bf16"
    return model, status


def enable_fp8_autocast(model: nn.Module, config: Optional[FP8Config] = None):
    """A null context (fp8_linear.py:164-174 enters TransformerEngine's
    fp8_autocast when TE is importable; here FP8 runs only through
    FP8LinearWrapper's own kernels, which need no autocast region)."""
    return contextlib.nullcontext()
