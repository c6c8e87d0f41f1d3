"""The HIP entry points as PyTorch custom operators (torch.library).

Registered under the `rocm_qlora` namespace, each with a fake (meta)
implementation for shape and dtype inference, so that torch.compile traces
QuantLinear / LoRALinear forwards and backwards through them as single graph
nodes instead of breaking the graph at every ctypes call:

    torch.ops.rocm_qlora.nf4_linear      ops.nf4_linear
    torch.ops.rocm_qlora.nf4_linear_dx   ops.nf4_linear_dx
    torch.ops.rocm_qlora.int8_linear     ops.int8_linear
    torch.ops.rocm_qlora.fp8_quantize    ops.fp8_quantize
    torch.ops.rocm_qlora.fp8_linear      ops.fp8_linear
    torch.ops.rocm_qlora.int8_linear_w8a8  ops.int8_linear_w8a8

Every operator returns new tensors and mutates none of its inputs.  Eager
calls in this package go to the `ops` functions directly (the dispatcher
round trip would only add host time); code being traced by torch.compile
goes through these operators (`call`).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from rocm_qlora import ops


@torch.library.custom_op("rocm_qlora::nf4_linear", mutates_args=())
def nf4_linear(x: Tensor, weight_quant: Tensor, weight_scales: Optional[Tensor], out_features: int,
               block_size: int, bias: Optional[Tensor], c2: Optional[Tensor], c2_scales: Optional[Tensor],
               blocksize_2: int, use_fp8_c2: bool, lora_a: Optional[Tensor], lora_b: Optional[Tensor],
               scaling: float, lora_x: Optional[Tensor]) -> Tensor:
    return ops.nf4_linear(x, weight_quant, weight_scales, out_features, block_size, bias, c2=c2,
                          c2_scales=c2_scales, blocksize_2=blocksize_2, use_fp8_c2=use_fp8_c2,
                          lora_a=lora_a, lora_b=lora_b, scaling=scaling, lora_x=lora_x)


@nf4_linear.register_fake
def _nf4_linear_fake(x, weight_quant, weight_scales, out_features, block_size, bias, c2, c2_scales,
                     blocksize_2, use_fp8_c2, lora_a, lora_b, scaling, lora_x):
    return x.new_empty((*x.shape[:-1], out_features))


@torch.library.custom_op("rocm_qlora::nf4_linear_dx", mutates_args=())
def nf4_linear_dx(dy: Tensor, weight_quant: Tensor, weight_scales: Optional[Tensor], in_features: int,
                  block_size: int, c2: Optional[Tensor], c2_scales: Optional[Tensor], blocksize_2: int,
                  use_fp8_c2: bool, lora_a: Optional[Tensor], lora_b: Optional[Tensor], scaling: float,
                  lora_mask: Optional[Tensor], mask_scale: float) -> Tensor:
    return ops.nf4_linear_dx(dy, weight_quant, weight_scales, in_features, block_size, c2=c2,
                             c2_scales=c2_scales, blocksize_2=blocksize_2, use_fp8_c2=use_fp8_c2,
                             lora_a=lora_a, lora_b=lora_b, scaling=scaling, lora_mask=lora_mask,
                             mask_scale=mask_scale)


@nf4_linear_dx.register_fake
def _nf4_linear_dx_fake(dy, weight_quant, weight_scales, in_features, block_size, c2, c2_scales, blocksize_2,
                        use_fp8_c2, lora_a, lora_b, scaling, lora_mask, mask_scale):
    return dy.new_empty((*dy.shape[:-1], in_features))


@torch.library.custom_op("rocm_qlora::int8_linear", mutates_args=())
def int8_linear(x: Tensor, q: Tensor, scales: Tensor, out_features: int, block_size: int,
                bias: Optional[Tensor]) -> Tensor:
    return ops.int8_linear(x, q, scales, out_features, block_size, bias)


@int8_linear.register_fake
def _int8_linear_fake(x, q, scales, out_features, block_size, bias):
    return x.new_empty((*x.shape[:-1], out_features))


@torch.library.custom_op("rocm_qlora::int8_linear_dx", mutates_args=())
def int8_linear_dx(dy: Tensor, q: Tensor, scales: Tensor, in_features: int, block_size: int) -> Tensor:
    return ops.int8_linear_dx(dy, q, scales, in_features, block_size)


@int8_linear_dx.register_fake
def _int8_linear_dx_fake(dy, q, scales, in_features, block_size):
    return dy.new_empty((*dy.shape[:-1], in_features))


@torch.library.custom_op("rocm_qlora::fp8_quantize", mutates_args=())
def fp8_quantize(t: Tensor) -> Tuple[Tensor, Tensor]:
    return ops.fp8_quantize(t)


@fp8_quantize.register_fake
def _fp8_quantize_fake(t):
    rows = 1
    for d in t.shape[:-1]:
        rows *= d
    return (t.new_empty((rows, t.shape[-1]), dtype=torch.float8_e4m3fnuz),
            t.new_empty((), dtype=torch.float32))


@torch.library.custom_op("rocm_qlora::fp8_linear", mutates_args=())
def fp8_linear(x: Tensor, w_codes: Tensor, w_scale: Tensor, bias: Optional[Tensor]) -> Tensor:
    return ops.fp8_linear(x, w_codes, w_scale, bias)


@fp8_linear.register_fake
def _fp8_linear_fake(x, w_codes, w_scale, bias):
    n = w_codes.numel() // x.shape[-1]
    return x.new_empty((*x.shape[:-1], n))


@torch.library.custom_op("rocm_qlora::int8_linear_w8a8", mutates_args=())
def int8_linear_w8a8(x: Tensor, q: Tensor, scales: Tensor, bias: Optional[Tensor]) -> Tensor:
    return ops.int8_linear_w8a8(x, q, scales, bias)


@int8_linear_w8a8.register_fake
def _int8_linear_w8a8_fake(x, q, scales, bias):
    n = q.numel() // x.shape[-1]
    return x.new_empty((*x.shape[:-1], n))


def _compiling() -> bool:
    try:
        return torch.compiler.is_compiling()
    except AttributeError:  # older torch
        return False


def call_nf4_linear(x, weight_quant, weight_scales, out_features, block_size=64, bias=None, *, c2=None,
                    c2_scales=None, blocksize_2=256, use_fp8_c2=True, lora_a=None, lora_b=None, scaling=0.0,
                    lora_x=None):
    """ops.nf4_linear, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.nf4_linear(x, weight_quant, weight_scales, int(out_features), int(block_size),
                                               bias, c2, c2_scales, int(blocksize_2), bool(use_fp8_c2), lora_a,
                                               lora_b, float(scaling), lora_x)
    return ops.nf4_linear(x, weight_quant, weight_scales, out_features, block_size, bias, c2=c2,
                          c2_scales=c2_scales, blocksize_2=blocksize_2, use_fp8_c2=use_fp8_c2, lora_a=lora_a,
                          lora_b=lora_b, scaling=scaling, lora_x=lora_x)


def call_nf4_linear_dx(dy, weight_quant, weight_scales, in_features, block_size=64, *, c2=None, c2_scales=None,
                       blocksize_2=256, use_fp8_c2=True, lora_a=None, lora_b=None, scaling=0.0, lora_mask=None,
                       mask_scale=1.0):
    """ops.nf4_linear_dx, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.nf4_linear_dx(dy, weight_quant, weight_scales, int(in_features),
                                                  int(block_size), c2, c2_scales, int(blocksize_2),
                                                  bool(use_fp8_c2), lora_a, lora_b, float(scaling), lora_mask,
                                                  float(mask_scale))
    return ops.nf4_linear_dx(dy, weight_quant, weight_scales, in_features, block_size, c2=c2, c2_scales=c2_scales,
                             blocksize_2=blocksize_2, use_fp8_c2=use_fp8_c2, lora_a=lora_a, lora_b=lora_b,
                             scaling=scaling, lora_mask=lora_mask, mask_scale=mask_scale)


def call_int8_linear(x, q, scales, out_features, block_size=0, bias=None):
    """ops.int8_linear, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.int8_linear(x, q, scales, int(out_features), int(block_size), bias)
    return ops.int8_linear(x, q, scales, out_features, block_size, bias)


def call_int8_linear_dx(dy, q, scales, in_features, block_size=0):
    """ops.int8_linear_dx, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.int8_linear_dx(dy, q, scales, int(in_features), int(block_size))
    return ops.int8_linear_dx(dy, q, scales, in_features, block_size)


def call_fp8_quantize(t):
    """ops.fp8_quantize, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.fp8_quantize(t)
    return ops.fp8_quantize(t)


def call_fp8_linear(x, w_codes, w_scale, bias=None):
    """ops.fp8_linear, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.fp8_linear(x, w_codes, w_scale, bias)
    return ops.fp8_linear(x, w_codes, w_scale, bias)


def call_int8_linear_w8a8(x, q, scales, bias=None):
    """ops.int8_linear_w8a8, through the registered operator while being traced."""
    if _compiling():
        return torch.ops.rocm_qlora.int8_linear_w8a8(x, q, scales, bias)
    return ops.int8_linear_w8a8(x, q, scales, bias)
