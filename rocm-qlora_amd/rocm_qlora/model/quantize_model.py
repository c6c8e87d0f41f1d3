"""Model surgery: nn.Linear -> LoRALinear(QuantLinear)
(model/quantize_model.py:36-142 of the reference)."""
from __future__ import annotations

import logging
from typing import Dict, List, Tuple

import torch
import torch.nn as nn

from rocm_qlora.quantization.quant_linear import QuantLinear
from rocm_qlora.lora.lora_layer import LoRALinear

logger = logging.getLogger("rocm_qlora.quantize_model")


def _get_parent_and_attr(model: nn.Module, full_name: str) -> Tuple[nn.Module, str]:
    parts = full_name.split(".")
    parent = model
    for p in parts[:-1]:
        parent = getattr(parent, p)
    return parent, parts[-1]


def estimate_model_memory(model: nn.Module, bits: int) -> Dict[str, float]:
    """fp16 vs quantized size of the model's parameters with 4-byte scales
    per 64 weights (utils/rocm_utils.py:53-83)."""
    total = sum(p.numel() for p in model.parameters())
    fp16_gb = total * 2 / 1024 ** 3
    quant_gb = total * (bits / 8.0 + 4 / 64) / 1024 ** 3
    reduction = (1 - quant_gb / fp16_gb) * 100 if fp16_gb else 0.0
    return {"fp16_gb": round(fp16_gb, 4), "quantized_gb": round(quant_gb, 4), "reduction_pct": round(reduction, 2)}


def print_model_summary(model: nn.Module) -> None:
    """Leaf modules with parameters: name, type, parameter count, trainable
    (utils/rocm_utils.py:85-105)."""
    print(f"{'Layer Name':<40} | {'Type':<20} | {'Params':<12} | {'Trainable':<10}")
    print("-" * 90)
    for name, module in model.named_modules():
        params = list(module.parameters(recurse=False))
        if next(module.children(), None) is None and params:
            n = sum(p.numel() for p in params)
            tr = any(p.requires_grad for p in params)
            print(f"{name[:40]:<40} | {type(module).__name__:<20} | {n:<12,} | {str(tr):<10}")


def _target_linears(model: nn.Module, target_modules: List[str]) -> List[Tuple[nn.Module, str, nn.Linear]]:
    """(parent, attribute, layer) of every nn.Linear whose name ends with one
    of target_modules and whose smaller side is >= 64 (quantize_model.py:58-70)."""
    found = []
    for name, module in model.named_modules():
        if isinstance(module, nn.Linear) and any(name.endswith(t) for t in target_modules):
            if min(module.in_features, module.out_features) < 64:
                logger.warning(f"Skipping layer '{name}' because it is too small "
                               f"({module.in_features}x{module.out_features} < 64)")
                continue
            parent, attr = _get_parent_and_attr(model, name)
            found.append((parent, attr, module))
    return found


def quantized_skeleton(model: nn.Module, bits: int = 8, lora_r: int = 8, lora_alpha: int = 16,
                       lora_dropout: float = 0.05, target_modules: List[str] = ["q_proj", "v_proj"],
                       block_size: int = 64, lora_dtype: torch.dtype = torch.float32) -> nn.Module:
    """The module tree quantize_model produces, without quantizing anything:
    every target nn.Linear becomes LoRALinear(QuantLinear.empty_quantized(...))
    on the layer's device (meta while transformers builds a model), with the
    buffer shapes and dtypes quantization of that layer's weight gives and
    `lora_dtype` adapters.  A state_dict saved after quantization then loads
    into it key for key (the reference reaches the same tree by quantizing the
    skeleton, hf_integration/quantizer.py:56-69)."""
    if bits not in (4, 8):
        raise ValueError(f"Invalid bit-depth: {bits}. Only 4 and 8 bits are supported.")
    model.requires_grad_(False)
    for parent, attr, linear in _target_linears(model, target_modules):
        w = linear.weight
        ql = QuantLinear.empty_quantized(linear.in_features, linear.out_features, bits=bits,
                                         bias=linear.bias is not None, block_size=block_size, dtype=w.dtype,
                                         device=w.device)
        ll = LoRALinear(ql, r=lora_r, lora_alpha=lora_alpha, lora_dropout=lora_dropout)
        ll.lora_A = nn.Parameter(ll.lora_A.detach().to(lora_dtype))
        ll.lora_B = nn.Parameter(ll.lora_B.detach().to(lora_dtype))
        setattr(parent, attr, ll)
    return model


def quantize_model(model: nn.Module, bits: int = 8, lora_r: int = 8, lora_alpha: int = 16,
                   lora_dropout: float = 0.05, target_modules: List[str] = ["q_proj", "v_proj"],
                   block_size: int = 64) -> nn.Module:
    """Freeze the model, then replace every nn.Linear whose name ends with one
    of target_modules (and whose smaller side is >= 64) by
    LoRALinear(QuantLinear.from_linear(...)), printing a summary."""
    if bits not in (4, 8):
        raise ValueError(f"Invalid bit-depth: {bits}. Only 4 and 8 bits are supported.")
    model.requires_grad_(False)
    replacements = _target_linears(model, target_modules)
    # one layer at a time, each source layer released once replaced, so the
    # peak holds one layer's 16-bit weight beside the quantized model
    replacements.reverse()
    while replacements:
        parent, attr, linear = replacements.pop()
        ql = QuantLinear.from_linear(linear, bits=bits, block_size=block_size)
        setattr(parent, attr, LoRALinear(ql, r=lora_r, lora_alpha=lora_alpha, lora_dropout=lora_dropout))
        del linear, ql

    print("\n--- Model Quantization Summary ---")
    print_model_summary(model)
    mem = estimate_model_memory(model, bits)
    total = sum(p.numel() for p in model.parameters())
    trainable = sum(p.numel() for p in model.parameters() if p.requires_grad)
    pct = trainable / total * 100 if total else 0.0
    print(f"\nTotal Parameters: {total:,}")
    print(f"Trainable Parameters: {trainable:,} ({pct:.4f}%)")
    print(f"Estimated FP16 VRAM: {mem['fp16_gb']:.4f} GB")
    print(f"Estimated Quantized VRAM: {mem['quantized_gb']:.4f} GB")
    print(f"Reduction: {mem['reduction_pct']:.2f}%")
    print("----------------------------------\n")
    return model


def enable_all_kernels(model: nn.Module) -> int:
    """enable_kernel() on every QuantLinear, bare or inside a LoRALinear;
    returns how many reported success (quantize_model.py:125-142)."""
    seen = set()
    count = 0
    for _, module in model.named_modules():
        target = None
        if isinstance(module, QuantLinear):
            target = module
        elif isinstance(getattr(module, "base_layer", None), QuantLinear):
            target = module.base_layer
        # a wrapped QuantLinear is met twice (as base_layer and as a module);
        # it is counted once
        if target is not None and id(target) not in seen:
            seen.add(id(target))
            if target.enable_kernel():
                count += 1
    return count
