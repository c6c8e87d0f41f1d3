"""Merged fp16 export (export/gguf_export.py:30-184 of the reference).

Each LoRALinear's weight is rebuilt as RND16(RND16(W_deq) + RND16((B @ A) *
scaling)) -- the dequantized base weight and the LoRA delta each rounded to
fp16, then added in fp16, with no re-quantization -- by one kernel that reads
the packed codes, the scales (double quantization included) and the adapters
(ops.merge_lora, mode "round_then_sum").  Every other parameter is copied as
fp16.  The file is written with safetensors (".safetensors") or torch.save.
"""
from __future__ import annotations

import json
import os
from typing import Any, Dict, Optional

import torch
import torch.nn as nn

from rocm_qlora.lora.lora_layer import LoRALinear


def _export_dequant_layer(lora_linear: nn.Module) -> torch.Tensor:
    """[out, in] fp16 merged weight of one LoRALinear (gguf_export.py:30-79)."""
    if not isinstance(lora_linear, LoRALinear):
        raise TypeError(f"Expected LoRALinear, got {type(lora_linear)}")
    return lora_linear.base_layer.merged_weight(lora_linear.lora_A, lora_linear.lora_B, lora_linear.scaling,
                                                "round_then_sum", torch.float16)


def _build_export_state_dict(model: nn.Module) -> Dict[str, torch.Tensor]:
    """fp16 state dict with merged LoRA weights under the layers' own keys
    ('<layer>.weight', '<layer>.bias') and no adapter keys
    (gguf_export.py:82-125)."""
    state_dict: Dict[str, torch.Tensor] = {}
    for name, param in model.named_parameters():
        if "lora_A" not in name and "lora_B" not in name:
            state_dict[name] = param.data.cpu().to(torch.float16)
    for name, module in model.named_modules():
        if isinstance(module, LoRALinear):
            state_dict[f"{name}.weight"] = _export_dequant_layer(module).cpu()
            if module.base_layer.bias is not None:
                state_dict[f"{name}.bias"] = module.base_layer.bias.data.cpu().to(torch.float16)
    return state_dict


def merge_and_export_fp16(model: nn.Module, output_path: str,
                          model_config: Optional[Dict[str, Any]] = None) -> str:
    """Write the merged fp16 weights to output_path (safetensors when it ends
    in '.safetensors', else torch.save) and model_config, if given, as
    config.json beside it (gguf_export.py:128-184).  Returns output_path."""
    model.eval()
    with torch.no_grad():
        state_dict = _build_export_state_dict(model)
        total = sum(v.numel() * v.element_size() for v in state_dict.values())
        print(f"[export] state dict: {len(state_dict)} tensors, {total / 1e9:.2f} GB")
        if output_path.endswith(".safetensors"):
            from safetensors.torch import save_file
            save_file({k: v.contiguous() for k, v in state_dict.items()}, output_path)
        else:
            torch.save(state_dict, output_path)
        if model_config is not None:
            with open(os.path.join(os.path.dirname(output_path), "config.json"), "w") as fh:
                json.dump(model_config, fh, indent=2)
        print(f"[export] wrote {output_path}")
    return output_path
