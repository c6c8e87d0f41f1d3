"""RocmQLoraQuantizer: the transformers HfQuantizer of rocm_qlora
(hf_integration/quantizer.py:28-94 of the reference).

The reference runs quantize_model in _process_model_before_weight_loading,
on the model skeleton, so the checkpoint's `*.weight` tensors then find no
parameter to load into and the quantized codes are those of the random
initialization.  Here a 16-bit checkpoint loads into the unchanged skeleton
(onto the GPU with device_map="cuda", where a 70B model's bf16 weights fit in
one MI355X's 288 GB), and _process_model_after_weight_loading quantizes the
loaded weights with the HIP codec kernels, one layer at a time, releasing
each 16-bit weight as its layer is replaced.

A checkpoint saved after quantization (save_pretrained of such a model: its
config carries the quantization_config, its state_dict the QuantLinear
buffers and the adapters) loads the way the reference's does: the skeleton's
target layers become empty LoRALinear(QuantLinear) modules before loading and
the saved codes, absmax, bias and adapters load into them unchanged.
"""
from __future__ import annotations

from typing import Any, List

import torch
import torch.nn as nn

from rocm_qlora.lora.lora_layer import LoRALinear
from rocm_qlora.model.quantize_model import enable_all_kernels, quantize_model, quantized_skeleton
from rocm_qlora.quantization.quant_linear import QuantLinear

try:
    from transformers.quantizers.base import HfQuantizer
except ImportError:  # transformers absent or too old
    class HfQuantizer:  # type: ignore[no-redef]
        def __init__(self, quantization_config, **kwargs):
            raise ImportError("transformers >= 4.40 required for the HF plugin. "
                              "Use quantize_model() directly instead.")


class RocmQLoraQuantizer(HfQuantizer):
    """Quantizes the target nn.Linear layers of a loaded model to NF4 / INT8
    QuantLinear with LoRA adapters (LoRALinear), on the GPU."""

    requires_calibration: bool = False
    required_packages: List[str] = ["rocm_qlora"]

    def validate_environment(self, *args: Any, **kwargs: Any) -> None:
        """transformers >= 4.40 (quantizer.py:36-49) and a GPU: the codec runs
        as HIP kernels only."""
        import transformers
        from packaging import version
        if version.parse(transformers.__version__) < version.parse("4.40.0"):
            raise ImportError(f"transformers >= 4.40.0 required for rocm-qlora plugin. "
                              f"Found {transformers.__version__}. Please upgrade.")
        if not torch.cuda.is_available():
            raise RuntimeError("rocm_qlora runs on the GPU (HIP kernels); no GPU is visible")

    def _process_model_before_weight_loading(self, model: nn.Module, **kwargs: Any) -> nn.Module:
        """A 16-bit checkpoint: nothing to change, the target layers load their
        weights as plain nn.Linear.  A checkpoint saved after quantization: the
        target layers become the empty quantized modules its state_dict fills
        (quantizer.py:56-69)."""
        if self.pre_quantized:
            cfg = self.quantization_config
            quantized_skeleton(model, bits=cfg.bits, lora_r=cfg.lora_r, lora_alpha=cfg.lora_alpha,
                               lora_dropout=cfg.lora_dropout, target_modules=cfg.target_modules,
                               block_size=cfg.block_size)
        return model

    def _process_model_after_weight_loading(self, model: nn.Module, **kwargs: Any) -> nn.Module:
        """Quantize the loaded target layers and attach LoRA adapters, or check
        that a pre-quantized checkpoint filled every quantized buffer
        (quantizer.py:56-69 plus :71-91's post-load steps)."""
        cfg = self.quantization_config
        if self.pre_quantized:
            _check_loaded(model)
            model.requires_grad_(False)
            for mod in model.modules():
                if isinstance(mod, LoRALinear):
                    mod.lora_A.requires_grad_(True)
                    mod.lora_B.requires_grad_(True)
        else:
            quantize_model(model, bits=cfg.bits, lora_r=cfg.lora_r, lora_alpha=cfg.lora_alpha,
                           lora_dropout=cfg.lora_dropout, target_modules=cfg.target_modules,
                           block_size=cfg.block_size)
        if cfg.use_triton_kernels:
            enable_all_kernels(model)  # marks the layers as running the fused HIP kernels
        trainable = sum(p.numel() for p in model.parameters() if p.requires_grad)
        total = sum(p.numel() for p in model.parameters())
        print(f"[rocm-qlora] Model ready. Trainable: {trainable:,} / Total: {total:,}")
        return model

    def is_serializable(self, safe_serialization: Any = None) -> bool:
        """True (quantizer.py:90-91): save_pretrained writes the codes, absmax
        and adapters, and from_pretrained loads them back through this
        quantizer."""
        return True

    @property
    def is_trainable(self) -> bool:
        return True


def _check_loaded(model: nn.Module) -> None:
    """Every QuantLinear of a pre-quantized load holds codes of the dtype and
    length its bits, block size and shape call for, and absmax for each block
    (a checkpoint of another bits / block_size fails here, not in a kernel)."""
    for name, mod in model.named_modules():
        if not isinstance(mod, QuantLinear):
            continue
        q, s = mod.weight_quant, mod.weight_scales
        nb = -(-mod.in_features * mod.out_features // mod.block_size)
        want_codes = nb * mod.block_size // (2 if mod.bits == 4 else 1)
        want_dtype = torch.uint8 if mod.bits == 4 else torch.int8
        if q.is_meta or s.is_meta:
            raise RuntimeError(f"rocm_qlora: the checkpoint holds no quantized weight for {name}")
        if q.dtype != want_dtype or q.numel() != want_codes or s.numel() != nb or not s.is_floating_point():
            raise RuntimeError(
                f"rocm_qlora: {name} holds {q.numel()} {q.dtype} codes and {s.numel()} scales; "
                f"{mod.bits}-bit, block {mod.block_size} of a [{mod.out_features}, {mod.in_features}] weight "
                f"needs {want_codes} {want_dtype} codes and {nb} scales")
