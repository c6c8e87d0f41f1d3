"""RocmQLoraQuantizer: the transformers HfQuantizer of rocm_qlora
(hf_integration/quantizer.py:28-94 of the reference).

The reference runs quantize_model in _process_model_before_weight_loading,
on the model skeleton, so the checkpoint's `*.weight` tensors then find no
parameter to load into and the quantized codes are those of the random
initialization.  Here the skeleton is left alone, transformers loads the
16-bit weights (onto the GPU with device_map="cuda", where a 70B model's
bf16 weights fit in one MI355X's 288 GB), and _process_model_after_weight_loading
quantizes the loaded weights with the HIP codec kernels, one layer at a
time, releasing each 16-bit weight as its layer is replaced.  Checkpoints
saved after quantization (QuantLinear buffers) are not loaded through this
path: load the original weights, or export merged fp16 weights with
rocm_qlora.export.merge_and_export_fp16.
"""
from __future__ import annotations

from typing import Any, List

import torch
import torch.nn as nn

from rocm_qlora.model.quantize_model import enable_all_kernels, quantize_model

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
            raise RuntimeError("rocm_qlora quantizes on the GPU (HIP kernels); no GPU is visible")
        if self.pre_quantized:
            raise ValueError("rocm_qlora: this checkpoint was saved after quantization; load the original "
                             "16-bit weights with RocmQLoraConfig instead")

    def _process_model_before_weight_loading(self, model: nn.Module, **kwargs: Any) -> nn.Module:
        """Nothing to change before loading: the target layers load their
        16-bit weights as plain nn.Linear."""
        return model

    def _process_model_after_weight_loading(self, model: nn.Module, **kwargs: Any) -> nn.Module:
        """Quantize the loaded target layers and attach LoRA adapters
        (quantizer.py:56-69 plus :71-91's post-load steps)."""
        cfg = self.quantization_config
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
        """False: a quantized checkpoint would not load back through this
        quantizer (the reference answers True, quantizer.py:90-91); save the
        adapters' state_dict, or merged fp16 weights."""
        return False

    @property
    def is_trainable(self) -> bool:
        return True
