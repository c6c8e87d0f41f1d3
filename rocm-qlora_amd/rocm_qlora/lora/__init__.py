"""LoRA adapter layer (lora/__init__.py of the reference)."""
from rocm_qlora.lora.lora_layer import LoRALinear

__all__ = ["LoRALinear"]
