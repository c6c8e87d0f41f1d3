"""transformers integration (hf_integration/__init__.py of the reference):

    from rocm_qlora.hf_integration import RocmQLoraConfig
    model = AutoModelForCausalLM.from_pretrained(
        path, quantization_config=RocmQLoraConfig(bits=4, lora_r=8), device_map="cuda")

Importing this module registers the config and the quantizer under the
quantization method "rocm_qlora" in transformers' quantizer registry (when
transformers provides the registration functions)."""
from rocm_qlora.hf_integration.config import RocmQLoraConfig
from rocm_qlora.hf_integration.quantizer import RocmQLoraQuantizer

__all__ = ["RocmQLoraConfig", "RocmQLoraQuantizer", "register_with_transformers"]


def register_with_transformers() -> bool:
    """Add "rocm_qlora" to transformers' quantizer registry (idempotent).
    False when transformers or its registration functions are absent."""
    try:
        from transformers.quantizers import auto
    except ImportError:
        return False
    if not hasattr(auto, "AUTO_QUANTIZER_MAPPING"):
        return False
    auto.AUTO_QUANTIZATION_CONFIG_MAPPING["rocm_qlora"] = RocmQLoraConfig
    auto.AUTO_QUANTIZER_MAPPING["rocm_qlora"] = RocmQLoraQuantizer
    return True


register_with_transformers()
