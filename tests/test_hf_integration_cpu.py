"""The transformers integration's host logic (hf_integration/config.py and
quantizer.py of the reference): config fields, defaults and dict round trip,
registration under "rocm_qlora", the quantizer's flags and its refusals."""
import pytest

transformers = pytest.importorskip("transformers")

from rocm_qlora.hf_integration import RocmQLoraConfig, RocmQLoraQuantizer, register_with_transformers  # noqa: E402


def test_config_defaults_and_round_trip():
    c = RocmQLoraConfig()
    assert (c.bits, c.lora_r, c.lora_alpha, c.lora_dropout, c.block_size) == (8, 8, 16, 0.05, 64)
    assert c.target_modules == ["q_proj", "v_proj", "k_proj", "o_proj"]
    d = RocmQLoraConfig(bits=4, lora_r=16, target_modules=["gate_proj"]).to_dict()
    assert d["quant_method"] == "rocm_qlora" and d["bits"] == 4 and d["target_modules"] == ["gate_proj"]
    assert RocmQLoraConfig.from_dict(d).to_dict() == d
    assert "RocmQLoraConfig(bits=4" in repr(RocmQLoraConfig.from_dict(d))
    with pytest.raises(ValueError):
        RocmQLoraConfig(bits=3)


def test_registered_with_transformers():
    from transformers.quantizers import auto
    assert register_with_transformers()
    assert auto.AUTO_QUANTIZER_MAPPING["rocm_qlora"] is RocmQLoraQuantizer
    cfg = auto.AutoQuantizationConfig.from_dict(RocmQLoraConfig(bits=4).to_dict())
    assert isinstance(cfg, RocmQLoraConfig) and cfg.bits == 4
    q = auto.AutoHfQuantizer.from_config(cfg, pre_quantized=False)
    assert isinstance(q, RocmQLoraQuantizer)
    assert q.is_trainable and not q.is_serializable() and not q.requires_calibration


def test_quantizer_needs_a_gpu_and_original_weights():
    import torch
    q = RocmQLoraQuantizer(RocmQLoraConfig(bits=4), pre_quantized=False)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError):
            q.validate_environment()
    pq = RocmQLoraQuantizer(RocmQLoraConfig(bits=4), pre_quantized=True)
    with pytest.raises((RuntimeError, ValueError)):
        pq.validate_environment()
