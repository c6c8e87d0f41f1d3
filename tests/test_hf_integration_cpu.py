"""The transformers integration's host logic (hf_integration/config.py and
quantizer.py of the reference): config fields, defaults and dict round trip,
registration under "rocm_qlora", the quantizer's flags and its refusals,
and the skeleton a checkpoint saved after quantization loads into."""
import json
import os

import torch
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
    assert q.is_trainable and q.is_serializable() and not q.requires_calibration


def test_quantizer_needs_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    for pre in (False, True):
        q = RocmQLoraQuantizer(RocmQLoraConfig(bits=4), pre_quantized=pre)
        with pytest.raises(RuntimeError):
            q.validate_environment()


TARGETS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]


def _tiny_llama_config():
    from transformers import LlamaConfig
    return LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=192, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)


@pytest.mark.parametrize("bits,block", [(4, 64), (8, 64), (4, 32), (8, 48)])
def test_skeleton_matches_quantized_layout(bits, block):
    """quantized_skeleton builds, on the meta device, the keys, shapes and
    dtypes the oracle's quantization of each target layer gives
    (quant_ops.py:17-126: padded flat codes, squeezed absmax in the weight's
    dtype), the bias in the weight's dtype and fp32 adapters."""
    from transformers import LlamaForCausalLM
    from oracle import qlora_ref as R
    from rocm_qlora import LoRALinear
    from rocm_qlora.model.quantize_model import quantized_skeleton
    with torch.device("meta"):
        model = LlamaForCausalLM(_tiny_llama_config()).to(torch.bfloat16)
        quantized_skeleton(model, bits=bits, lora_r=8, lora_alpha=16, lora_dropout=0.0,
                           target_modules=TARGETS, block_size=block)
    n = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, LoRALinear):
            continue
        n += 1
        q = mod.base_layer
        w = torch.randn(q.out_features, q.in_features).to(torch.bfloat16)
        codes, scales = (R.quantize_int4 if bits == 4 else R.quantize_int8)(w, block)
        assert q.weight_quant.is_meta and q.weight_quant.shape == codes.shape, name
        assert q.weight_quant.dtype == codes.dtype and q.weight_scales.dtype == scales.dtype, name
        assert q.weight_scales.shape == scales.shape, name
        assert q.bias is None and (q.bits, q.block_size) == (bits, block)
        assert mod.lora_A.shape == (8, q.in_features) and mod.lora_B.shape == (q.out_features, 8)
        assert mod.lora_A.dtype == mod.lora_B.dtype == torch.float32
    assert n == 2 * len(TARGETS)
    assert not any(p.requires_grad for nm, p in model.named_parameters() if "lora_" not in nm)


def _write_prequantized(path, bits, block, seed=0):
    """A checkpoint as save_pretrained writes one for a quantized model: the
    config with its quantization_config, and a state_dict whose target layers
    hold the oracle's codes and absmax of a random weight plus random
    adapters (the 16-bit `*.weight` of those layers is absent)."""
    from safetensors.torch import save_file
    from transformers import LlamaForCausalLM
    from oracle import qlora_ref as R
    cfg = _tiny_llama_config()
    torch.manual_seed(seed)
    model = LlamaForCausalLM(cfg).to(torch.bfloat16)
    sd = {}
    g = torch.Generator().manual_seed(seed + 1)
    for name, t in model.state_dict().items():
        layer = name.rsplit(".", 1)[0]
        if name.endswith(".weight") and any(layer.endswith(x) for x in TARGETS):
            codes, scales = (R.quantize_int4 if bits == 4 else R.quantize_int8)(t, block)
            sd[layer + ".base_layer.weight_quant"] = codes
            sd[layer + ".base_layer.weight_scales"] = scales
            sd[layer + ".base_layer.weight_zeros"] = torch.zeros(1)
            sd[layer + ".lora_A"] = torch.randn(8, t.shape[1], generator=g)
            sd[layer + ".lora_B"] = torch.randn(t.shape[0], 8, generator=g)
        else:
            sd[name] = t.contiguous()
    if cfg.tie_word_embeddings:
        sd.pop("lm_head.weight", None)
    os.makedirs(path, exist_ok=True)
    save_file(sd, os.path.join(path, "model.safetensors"), metadata={"format": "pt"})
    d = cfg.to_dict()
    d["architectures"] = ["LlamaForCausalLM"]
    d["dtype"] = "bfloat16"
    d["quantization_config"] = RocmQLoraConfig(bits=bits, lora_r=8, lora_alpha=16, lora_dropout=0.0,
                                               target_modules=TARGETS, block_size=block).to_dict()
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(d, f)
    return sd


@pytest.mark.parametrize("bits,block", [(4, 64), (8, 32)])
def test_prequantized_checkpoint_loads_through_transformers(tmp_path, monkeypatch, bits, block):
    """from_pretrained of a checkpoint saved after quantization, with no
    quantization_config argument: transformers picks the quantizer from the
    config, the skeleton takes the saved buffers and adapters key for key and
    bit for bit, nothing is reported missing or unexpected, and only the
    adapters train.  Loading runs no kernel, so the quantizer's GPU check is
    the only thing stood in for here (the GPU test runs the loaded model)."""
    from transformers import AutoModelForCausalLM
    from rocm_qlora import LoRALinear
    import rocm_qlora.hf_integration.quantizer as qz
    monkeypatch.setattr(qz.torch.cuda, "is_available", lambda: True)
    sd = _write_prequantized(str(tmp_path), bits, block)
    model, info = AutoModelForCausalLM.from_pretrained(str(tmp_path), dtype=torch.bfloat16,
                                                       output_loading_info=True)
    assert not info["missing_keys"] and not info["unexpected_keys"] and not info["mismatched_keys"], info
    assert isinstance(model.hf_quantizer, RocmQLoraQuantizer) and model.hf_quantizer.pre_quantized
    n = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, LoRALinear):
            continue
        n += 1
        q = mod.base_layer
        assert torch.equal(q.weight_quant, sd[name + ".base_layer.weight_quant"]), name
        assert q.weight_scales.dtype == torch.bfloat16
        assert torch.equal(q.weight_scales, sd[name + ".base_layer.weight_scales"]), name
        assert mod.lora_A.dtype == torch.float32 and torch.equal(mod.lora_A, sd[name + ".lora_A"]), name
        assert torch.equal(mod.lora_B, sd[name + ".lora_B"]), name
    assert n == 2 * len(TARGETS)
    trainable = {nm for nm, p in model.named_parameters() if p.requires_grad}
    assert trainable and all(nm.endswith(("lora_A", "lora_B")) for nm in trainable)
    emb = model.get_input_embeddings().weight
    assert torch.equal(emb, sd["model.embed_tokens.weight"])


def test_prequantized_checkpoint_of_other_block_size_is_refused(tmp_path, monkeypatch):
    """Codes saved with block 64 under a config that says block 32 hold half
    the absmax the layers need: the load fails naming the layer."""
    from transformers import AutoModelForCausalLM
    import rocm_qlora.hf_integration.quantizer as qz
    monkeypatch.setattr(qz.torch.cuda, "is_available", lambda: True)
    _write_prequantized(str(tmp_path), 4, 64)
    cfgp = os.path.join(str(tmp_path), "config.json")
    with open(cfgp) as f:
        d = json.load(f)
    d["quantization_config"]["block_size"] = 32
    with open(cfgp, "w") as f:
        json.dump(d, f)
    with pytest.raises(RuntimeError, match="scales"):
        AutoModelForCausalLM.from_pretrained(str(tmp_path), dtype=torch.bfloat16)
