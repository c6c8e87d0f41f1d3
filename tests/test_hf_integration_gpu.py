"""End to end through transformers: from_pretrained with RocmQLoraConfig on
a small random Llama checkpoint written to disk (hf_integration/quantizer.py
of the reference, which calls quantize_model on the skeleton; here the
loaded weights are quantized).  The codes of every target layer equal the
oracle's quantize_int4 / quantize_int8 of the checkpoint's weight bit for
bit, the logits match the same model run with the oracle's dequantized
weights (tolerance 1e-2 of the largest logit: only summation order
differs), and only the LoRA adapters train.  A quantized model saved with
save_pretrained loads back (quantizer.py:90-91 of the reference: the
quantizer is serializable) with the same codes, absmax, adapters and
logits, bit for bit."""
import os

import pytest
import torch

transformers = pytest.importorskip("transformers")

from oracle import qlora_ref as R  # noqa: E402
from rocm_qlora import LoRALinear  # noqa: E402
from rocm_qlora.hf_integration import RocmQLoraConfig  # noqa: E402
from rocm_qlora.optim import PagedAdamW  # noqa: E402

pytestmark = pytest.mark.gpu

TARGETS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]


def _checkpoint(path):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(0)
    LlamaForCausalLM(cfg).to(torch.bfloat16).save_pretrained(path)
    from safetensors.torch import load_file
    return load_file(os.path.join(path, "model.safetensors"))


@pytest.mark.parametrize("bits", [4, 8])
def test_from_pretrained_quantizes_loaded_weights(dev, tmp_path, bits):
    from transformers import AutoModelForCausalLM
    print(f"hf from_pretrained bits={bits}", flush=True)
    sd = _checkpoint(str(tmp_path))
    qc = RocmQLoraConfig(bits=bits, lora_r=8, lora_alpha=16, lora_dropout=0.0, target_modules=TARGETS)
    model = AutoModelForCausalLM.from_pretrained(str(tmp_path), quantization_config=qc, dtype=torch.bfloat16,
                                                 device_map={"": dev.index or 0})
    ref = AutoModelForCausalLM.from_pretrained(str(tmp_path), dtype=torch.bfloat16).to(dev)
    n = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, LoRALinear):
            continue
        n += 1
        w = sd[name + ".weight"]
        q = mod.base_layer
        if bits == 4:
            codes, scales = R.quantize_int4(w, 64)
            deq = R.dequantize_int4(codes, scales, 64)[:w.numel()].reshape(w.shape)
        else:
            codes, scales = R.quantize_int8(w, 64)
            deq = R.dequantize_int8(codes, scales, 64)[:w.numel()].reshape(w.shape)
        assert torch.equal(q.weight_quant.cpu(), codes), name
        assert torch.equal(q.weight_scales.cpu(), scales), name
        ref.get_submodule(name).weight.data.copy_(deq.to(torch.bfloat16))
    assert n == 2 * len(TARGETS)
    ids = torch.randint(0, 512, (2, 16), generator=torch.Generator().manual_seed(1)).to(dev)
    with torch.no_grad():
        got = model(ids).logits.float()
        want = ref(ids).logits.float()
    assert float((got - want).abs().max()) <= 1e-2 * float(want.abs().max())
    trainable = {nm for nm, p in model.named_parameters() if p.requires_grad}
    assert trainable and all(nm.endswith(("lora_A", "lora_B")) for nm in trainable)
    assert model.config.quantization_config is not None


def test_quantized_model_trains_with_paged_adamw(dev, tmp_path):
    from transformers import AutoModelForCausalLM
    print("hf train step", flush=True)
    _checkpoint(str(tmp_path))
    qc = RocmQLoraConfig(bits=4, lora_r=8, target_modules=TARGETS, lora_dropout=0.1)
    model = AutoModelForCausalLM.from_pretrained(str(tmp_path), quantization_config=qc, dtype=torch.bfloat16,
                                                 device_map={"": dev.index or 0})
    model.train()
    opt = PagedAdamW([p for p in model.parameters() if p.requires_grad], lr=1e-3)
    ids = torch.randint(0, 512, (4, 32), generator=torch.Generator().manual_seed(2)).to(dev)
    losses = []
    for _ in range(6):
        opt.zero_grad()
        out = model(ids, labels=ids)
        out.loss.backward()
        opt.step()
        losses.append(float(out.loss.detach()))
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < losses[0]


@pytest.mark.parametrize("bits", [4, 8])
def test_save_pretrained_round_trip(dev, tmp_path, bits):
    from transformers import AutoModelForCausalLM
    print(f"hf save/load bits={bits}", flush=True)
    src, dst = tmp_path / "src", tmp_path / "dst"
    _checkpoint(str(src))
    qc = RocmQLoraConfig(bits=bits, lora_r=8, lora_alpha=16, lora_dropout=0.0, target_modules=TARGETS)
    model = AutoModelForCausalLM.from_pretrained(str(src), quantization_config=qc, dtype=torch.bfloat16,
                                                 device_map={"": dev.index or 0})
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, LoRALinear):
                mod.lora_B.copy_(0.02 * torch.randn(mod.lora_B.shape, generator=g))
    model.save_pretrained(str(dst))
    back = AutoModelForCausalLM.from_pretrained(str(dst), dtype=torch.bfloat16, device_map={"": dev.index or 0})
    assert back.hf_quantizer.pre_quantized
    n = 0
    mods = dict(back.named_modules())
    for name, mod in model.named_modules():
        if not isinstance(mod, LoRALinear):
            continue
        n += 1
        other = mods[name]
        assert isinstance(other, LoRALinear), name
        for a, b in ((mod.base_layer.weight_quant, other.base_layer.weight_quant),
                     (mod.base_layer.weight_scales, other.base_layer.weight_scales),
                     (mod.lora_A, other.lora_A), (mod.lora_B, other.lora_B)):
            assert a.dtype == b.dtype and torch.equal(a, b), name
    assert n == 2 * len(TARGETS)
    ids = torch.randint(0, 512, (2, 16), generator=torch.Generator().manual_seed(4)).to(dev)
    with torch.no_grad():
        want = model(ids).logits
        got = back(ids).logits
    assert torch.equal(got, want)
    trainable = {nm for nm, p in back.named_parameters() if p.requires_grad}
    assert trainable and all(nm.endswith(("lora_A", "lora_B")) for nm in trainable)
