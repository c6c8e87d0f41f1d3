"""GPU parity of the merged-weight kernel (rq_merge_lora) behind
LoRALinear.merge_lora (lora_layer.py:72-113) and merge_and_export_fp16
(export/gguf_export.py:30-184) against the oracle's restatements.

Bit-exact wherever the reference's result does not depend on the order of
its fp32 sum over the rank: zero adapters (the merged weight is the
dequantized weight cast to fp16) and dyadic adapters (every product and rank
sum exact in fp32).  With random adapters torch's CPU matmul and the kernel
sum the rank in different orders, so the fp16 results may differ in the last
place: within one ulp."""
import math
import os

import pytest
import torch
import torch.nn as nn

from oracle import qlora_ref as R
from rocm_qlora import LoRALinear, QuantLinear, ops
from rocm_qlora.export import merge_and_export_fp16
from rocm_qlora.export.gguf_export import _export_dequant_layer

pytestmark = pytest.mark.gpu


def _dyadic(shape, g, scale_pow):
    return torch.randint(-8, 9, shape, generator=g).to(torch.float32) * 2.0 ** -scale_pow


def _layer(dev, N, K, bits, dq, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    lin = nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
    ql = QuantLinear.from_linear(lin.to(dev), bits=bits, block_size=64)
    if dq:
        assert ql.enable_double_quant()
    return ql


def _w_flat(ql):
    """The reference's fp32 dequantized flat weight (oracle)."""
    if ql.bits == 8:
        return R.dequantize_int8(ql.weight_quant.cpu(), ql.weight_scales.cpu(), 64)
    if ql.use_double_quant:
        return R.double_dequantize(ql.weight_quant.cpu(), ql.c2.cpu(), ql.c2_scales.cpu(),
                                   (ql.out_features * ql.in_features,), 64, ql.blocksize_2, ql.use_fp8_c2)
    return R.dequantize_int4(ql.weight_quant.cpu(), ql.weight_scales.cpu(), 64)


def _ulps(a, b):
    return int((a.view(torch.int16).to(torch.int32) - b.view(torch.int16).to(torch.int32)).abs().max())


@pytest.mark.parametrize("bits,dq", [(4, False), (4, True), (8, False)])
@pytest.mark.parametrize("mode", ["sum_then_round", "round_then_sum"])
def test_merge_zero_adapters_is_dequant(dev, bits, dq, mode):
    N, K = 192, 320
    ql = _layer(dev, N, K, bits, dq, seed=3)
    a = torch.randn(16, K, device=dev)
    b = torch.zeros(N, 16, device=dev)
    got = ql.merged_weight(a, b, 2.0, mode).cpu()
    want = _w_flat(ql)[:N * K].reshape(N, K).to(torch.float16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_merge_int8_per_row_scales(dev):
    N, K = 96, 256
    g = torch.Generator().manual_seed(4)
    w = torch.randn(N, K, generator=g) * 0.02
    q, s = R.quantize_int8(w, per_channel=True)
    got = ops.merge_lora(q.to(dev), s.to(dev), N, K, 0, bits=8).cpu()
    want = R.dequantize_int8(q, s).to(torch.float16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("bits,dq", [(4, False), (4, True), (8, False)])
@pytest.mark.parametrize("rank", [16, 40, 64])
def test_merge_dyadic_adapters_bit_exact(dev, bits, dq, rank):
    N, K, s = 256, 512, 0.25
    ql = _layer(dev, N, K, bits, dq, seed=rank + bits)
    g = torch.Generator().manual_seed(rank)
    a, b = _dyadic((rank, K), g, 6), _dyadic((N, rank), g, 7)
    w = _w_flat(ql)
    m = ql.merged_weight(a.to(dev), b.to(dev), s, "sum_then_round").cpu()
    assert torch.equal(m.view(torch.int16), R.merge_lora_weight(w, a, b, s, N, K).view(torch.int16))
    e = ql.merged_weight(a.to(dev), b.to(dev), s, "round_then_sum").cpu()
    assert torch.equal(e.view(torch.int16), R.export_dequant_layer(w, a, b, s, N, K).view(torch.int16))


def test_merge_bf16_adapters_and_bf16_output(dev):
    """bf16 adapters: B @ A and its scaling rounded to bf16 as torch does for
    bf16 parameters; a bf16 merged weight."""
    N, K, rank, s = 128, 256, 16, 2.0
    ql = _layer(dev, N, K, 4, False, seed=11)
    g = torch.Generator().manual_seed(12)
    a, b = _dyadic((rank, K), g, 6).to(torch.bfloat16), _dyadic((N, rank), g, 7).to(torch.bfloat16)
    w = _w_flat(ql)[:N * K].reshape(N, K)
    d = ((b @ a) * s).to(torch.float32)
    got = ql.merged_weight(a.to(dev), b.to(dev), s, "sum_then_round", torch.bfloat16).cpu()
    want = (w + d).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("dq", [False, True])
def test_merge_random_adapters_within_one_ulp(dev, dq):
    N, K, rank = 4096, 4096, 16
    ql = _layer(dev, N, K, 4, dq, seed=21)
    g = torch.Generator().manual_seed(22)
    a = torch.empty(rank, K)
    nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
    b = torch.randn(N, rank, generator=g) * 0.01
    w = _w_flat(ql)
    m = ql.merged_weight(a.to(dev), b.to(dev), 2.0, "sum_then_round").cpu()
    assert _ulps(m, R.merge_lora_weight(w, a, b, 2.0, N, K)) <= 1
    e = ql.merged_weight(a.to(dev), b.to(dev), 2.0, "round_then_sum").cpu()
    assert _ulps(e, R.export_dequant_layer(w, a, b, 2.0, N, K)) <= 1


def test_lora_linear_merge_uses_kernel_and_unmerges(dev):
    N, K = 256, 256
    ql = _layer(dev, N, K, 4, False, seed=31)
    lora = LoRALinear(ql, r=8, lora_alpha=16)
    g = torch.Generator().manual_seed(32)
    with torch.no_grad():
        lora.lora_A.copy_(_dyadic((8, K), g, 6))
        lora.lora_B.copy_(_dyadic((N, 8), g, 7))
    x = torch.randn(3, K, device=dev, dtype=torch.bfloat16)
    pre = lora(x)
    lora.merge_lora()
    want = R.merge_lora_weight(_w_flat(ql), lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu(), lora.scaling,
                               N, K)
    assert torch.equal(ql.merged_fp16_weight.cpu().view(torch.int16), want.view(torch.int16))
    post = lora(x)
    assert (post.float() - pre.float()).abs().max() < 0.05
    lora.unmerge_lora()
    assert torch.equal(lora(x), pre)


def test_merge_and_export_fp16_file(dev, tmp_path):
    """merge_and_export_fp16 writes every non-adapter parameter as fp16 and
    each LoRALinear's weight as _export_dequant_layer builds it, under the
    layer's own keys; config.json beside it."""
    from safetensors.torch import load_file
    torch.manual_seed(41)
    model = nn.Sequential(nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 64)).to(dev)
    layers = []
    for i in (0, 2):
        ql = QuantLinear.from_linear(model[i], bits=4, block_size=64)
        lora = LoRALinear(ql, r=8, lora_alpha=16)
        with torch.no_grad():
            lora.lora_B.normal_(0, 0.01)
        model[i] = lora
        layers.append(lora)
    model.add_module("norm", nn.LayerNorm(64).to(dev))
    out = str(tmp_path / "merged.safetensors")
    assert merge_and_export_fp16(model, out, {"model_type": "test"}) == out
    sd = load_file(out)
    assert os.path.exists(tmp_path / "config.json")
    assert set(sd) == {"0.weight", "0.bias", "2.weight", "2.bias", "norm.weight", "norm.bias"}
    for i, lora in zip((0, 2), layers):
        ql = lora.base_layer
        want = R.export_dequant_layer(_w_flat(ql), lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu(),
                                      lora.scaling, ql.out_features, ql.in_features)
        assert _ulps(sd[f"{i}.weight"], want) <= 1
        assert torch.equal(sd[f"{i}.weight"], _export_dequant_layer(lora).cpu())
        assert torch.equal(sd[f"{i}.bias"], ql.bias.cpu().to(torch.float16))
        assert sd[f"{i}.weight"].dtype == torch.float16
    assert torch.equal(sd["norm.weight"], model.norm.weight.detach().cpu().to(torch.float16))
