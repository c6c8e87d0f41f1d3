"""Known-answer vectors (tests/golden/golden_vectors.npz, written by
tests/golden/make_golden.py from the oracle and confirmed bit for bit by the
C restatement): the oracle must still reproduce them (CPU), and the HIP
codecs and linear must reproduce them on the GPU -- bit for bit for codes,
scales and dequantized weights, rtol = atol = 1e-2 for the linear output."""
import os

import numpy as np
import pytest
import torch

from oracle import qlora_ref as R

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_vectors.npz"))
DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _t(name, dtype=None):
    t = torch.from_numpy(GOLD[name].copy())
    if dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).view(dtype)
    return t


def _same(a, b):
    """Bitwise equality of two tensors of one dtype."""
    a, b = a.contiguous().view(-1), b.contiguous().view(-1)
    if a.dtype in (torch.bfloat16, torch.float16):
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


@pytest.mark.parametrize("name", ["f32", "bf16", "f16"])
def test_oracle_reproduces_nf4_vectors(name):
    w = _t(f"nf4_{name}_w", DT[name])
    packed, absmax = R.quantize_int4(w, 64)
    assert np.array_equal(packed.numpy(), GOLD[f"nf4_{name}_packed"])
    assert _same(absmax, _t(f"nf4_{name}_absmax", DT[name]))
    deq = R.dequantize_int4(packed, absmax, 64).to(torch.bfloat16)
    assert _same(deq, _t(f"nf4_{name}_deq_bf16", torch.bfloat16))


def test_oracle_reproduces_dq_int8_fp8_linear_vectors():
    wb = _t("nf4_bf16_w", torch.bfloat16)
    packed, c2, c2s, _ = R.double_quantize(wb, 64, 256)
    assert np.array_equal(c2.view(torch.uint8).numpy(), GOLD["dq_c2"])
    assert _same(c2s, _t("dq_c2_scales", torch.bfloat16))
    q, s = R.quantize_int8(_t("int8_w"), per_channel=True)
    assert np.array_equal(q.numpy(), GOLD["int8_q"]) and np.array_equal(s.numpy(), GOLD["int8_s"])
    codes, scale = R.fp8_quantize_tensor(_t("fp8_w_bf16", torch.bfloat16))
    assert np.array_equal(codes.view(torch.uint8).numpy(), GOLD["fp8_codes"])
    assert float(scale) == float(GOLD["fp8_scale"][0])
    y = R.nf4_lora_linear(_t("lin_x", torch.bfloat16), _t("lin_packed"), _t("lin_absmax"), None, _t("lin_a"),
                          _t("lin_b"), 2.0, 96, 64)
    assert _same(y, _t("lin_y", torch.bfloat16))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["f32", "bf16", "f16"])
def test_hip_nf4_codec_matches_vectors(dev, name):
    from rocm_qlora.quantization import quantize_int4
    from rocm_qlora.quantization.quant_ops import nf4_dequantize_to
    packed, absmax = quantize_int4(_t(f"nf4_{name}_w", DT[name]).to(dev), 64)
    assert np.array_equal(packed.cpu().numpy(), GOLD[f"nf4_{name}_packed"])
    assert _same(absmax.cpu(), _t(f"nf4_{name}_absmax", DT[name]))
    deq = nf4_dequantize_to(packed, absmax, 64, torch.bfloat16)
    assert _same(deq.cpu(), _t(f"nf4_{name}_deq_bf16", torch.bfloat16))


@pytest.mark.gpu
def test_hip_dq_int8_fp8_linear_match_vectors(dev):
    from rocm_qlora import ops
    from rocm_qlora.quantization import double_quantize, quantize_int8
    from rocm_qlora.quantization.double_quant import dq_dequantize_to
    st = double_quantize(_t("nf4_bf16_w", torch.bfloat16).to(dev), 64, 256)
    assert np.array_equal(st.c2.view(torch.uint8).cpu().numpy(), GOLD["dq_c2"])
    assert _same(st.c2_scales.cpu(), _t("dq_c2_scales", torch.bfloat16))
    deq = dq_dequantize_to(st.W_quant, st.c2, st.c2_scales, 64, 256, True, torch.bfloat16, 128 * 256)
    assert _same(deq.cpu(), _t("dq_deq_bf16", torch.bfloat16))
    q, s = quantize_int8(_t("int8_w").to(dev), per_channel=True)
    assert np.array_equal(q.cpu().numpy(), GOLD["int8_q"]) and np.array_equal(s.cpu().numpy(), GOLD["int8_s"])
    codes, scale = ops.fp8_quantize(_t("fp8_w_bf16", torch.bfloat16).to(dev))
    assert np.array_equal(codes.view(torch.uint8).cpu().numpy(), GOLD["fp8_codes"])
    assert float(scale) == float(GOLD["fp8_scale"][0])
    y = ops.nf4_linear(_t("lin_x", torch.bfloat16).to(dev), _t("lin_packed").to(dev), _t("lin_absmax").to(dev), 96,
                       64, lora_a=_t("lin_a").to(dev), lora_b=_t("lin_b").to(dev), scaling=2.0)
    ref = _t("lin_y", torch.bfloat16).float()
    err = (y.cpu().float() - ref).abs()
    assert bool((err <= 1e-2 + 1e-2 * ref.abs()).all())
