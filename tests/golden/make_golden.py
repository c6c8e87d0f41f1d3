"""Writes tests/golden/golden_vectors.npz: small known-answer vectors for the
quantized-linear path, computed by the oracle's torch restatement of the
reference (oracle/qlora_ref.py) and, for every codec vector, confirmed bit
for bit by the independent C restatement (oracle/codec_ref.c) before being
written.  Inputs are seeded and stored with the outputs, so a test needs
nothing but this file.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import codec_ref as C  # noqa: E402
from oracle import qlora_ref as R  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_vectors.npz")


def bits(t):
    """Tensor -> numpy array of its raw bits (bf16/fp16 as uint16, fp8 as uint8)."""
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.float8_e4m3fnuz,):
        return t.contiguous().view(torch.uint8).numpy()
    return t.contiguous().numpy()


def main():
    g = torch.Generator().manual_seed(20261201)
    v = {}
    # NF4 codec: 128 x 256 weights (N(0, 0.02) with a few +-8 sigma outliers) per dtype
    base = torch.randn(128, 256, generator=g) * 0.02
    idx = torch.randperm(base.numel(), generator=g)[:32]
    base.view(-1)[idx] = torch.where(torch.rand(32, generator=g) < 0.5, -0.16, 0.16)
    base[3, :64] = 0.0  # an all-zero block
    for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float16)):
        w = base.to(dt)
        packed, absmax = R.quantize_int4(w, 64)
        cp, cs = C.nf4_quantize(w, 64)
        assert np.array_equal(packed.numpy(), cp) and np.array_equal(bits(absmax), bits(cs)), name
        deq = R.dequantize_int4(packed, absmax, 64)
        assert np.array_equal(deq.numpy(), C.nf4_dequantize(packed.numpy(), absmax, 64).numpy()), name
        v[f"nf4_{name}_w"] = bits(w)
        v[f"nf4_{name}_packed"] = packed.numpy()
        v[f"nf4_{name}_absmax"] = bits(absmax)
        v[f"nf4_{name}_deq_bf16"] = bits(deq.to(torch.bfloat16))
    # double quantization of the bf16 weights (fp8 c2)
    wb = base.to(torch.bfloat16)
    packed, c2, c2s, _ = R.double_quantize(wb, 64, 256)
    cc2, cc2s = C.dq_quantize(R.quantize_int4(wb, 64)[1], 256, False)
    assert np.array_equal(bits(c2), cc2) and np.array_equal(bits(c2s), bits(cc2s))
    v["dq_packed"] = packed.numpy()
    v["dq_c2"] = bits(c2)
    v["dq_c2_scales"] = bits(c2s)
    v["dq_deq_bf16"] = bits(R.double_dequantize(packed, c2, c2s, (128, 256), 64, 256, True).to(torch.bfloat16))
    # INT8 row-absmax and FP8 per-tensor quantization
    w8 = torch.randn(64, 256, generator=g) * 0.02
    q, s = R.quantize_int8(w8, per_channel=True)
    cq, cs = C.int8_quantize(w8, 64, 256, 0)
    assert np.array_equal(q.numpy().reshape(-1), cq) and np.array_equal(s.numpy(), cs.numpy())
    v["int8_w"] = w8.numpy()
    v["int8_q"] = q.numpy()
    v["int8_s"] = s.numpy()
    wf8 = w8.to(torch.bfloat16)
    codes, scale = R.fp8_quantize_tensor(wf8)
    assert np.array_equal(bits(codes).reshape(-1), C.fnuz_encode((wf8.float() / scale).to(torch.bfloat16).float().numpy().reshape(-1)))
    v["fp8_w_bf16"] = bits(wf8)
    v["fp8_codes"] = bits(codes)
    v["fp8_scale"] = np.array([float(scale)], dtype=np.float32)
    # a small NF4 LoRA linear: x bf16 [5, 256], W [96, 256], r = 8, s = 2
    w = torch.randn(96, 256, generator=g) * 0.02
    packed, absmax = R.quantize_int4(w, 64)
    a = (torch.rand(8, 256, generator=g) * 2 - 1) / 16
    b = torch.randn(96, 8, generator=g) * 0.01
    x = torch.randn(5, 256, generator=g).to(torch.bfloat16)
    y = R.nf4_lora_linear(x, packed, absmax, None, a, b, 2.0, 96, 64)
    v.update(lin_packed=packed.numpy(), lin_absmax=absmax.numpy(), lin_a=a.numpy(), lin_b=b.numpy(),
             lin_x=bits(x), lin_y=bits(y))
    np.savez_compressed(OUT, **v)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(v)} arrays")


if __name__ == "__main__":
    main()
