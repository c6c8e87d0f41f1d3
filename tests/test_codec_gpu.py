"""GPU parity of the codecs: HIP kernels vs the oracle, bit-exact (NaN
positions compared as positions).  Reference behaviours from
tests/test_quant_ops.py and tests/v4/test_double_quant.py are re-pinned here."""
import numpy as np
import pytest
import torch

from oracle import codec_ref as C
from oracle import qlora_ref as R
from rocm_qlora.quantization import (dequantize_int4, dequantize_int8, double_dequantize,
                                     double_quantize, quantize_int4, quantize_int8)
from rocm_qlora.quantization.quant_ops import nf4_dequantize_to

pytestmark = pytest.mark.gpu
from tests.test_oracle_codec import _edge_weights, _weights  # noqa: E402


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.cpu(), b.cpu()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype.is_floating_point:
        nan = torch.isnan(a) & torch.isnan(b)
        iv = {4: torch.int32, 2: torch.int16}[a.element_size()]
        return bool(((a.view(iv) == b.view(iv)) | nan).all())
    return torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block", [32, 64, 128, 96, 6])
def test_quantize_int4_bit_exact(dev, dtype, block):
    cases = [_weights((37, 300), dtype, 3), _edge_weights(dtype, block),
             _weights((64, 1024), dtype, 4)[:, 1:]]  # non-contiguous view, ragged
    for w in cases:
        print(f"quantize_int4 dtype={dtype} block={block} shape={tuple(w.shape)}", flush=True)
        p_ref, s_ref = R.quantize_int4(w.contiguous(), block)
        p, s = quantize_int4(w.to(dev), block)
        assert bits_equal(p, p_ref)
        assert bits_equal(s, s_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("block", [32, 64, 256])
def test_quantize_int4_large_with_edge_blocks(dev, dtype, block):
    """Sizes where whole workgroups take the straight 16-byte path and the
    last one the per-group tail: zero, constant, NaN, Inf and tiny blocks first,
    then N(0, 0.02) weights with outliers, 301 x 4096 + the edge blocks."""
    edge = _edge_weights(dtype, block).reshape(-1)
    w = torch.cat([edge, _weights((301, 4096), dtype, 21).reshape(-1)])
    print(f"quantize_int4 large dtype={dtype} block={block} numel={w.numel()}", flush=True)
    p_ref, s_ref = R.quantize_int4(w, block)
    p, s = quantize_int4(w.to(dev), block)
    assert bits_equal(p, p_ref)
    assert bits_equal(s, s_ref)


def test_quantize_int4_unaligned_view(dev):
    w = _weights((4096 + 3,), torch.bfloat16, 9)
    view = w.to(dev)[3:]  # 6-byte offset: generic (non-vector) loads
    p, s = quantize_int4(view, 64)
    p_ref, s_ref = R.quantize_int4(w[3:].contiguous(), 64)
    assert bits_equal(p, p_ref) and bits_equal(s, s_ref)


def test_quantize_int4_cpu_tensor_runs_on_gpu_and_returns_cpu():
    w = _weights((128, 64), torch.float32, 1)
    p, s = quantize_int4(w, 64)
    assert p.device.type == "cpu" and s.device.type == "cpu"
    p_ref, s_ref = R.quantize_int4(w, 64)
    assert bits_equal(p, p_ref) and bits_equal(s, s_ref)


@pytest.mark.parametrize("sdtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block", [64, 32, 128, 6])
def test_dequantize_int4_bit_exact(dev, sdtype, block):
    w = _weights((33, 192), sdtype, 6)
    p_ref, s_ref = R.quantize_int4(w, block)
    ref = R.dequantize_int4(p_ref, s_ref, block)
    got = dequantize_int4(p_ref.to(dev), s_ref.to(dev), block)
    assert bits_equal(got, ref)
    n = 33 * 192 - 5
    for od in (torch.bfloat16, torch.float16, torch.float32):
        print(f"dequant block={block} sdtype={sdtype} out={od}", flush=True)
        got = nf4_dequantize_to(p_ref.to(dev), s_ref.to(dev), block, od, n)
        assert bits_equal(got, ref[:n].to(od))


@pytest.mark.parametrize("sdtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("od", [torch.bfloat16, torch.float16, torch.float32])
def test_dequantize_int4_large_and_offset_codes(dev, sdtype, od):
    """Whole workgroups of 16-byte code loads and a ragged last one (300 x
    4096 - 40 weights), and the same codes through an 8-byte (not 16-byte)
    aligned view, which takes the 8-byte path everywhere."""
    w = _weights((300, 4096), sdtype, 22)
    p_ref, s_ref = R.quantize_int4(w, 64)
    ref = R.dequantize_int4(p_ref, s_ref, 64)
    n = w.numel() - 40
    print(f"dequant large sdtype={sdtype} out={od}", flush=True)
    got = nf4_dequantize_to(p_ref.to(dev), s_ref.to(dev), 64, od, n)
    assert bits_equal(got, ref[:n].to(od))
    # codes from byte 8 on (weights 16 ..): an 8-byte aligned view
    pad = torch.zeros(8, dtype=torch.uint8)
    buf = torch.cat([pad, p_ref]).to(dev)
    view = buf[8:]
    assert view.data_ptr() % 16 == 8
    s_view = s_ref.to(dev)
    got = nf4_dequantize_to(view, s_view, 64, od, n)
    assert bits_equal(got, ref[:n].to(od))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("use_fp8", [True, False])
def test_double_quant_bit_exact(dev, dtype, use_fp8, monkeypatch):
    import rocm_qlora.quantization.double_quant as dqm
    monkeypatch.setattr(dqm, "_has_fp8", lambda: use_fp8)
    w = _weights((96, 700), dtype, 11)  # 67200 weights: c1 padded inside the last 256-block
    st = double_quantize(w.to(dev), 64, 256)
    p_ref, c2_ref, c2s_ref, _ = R.double_quantize(w, 64, 256, use_fp8=use_fp8)
    assert st.use_fp8_c2 == use_fp8
    assert bits_equal(st.W_quant, p_ref)
    assert st.c2.dtype == (torch.float8_e4m3fnuz if use_fp8 else torch.int8)
    assert bits_equal(st.c2.view(torch.uint8), c2_ref.view(torch.uint8))
    assert bits_equal(st.c2_scales, c2s_ref)
    rec = double_dequantize(st)
    ref = R.double_dequantize(p_ref, c2_ref, c2s_ref, w.shape, 64, 256, use_fp8)
    assert rec.shape == w.shape
    assert bits_equal(rec, ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_int8_bit_exact(dev, dtype):
    w = _weights((48, 200), dtype, 13)
    q, s = quantize_int8(w.to(dev).flatten(), 64)
    q_ref, s_ref = R.quantize_int8(w.flatten(), 64)
    assert bits_equal(q, q_ref) and bits_equal(s, s_ref)
    assert bits_equal(dequantize_int8(q, s, 64), R.dequantize_int8(q_ref, s_ref, 64))
    q, s = quantize_int8(w.to(dev), per_channel=True)
    q_ref, s_ref = R.quantize_int8(w, per_channel=True)
    assert bits_equal(q, q_ref) and bits_equal(s, s_ref)
    assert bits_equal(dequantize_int8(q, s), R.dequantize_int8(q_ref, s_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cols", [8192, 11008, 512])
def test_int8_per_channel_large_bit_exact(dev, dtype, cols):
    """Rows of 512 .. 11008 elements (one workgroup per row; rows past 8192
    elements load their tail twice), edge rows first: zeros, a NaN, an Inf,
    tiny values; then the fp32 reconstruction of the same codes."""
    w = _weights((70, cols), dtype, 31)
    w[0] = 0
    w[1, 7] = float("nan")
    w[2, 3] = float("inf")
    w[3] = (w[3].float() * 1e-30).to(dtype)
    print(f"int8 per-channel dtype={dtype} cols={cols}", flush=True)
    q, s = quantize_int8(w.to(dev), per_channel=True)
    q_ref, s_ref = R.quantize_int8(w, per_channel=True)
    assert bits_equal(q, q_ref) and bits_equal(s, s_ref)
    assert bits_equal(dequantize_int8(q, s), R.dequantize_int8(q_ref, s_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block,cols", [(64, 1024), (32, 1032), (512, 1024), (8, 1032), (64, 1032)])
def test_int8_blockwise_large_bit_exact(dev, dtype, block, cols):
    """Blockwise scales over a flat tensor (300 x cols): whole blocks on the
    vector kernels (several workgroups of 1024 groups, a partly filled last
    one), a partial last block (64 x 1032 elements) on the generic kernel;
    dequantized to fp32."""
    w = _weights((300, cols), dtype, 32).flatten()
    w[5] = float("nan")
    print(f"int8 blockwise dtype={dtype} block={block}", flush=True)
    q, s = quantize_int8(w.to(dev), block)
    q_ref, s_ref = R.quantize_int8(w, block)
    assert bits_equal(q, q_ref) and bits_equal(s, s_ref)
    assert bits_equal(dequantize_int8(q, s, block), R.dequantize_int8(q_ref, s_ref, block))


def _config2_weight():
    """11008x4096 (down-proj) bf16 ~ N(0, 0.02), 0.1% outliers at +-8 sigma."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(4096, 11008, generator=g) * 0.02
    flat = w.view(-1)
    k = flat.numel() // 1000
    pos = torch.randperm(flat.numel(), generator=g)[:k]
    flat[pos] = 0.16 * (torch.randint(0, 2, (k,), generator=g).float() * 2 - 1)
    return w.to(torch.bfloat16)


def test_config2_full_size_bit_exact(dev):
    """quantize -> pack -> double-quant -> dequantize at 11008x4096, checked
    against the C oracle (every packed nibble, absmax, c2, c2_scales and
    dequantized bf16 value)."""
    w = _config2_weight()
    print("config2: GPU double_quantize", flush=True)
    st = double_quantize(w.to(dev), 64, 256)
    print("config2: C oracle", flush=True)
    p_c, s_c = C.nf4_quantize(w, 64)
    assert np.array_equal(st.W_quant.cpu().numpy(), p_c)
    c2_c, c2s_c = C.dq_quantize(s_c, 256)
    assert np.array_equal(st.c2.view(torch.uint8).cpu().numpy(), c2_c)
    assert bits_equal(st.c2_scales, c2s_c)
    from rocm_qlora.quantization.double_quant import dq_dequantize_to
    got = dq_dequantize_to(st.W_quant, st.c2, st.c2_scales, 64, 256, True, torch.bfloat16, w.numel())
    ref = C.dq_dequantize(p_c, c2_c, c2s_c, 64, 256, out_dtype="bf16", n_out=w.numel())
    assert bits_equal(got, ref)
    # size-independent property: re-quantizing the single-quant dequantized
    # weights reproduces every code (quant_ops.py:104-115 with n = T_j exactly)
    _, s_gpu = quantize_int4(w.to(dev), 64)
    deq = nf4_dequantize_to(st.W_quant, s_gpu, 64, torch.float32, w.numel())
    p2, s2 = quantize_int4(deq, 64)
    assert torch.equal(p2, st.W_quant)
    assert torch.equal(s2, s_gpu.float())


def test_reference_roundtrip_behaviours(dev):
    """tests/test_quant_ops.py:13-63 and tests/v4/test_double_quant.py:43-66."""
    torch.manual_seed(42)
    t = (torch.randn(1024) * 2.0).to(dev)
    t[0] = 100.0
    q, s = quantize_int8(t, 64)
    assert q.dtype == torch.int8
    assert (t - dequantize_int8(q, s, 64)[:1024]).abs().max() < 0.01 * t.abs().max()
    t = torch.randn(1024, device=dev)
    p, s = quantize_int4(t, 64)
    assert p.dtype == torch.uint8 and p.numel() * 2 >= t.numel()
    assert (t - dequantize_int4(p, s, 64)[:1024]).abs().max() < 0.15 * t.abs().max()
    W = torch.randn(256, 256, device=dev)
    q, s = quantize_int4(W, 64)
    single = dequantize_int4(q, s, 64)[:W.numel()].reshape(W.shape)
    double = double_dequantize(double_quantize(W, 64, 256))
    assert (double - single).abs().mean() < 0.1
