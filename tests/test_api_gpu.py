"""GPU checks of the reference's Python API on the HIP path: QuantLinear,
LoRALinear (forward, autograd, merge), double quantization on a layer,
quantize_model on a small transformer, the kernels / hip_kernels / fp8
entry points.  Every value is compared with the oracle's restatement of the
reference CPU path on the same inputs: quantized buffers bit-exact; outputs
and gradients within rtol = atol = 1e-2 (bf16 / fp16; for gradients atol is
taken relative to the largest reference magnitude) and 1e-3 for fp32
activations."""
import math

import pytest
import torch
import torch.nn as nn

import rocm_qlora
from oracle import qlora_ref as R
from rocm_qlora import QuantLinear, LoRALinear, quantize_model

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2
FP32_TOL = 1e-3


def _check(got, ref, tol=RTOL):
    got = got.detach().cpu().float()
    ref = ref.detach().float()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = (got - ref).abs()
    bad = err > tol + tol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


def _check_grad(got, ref, tol=RTOL):
    """|got - ref| <= tol * max|ref| + tol * |ref|."""
    got = got.detach().cpu().float()
    ref = ref.detach().float()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    scale = float(ref.abs().max())
    err = (got - ref).abs()
    bad = err > tol * scale + tol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g} " \
                          f"(scale {scale:.4g})"


def _linear(K, N, seed, bias=True):
    torch.manual_seed(seed)
    lin = nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.normal_(0.0, 0.02)
        if bias:
            lin.bias.normal_(0.0, 0.1)
    return lin


def _oracle_weight(ql):
    """fp32 flat dequantized weight of a QuantLinear by the oracle."""
    q, s = ql.weight_quant.cpu(), ql.weight_scales.cpu()
    if ql.bits == 8:
        return R.dequantize_int8(q, s, ql.block_size)
    return R.dequantize_int4(q, s, ql.block_size)


@pytest.mark.parametrize("bits", [8, 4])
def test_from_linear_buffers_bit_exact(dev, bits):
    lin = _linear(512, 384, seed=1)
    w = lin.weight.detach().clone()
    b = lin.bias.detach().clone()
    ql = QuantLinear.from_linear(lin.to(dev), bits=bits)
    ref = R.quantize_int8(w.flatten(), 64) if bits == 8 else R.quantize_int4(w.flatten(), 64)
    assert torch.equal(ql.weight_quant.cpu(), ref[0])
    assert torch.equal(ql.weight_scales.cpu(), ref[1])
    assert torch.equal(ql.bias.cpu(), b)
    assert not hasattr(lin, "weight") and not hasattr(lin, "bias")
    assert ql.weight_quant.numel() == (512 * 384 if bits == 8 else 512 * 384 // 2)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [1, 5, 300])
def test_quant_linear_forward_vs_oracle(dev, bits, dtype, M):
    """quant_linear.py:121-197: dequantize -> .to(x.dtype) -> F.linear(x, W, bias)."""
    K, N = 512, 384
    ql = QuantLinear.from_linear(_linear(K, N, seed=2).to(dev), bits=bits)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).to(dtype)
    y = ql(x.to(dev))
    assert y.dtype == dtype and y.shape == (M, N)
    ref = R.quant_linear_forward(x, _oracle_weight(ql), ql.bias.cpu(), N, K)
    _check(y, ref, FP32_TOL if dtype == torch.float32 else RTOL)


@pytest.mark.parametrize("bits", [8, 4])
def test_shape_restoration_and_leading_dims(dev, bits):
    """Sizes that are not multiples of the block (37 x 73) and 3-D inputs
    (test_quant_linear.py:94-104 of the reference)."""
    ql = QuantLinear.from_linear(_linear(37, 73, seed=3).to(dev), bits=bits)
    x = torch.randn(1, 37)
    y = ql(x.to(dev))
    assert y.shape == (1, 73)
    _check(y, R.quant_linear_forward(x, _oracle_weight(ql), ql.bias.cpu(), 73, 37), FP32_TOL)
    ql2 = QuantLinear.from_linear(_linear(256, 128, seed=4).to(dev), bits=bits)
    x3 = torch.randn(2, 7, 256).to(torch.bfloat16)
    y3 = ql2(x3.to(dev))
    assert y3.shape == (2, 7, 128)
    _check(y3, R.quant_linear_forward(x3, _oracle_weight(ql2), ql2.bias.cpu(), 128, 256))


@pytest.mark.parametrize("bits,atol", [(8, 0.15), (4, 0.3)])
def test_forward_close_to_full_precision(dev, bits, atol):
    """test_quant_linear.py:50-76 of the reference: quantized vs nn.Linear."""
    torch.manual_seed(42)
    lin = nn.Linear(64, 128).to(dev)
    x = torch.randn(4, 64, device=dev)
    with torch.no_grad():
        expected = lin(x)
        ql = QuantLinear.from_linear(lin, bits=bits)
        actual = ql(x)
    assert torch.allclose(actual, expected, atol=atol)


@pytest.mark.parametrize("M", [1, 300])
def test_lora_zero_init_exact(dev, M):
    ql = QuantLinear.from_linear(_linear(512, 384, seed=5).to(dev), bits=4)
    lora = LoRALinear(ql, r=16, lora_alpha=32)
    x = torch.randn(M, 512).to(dev, torch.bfloat16)
    assert torch.equal(lora(x), ql(x))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [4, 300])
@pytest.mark.parametrize("bias", [True, False])
def test_lora_forward_and_grads_vs_oracle(dev, dtype, M, bias):
    """LoRALinear(QuantLinear(bits=4)) forward and backward (dX, dA, dB) vs
    torch autograd through the reference's CPU expression
    (quant_linear.py:189-197, lora_layer.py:67-70)."""
    K, N, r = 512, 384, 16
    ql = QuantLinear.from_linear(_linear(K, N, seed=6, bias=bias).to(dev), bits=4)
    lora = LoRALinear(ql, r=r, lora_alpha=32)
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        lora.lora_B.copy_(torch.randn(N, r, generator=g) * 0.01)
    x = torch.randn(M, K, generator=g).to(dtype)
    dy = (torch.randn(M, N, generator=g) * 0.1).to(dtype)
    xd = x.to(dev).requires_grad_(True)
    y = lora(xd)
    y.backward(dy.to(dev))
    ry, rdx, rda, rdb = R.lora_linear_grads(x, _oracle_weight(ql), ql.bias.cpu() if bias else None,
                                            lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu(),
                                            lora.scaling, dy)
    tol = FP32_TOL if dtype == torch.float32 else RTOL
    _check(y, ry, tol)
    _check(xd.grad, rdx, tol)
    _check_grad(lora.lora_A.grad, rda, tol)
    _check_grad(lora.lora_B.grad, rdb, tol)
    assert lora.lora_A.grad.dtype == torch.float32 and lora.lora_B.grad.dtype == torch.float32
    for _, buf in ql.named_buffers():
        assert buf.grad is None


def test_lora_dropout_path_and_int8_base(dev):
    """With active dropout an NF4 base runs the fused kernels on drop(x) (the
    dX kernel applies dropout's backward); an INT8 base adds the adapter after
    the int8 kernel.  Both give LoRA gradients."""
    for bits in (4, 8):
        ql = QuantLinear.from_linear(_linear(256, 192, seed=8).to(dev), bits=bits)
        lora = LoRALinear(ql, r=8, lora_dropout=0.1)
        with torch.no_grad():
            lora.lora_B.normal_()
        lora.train()
        x = torch.randn(6, 256, device=dev, dtype=torch.bfloat16)
        lora(x).float().sum().backward()
        assert lora.lora_A.grad.abs().sum() > 0 and lora.lora_B.grad.abs().sum() > 0
        lora.eval()
        with torch.no_grad():
            y = lora(x)
            ref = R.lora_forward(x.cpu(), ql(x).cpu(), lora.lora_A.cpu(), lora.lora_B.cpu(), lora.scaling)
        _check(y, ref)


@pytest.mark.parametrize("M", [4, 300])
def test_lora_dropout_fused_matches_oracle(dev, M):
    """LoRALinear with lora_dropout = 0.1 in training mode (lora_layer.py:67,
    quantize_model's default dropout, model/quantize_model.py:41) runs the
    fused kernels on drop(x): y, dX (the dX kernel applies the dropout mask to
    the adapter's input gradient), dA and dB against the oracle with the same
    keep-mask, which torch's dropout kernel regenerates from the same seed."""
    K, N, r, p = 512, 384, 16, 0.1
    ql = QuantLinear.from_linear(_linear(K, N, seed=31).to(dev), bits=4)
    lora = LoRALinear(ql, r=r, lora_alpha=32, lora_dropout=p)
    with torch.no_grad():
        lora.lora_B.normal_(0.0, 0.01)
    lora.train()
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    dy = (torch.randn(M, N, generator=g) * 0.1).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    torch.cuda.manual_seed(1234)
    y = lora(xd)
    y.backward(dy.to(dev))
    torch.cuda.manual_seed(1234)
    _, mask = torch.ops.aten.native_dropout(x.to(dev), p, True)
    mask = mask.cpu()
    assert 0 < int(mask.sum()) < mask.numel()
    ry, rdx, rda, rdb = R.lora_linear_grads(x, _oracle_weight(ql)[:N * K].reshape(N, K), ql.bias.cpu(),
                                            lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu(),
                                            lora.scaling, dy, dropout_mask=mask, dropout_p=p)
    _check(y, ry)
    _check(xd.grad, rdx)
    _check_grad(lora.lora_A.grad, rda)
    _check_grad(lora.lora_B.grad, rdb)
    # without the mask the adapter term differs: the test sees the dropout
    ny, _, _, _ = R.lora_linear_grads(x, _oracle_weight(ql)[:N * K].reshape(N, K), ql.bias.cpu(),
                                      lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu(), lora.scaling, dy)
    assert not torch.equal(ny, ry)


def test_merge_and_unmerge(dev):
    """lora_layer.py:72-128: merged fp16 weight = fp16(W_deq + B @ A * s),
    guard on a second merge, unmerge back to the adapted quantized forward.
    The adapters are kept through the merge (the reference zeroes them,
    lora_layer.py:111-113, so its unmerge cannot restore the adapted layer)."""
    ql = QuantLinear.from_linear(_linear(256, 128, seed=9).to(dev), bits=4)
    lora = LoRALinear(ql, r=8)
    with torch.no_grad():
        lora.lora_A.normal_()
        lora.lora_B.normal_()
    a, b = lora.lora_A.detach().cpu().clone(), lora.lora_B.detach().cpu().clone()
    x = torch.randn(2, 256, device=dev)
    pre = lora(x)
    lora.merge_lora()
    post = lora(x)
    ref_w = (_oracle_weight(ql)[:128 * 256].reshape(128, 256) + (b @ a) * lora.scaling).to(torch.float16)
    assert torch.allclose(ql.merged_fp16_weight.cpu().float(), ref_w.float(), atol=2e-3, rtol=1e-3)
    assert torch.allclose(post, pre, atol=2.0)
    assert lora.merged
    assert torch.equal(lora.lora_A.detach().cpu(), a) and torch.equal(lora.lora_B.detach().cpu(), b)
    with pytest.raises(RuntimeError, match="LoRA already merged"):
        lora.merge_lora()
    lora.unmerge_lora()
    assert ql.merged_fp16_weight is None and not ql.merged_mode
    assert torch.equal(lora(x), pre)


@pytest.mark.parametrize("M", [1, 300])
def test_double_quant_layer(dev, M):
    """enable_double_quant (quant_linear.py:108-119, double_quant.py:160-200):
    codes unchanged, weight_scales emptied, forward = double_dequantize +
    F.linear."""
    K, N = 512, 384
    ql = QuantLinear.from_linear(_linear(K, N, seed=10).to(dev), bits=4)
    codes = ql.weight_quant.clone()
    w32 = R.dequantize_int4(ql.weight_quant.cpu(), ql.weight_scales.cpu(), 64)[:N * K].reshape(N, K)
    assert ql.enable_double_quant()
    assert torch.equal(ql.weight_quant, codes) and ql.weight_scales.numel() == 0
    assert ql.c2.dtype == torch.float8_e4m3fnuz and ql.use_double_quant
    _, c2, c2s, _ = R.double_quantize(w32, 64, 256)
    assert torch.equal(ql.c2.cpu().view(torch.uint8), c2.view(torch.uint8))
    assert torch.equal(ql.c2_scales.cpu(), c2s)
    x = torch.randn(M, K).to(torch.bfloat16)
    y = ql(x.to(dev))
    wdq = R.double_dequantize(ql.weight_quant.cpu(), c2, c2s, (N, K), 64, 256, True)
    _check(y, R.quant_linear_forward(x, wdq.reshape(-1), ql.bias.cpu(), N, K))


class _FakeAttention(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(128, 128)
        self.k_proj = nn.Linear(128, 128)
        self.v_proj = nn.Linear(128, 128)
        self.ff = nn.Linear(128, 512)


class _FakeTransformer(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([_FakeAttention() for _ in range(4)])

    def forward(self, x):
        for layer in self.layers:
            x = layer.v_proj(layer.q_proj(x))
        return x


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_model_train_step(dev, bits, dtype):
    """test_quantize_model.py of the reference on the GPU: forward, backward,
    only adapters get gradients."""
    torch.manual_seed(0)
    model = _FakeTransformer().to(dev)
    quantize_model(model, bits=bits, lora_dropout=0.0)
    for layer in model.layers:
        with torch.no_grad():
            layer.q_proj.lora_B.normal_(0, 0.01)
    x = torch.randn(2, 128, device=dev, dtype=dtype)
    out = model(x)
    assert out.shape == (2, 128) and out.dtype == dtype
    out.float().mean().backward()
    for name, p in model.named_parameters():
        if "lora_" in name:
            assert p.grad is not None and torch.isfinite(p.grad).all()
        else:
            assert p.grad is None or not p.requires_grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_dequant_nf4_matmul(dev, dtype):
    """dequant_matmul.py:214-229,338-351,367-376: 1-D or 2-D packed weight,
    leading dims kept, dX = dY . W_deq."""
    K, N = 512, 384
    w = torch.randn(N, K) * 0.02
    packed, absmax = R.quantize_int4(w, 64)
    bias = torch.randn(N) * 0.1
    x = torch.randn(2, 5, K).to(dtype)
    xd = x.to(dev).requires_grad_(True)
    y = rocm_qlora.fused_dequant_nf4_matmul(xd, packed.to(dev), absmax.to(dev), bias.to(dev))
    y2 = rocm_qlora.fused_dequant_nf4_matmul(x.to(dev), packed.view(N, K // 2).to(dev), absmax.to(dev),
                                             bias.to(dev))
    assert torch.equal(y.detach(), y2)
    wf = R.dequantize_int4(packed, absmax, 64)
    tol = FP32_TOL if dtype == torch.float32 else RTOL
    _check(y, R.quant_linear_forward(x, wf, bias, N, K), tol)
    dy = (torch.randn(2, 5, N) * 0.1).to(dtype)
    y.backward(dy.to(dev))
    _check(xd.grad, R.nf4_dx(dy, packed, absmax, N, K), tol)


def test_fused_dequant_int8_matmul(dev):
    """Per-row and blockwise scales, the reference's block 32 (unfused route),
    bias added exactly (tests/v2/test_kernels.py:31-105 of the reference)."""
    M, N, K = 4, 128, 64
    x = torch.randn(M, K)
    w = torch.randn(N, K)
    for bs in (32, 64):
        q, s = R.quantize_int8(w.flatten(), bs)
        q = q.reshape(N, K)
        ref = torch.nn.functional.linear(x, R.dequantize_int8(q, s, bs).reshape(N, K))
        got = rocm_qlora.fused_dequant_int8_matmul(x.to(dev), q.to(dev), s.to(dev), block_size=bs)
        _check(got, ref, FP32_TOL)
    qr, sr = R.quantize_int8(w, per_channel=True)
    xb = x.to(torch.bfloat16)
    got = rocm_qlora.fused_dequant_int8_matmul(xb.to(dev), qr.to(dev), sr.to(dev))
    _check(got, R.int8_linear(xb, qr, sr))
    zq = torch.zeros(N, K, dtype=torch.int8, device=dev)
    ones = torch.ones(N * K // 64, device=dev)
    bias = torch.ones(N, device=dev) * 5.0
    for xx in (x.to(dev), xb.to(dev)):
        d = (rocm_qlora.fused_dequant_int8_matmul(xx, zq, ones, bias=bias)
             - rocm_qlora.fused_dequant_int8_matmul(xx, zq, ones))
        assert torch.equal(d, bias.to(xx.dtype).expand(M, N))


def test_hip_kernels_entry_points(dev):
    from rocm_qlora.hip_kernels import (hip_dequant_int4_matmul, hip_dequant_int8_matmul, enable_hip_kernels,
                                        is_hip_kernel_available, benchmark_hip_vs_triton)
    assert is_hip_kernel_available()
    K, N = 256, 512
    w = torch.randn(N, K, device=dev) * 0.02
    packed, absmax = rocm_qlora.quantize_int4(w.flatten())
    x = torch.randn(3, K, device=dev, dtype=torch.float16)
    assert torch.equal(hip_dequant_int4_matmul(x, packed, absmax), rocm_qlora.fused_dequant_nf4_matmul(x, packed, absmax))
    q, s = rocm_qlora.quantize_int8(w.flatten())
    y8 = hip_dequant_int8_matmul(x, q, s)
    _check(y8, R.quant_linear_forward(x.cpu(), R.dequantize_int8(q.cpu(), s.cpu()), None, N, K))
    model = nn.Sequential(QuantLinear(64, 128, bits=4), nn.ReLU(), QuantLinear(128, 64, bits=8))
    assert enable_hip_kernels(model) == 2
    r = benchmark_hip_vs_triton(size=(128, 128), n_runs=5)
    assert r["hip_available"] and r["hip_ms"] > 0 and r["triton_ms"] > 0 and r["winner"] in ("hip", "triton")


def test_dequantize_nf4_triton_bf16_bit_exact(dev):
    w = torch.randn(96, 128) * 0.02
    packed, absmax = R.quantize_int4(w, 64)
    out = rocm_qlora.kernels.dequantize_nf4_triton(packed.to(dev), absmax.to(dev), 64, (96, 128))
    ref = R.dequantize_int4(packed, absmax, 64).to(torch.bfloat16).view(96, 128)
    assert out.dtype == torch.bfloat16
    assert torch.equal(out.cpu().view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 300])
def test_fp8_wrapper_native(dev, M, bits):
    """FP8LinearWrapper (fp8_linear.py:69-118) on gfx950: base matmul by the
    FP8 kernels (per-tensor e4m3fnuz of x and W_deq), LoRA term in bf16,
    dX = dY . W by the NF4 / INT8 dX kernels from the stored codes."""
    from rocm_qlora.fp8 import FP8LinearWrapper, wrap_model_for_fp8
    K, N = 512, 384
    ql = QuantLinear.from_linear(_linear(K, N, seed=11).to(dev), bits=bits)
    lora = LoRALinear(ql, r=8, lora_alpha=16)
    with torch.no_grad():
        lora.lora_B.normal_(0, 0.01)
    wrapped = FP8LinearWrapper(lora)
    assert wrapped.backend == "native", wrapped.fp8_info
    x = torch.randn(M, K).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y = wrapped(xd)
    wdeq = _oracle_weight(ql)[:N * K].reshape(N, K).to(torch.bfloat16)
    base = R.fp8_linear(x, wdeq, ql.bias.cpu().to(torch.bfloat16))
    ref = R.lora_forward(x, base, lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu(), lora.scaling)
    _check(y, ref)
    dy = (torch.randn(M, N) * 0.1).to(torch.bfloat16)
    y.backward(dy.to(dev))
    dx_ref = dy @ wdeq + ((dy * lora.scaling) @ lora.lora_B.detach().cpu().to(torch.bfloat16)) \
        @ lora.lora_A.detach().cpu().to(torch.bfloat16)
    _check(xd.grad, dx_ref)
    model = nn.Sequential(LoRALinear(QuantLinear.from_linear(_linear(K, N, seed=12).to(dev), bits=4)))
    model, status = wrap_model_for_fp8(model)
    assert status["layers_wrapped"] == 1 and status["enabled"] and status["backend"] == "native"


def test_custom_operators_opcheck(dev):
    """torch.library.opcheck of the registered NF4 operators on GPU inputs:
    schema, fake implementation and dispatch agree with the real kernels."""
    K, N, M = 256, 128, 5
    g = torch.Generator().manual_seed(71)
    w = torch.randn(N, K, generator=g) * 0.02
    p, s = rocm_qlora.quantize_int4(w.to(dev), 64)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    a = (torch.randn(16, K, generator=g) * 0.05).to(dev)
    b = (torch.randn(N, 16, generator=g) * 0.01).to(dev)
    torch.library.opcheck(torch.ops.rocm_qlora.nf4_linear.default,
                          (x, p, s, N, 64, None, None, None, 256, True, a, b, 2.0, None))
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    torch.library.opcheck(torch.ops.rocm_qlora.nf4_linear_dx.default,
                          (dy, p, s, K, 64, None, None, 256, True, a, b, 2.0, None, 1.0))


def test_torch_compile_without_graph_breaks(dev):
    """LoRALinear(QuantLinear) under torch.compile (fullgraph: no graph break
    at the HIP calls; AOT autograd traces the backward through the dX
    operator) matches eager bit for bit, forward and gradients."""
    torch.manual_seed(5)
    lin = nn.Linear(256, 128).to(dev)
    ql = QuantLinear.from_linear(lin, bits=4, block_size=64)
    lora = LoRALinear(ql, r=8, lora_alpha=16)
    with torch.no_grad():
        lora.lora_B.normal_(0, 0.01)
    x = torch.randn(2, 7, 256, device=dev, dtype=torch.bfloat16)

    def run(module):
        xi = x.clone().requires_grad_(True)
        y = module(xi)
        y.float().square().sum().backward()
        grads = (xi.grad.clone(), lora.lora_A.grad.clone(), lora.lora_B.grad.clone())
        lora.zero_grad()
        return y.detach(), grads

    ye, ge = run(lora)
    yc, gc = run(torch.compile(lora, backend="aot_eager", fullgraph=True))
    assert torch.equal(yc, ye)
    for a, b in zip(gc, ge):
        assert torch.equal(a, b)
