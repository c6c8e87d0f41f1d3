"""Calls outside the specialized kernels' shapes run on the library's
generic HIP kernels (csrc/generic_linear.hip), never on a vendor GEMM:

- the reference's own 37 x 73 layer (tests/test_quant_linear.py:92-101 of
  the reference), INT8 and NF4, at M = 1, 5 and 40, fp32 / bf16 / fp16;
- NF4 with K = 320 and block size 32 (blocks straddle no 64-multiple),
  with bias and LoRA, forward and dX (LoRA and dropout mask), 16-bit and
  fp32;
- fp32 NF4 with LoRA rank 128 (the fp32 kernel stages 64 ranks);
- INT8 with fp32 activations, odd K, per-row and blockwise scales, and the
  INT8 dX;
- FP8 with fp32 activations and with an odd K;
- activations whose rows are not 16-byte aligned, straight through the ABI.

Each output is checked against the oracle's restatement of the reference's
dequantize-then-F.linear path at rtol = atol = 1e-2 (16-bit results) or
1e-3 (fp32 results); gradients with atol taken relative to the largest
reference magnitude.  The last test profiles such calls and finds only this
library's kernels and torch's elementwise kernels among the GPU kernels.
"""
import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import qlora_ref as R
from rocm_qlora import LoRALinear, QuantLinear, ops
from rocm_qlora import _native as nat
from rocm_qlora.kernels import dequant_matmul as dm
from rocm_qlora.quantization import quantize_int4

pytestmark = pytest.mark.gpu

TOL16 = 1e-2
TOL32 = 1e-3


def _tol(dtype):
    return TOL32 if dtype == torch.float32 else TOL16


def _check(got, ref, tol):
    got = got.detach().cpu().float()
    ref = ref.detach().float()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = (got - ref).abs()
    bad = err > tol + tol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


def _check_grad(got, ref, tol):
    got = got.detach().cpu().float()
    ref = ref.detach().float()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    scale = float(ref.abs().max())
    err = (got - ref).abs()
    bad = err > tol * scale + tol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


def _linear(K, N, seed):
    torch.manual_seed(seed)
    lin = nn.Linear(K, N)
    with torch.no_grad():
        lin.weight.normal_(0.0, 0.02)
        lin.bias.normal_(0.0, 0.1)
    return lin


def _randn(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _oracle_weight(ql):
    q, s = ql.weight_quant.cpu(), ql.weight_scales.cpu()
    if ql.bits == 8:
        return R.dequantize_int8(q, s, ql.block_size)
    return R.dequantize_int4(q, s, ql.block_size)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 5, 40])
def test_reference_37x73_layer(dev, bits, dtype, M):
    print(f"37x73 bits={bits} {dtype} M={M}", flush=True)
    ql = QuantLinear.from_linear(_linear(37, 73, seed=3).to(dev), bits=bits, block_size=64)
    x = _randn((M, 37), seed=M, dtype=dtype)
    y = ql(x.to(dev))
    assert y.shape == (M, 73) and y.dtype == dtype
    _check(y, R.quant_linear_forward(x, _oracle_weight(ql), ql.bias.cpu(), 73, 37), _tol(dtype))


def _nf4_layer(N, K, bs, rank, seed, dev, lora_dtype=torch.float32):
    w = _randn((N, K), seed, scale=0.02)
    packed, absmax = quantize_int4(w.to(dev), bs)
    a = torch.empty(rank, K)
    nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=torch.Generator().manual_seed(seed + 1))
    b = _randn((N, rank), seed + 2, scale=0.05)
    bias = _randn((N,), seed + 3, scale=0.1)
    return packed, absmax, a.to(lora_dtype), b.to(lora_dtype), bias


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [1, 5, 40])
def test_nf4_k320_block32_lora_forward(dev, dtype, M):
    K, N, bs, rank = 320, 200, 32, 16
    print(f"nf4 K={K} block={bs} {dtype} M={M}", flush=True)
    packed, absmax, a, b, bias = _nf4_layer(N, K, bs, rank, seed=11, dev=dev)
    x = _randn((M, K), seed=20 + M, dtype=dtype)
    y = ops.nf4_linear(x.to(dev), packed, absmax, N, bs, bias.to(dev), lora_a=a.to(dev), lora_b=b.to(dev),
                       scaling=0.5)
    ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), bias, a, b, 0.5, N, block_size=bs)
    _check(y, ref, _tol(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("masked", [False, True])
def test_nf4_k320_block32_dx(dev, dtype, masked):
    K, N, bs, rank, M, s = 320, 200, 32, 16, 24, 0.5
    print(f"nf4 dX K={K} N={N} block={bs} {dtype} masked={masked}", flush=True)
    packed, absmax, a, b, _ = _nf4_layer(N, K, bs, rank, seed=31, dev=dev)
    dy = _randn((M, N), seed=5, dtype=dtype)
    mask = torch.rand(M, K, generator=torch.Generator().manual_seed(6)) > 0.3 if masked else None
    p = 0.3
    dx = ops.nf4_linear_dx(dy.to(dev), packed, absmax, K, bs, lora_a=a.to(dev), lora_b=b.to(dev), scaling=s,
                           lora_mask=mask.to(dev) if masked else None, mask_scale=1.0 / (1.0 - p))
    base = R.nf4_dx(dy, packed.cpu(), absmax.cpu(), N, K, block_size=bs)
    dl = ((dy * s) @ b.to(dtype)) @ a.to(dtype)
    if masked:
        dl = torch.ops.aten.native_dropout_backward(dl, mask, 1.0 / (1.0 - p))
    _check(dx, base + dl, _tol(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nf4_odd_layer_autograd(dev, dtype):
    """LoRALinear on a 37 -> 73 NF4 layer (block 64 over the flat weight):
    y, dX, dA and dB against the oracle's float64 / CPU restatement."""
    print(f"nf4 autograd 37x73 {dtype}", flush=True)
    ql = QuantLinear.from_linear(_linear(37, 73, seed=8).to(dev), bits=4)
    lora = LoRALinear(ql, r=8, lora_alpha=16)
    with torch.no_grad():
        lora.lora_B.copy_(_randn((73, 8), seed=9, scale=0.05).to(dev))
    x = _randn((6, 37), seed=10, dtype=dtype)
    xd = x.to(dev).requires_grad_(True)
    y = lora(xd)
    dy = _randn((6, 73), seed=12, dtype=dtype)
    y.backward(dy.to(dev))
    w = _oracle_weight(ql)[:73 * 37].reshape(73, 37)
    A, B = lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu()
    ref = R.lora_forward(x, R.quant_linear_forward(x, w.flatten(), ql.bias.cpu(), 73, 37), A, B, lora.scaling)
    _check(y, ref, _tol(dtype))
    wd = w.to(dtype)
    dx_ref = dy @ wd + ((dy * lora.scaling) @ B.to(dtype)) @ A.to(dtype)
    _check_grad(xd.grad, dx_ref, _tol(dtype))
    dv = dy.double() * lora.scaling
    _check_grad(lora.lora_B.grad, dv.T @ (x.double() @ A.double().T), _tol(dtype))
    _check_grad(lora.lora_A.grad, (dv @ B.double()).T @ x.double(), _tol(dtype))


@pytest.mark.parametrize("M", [1, 40])
def test_nf4_fp32_rank128(dev, M):
    K, N, rank = 512, 384, 128
    print(f"nf4 fp32 rank={rank} M={M}", flush=True)
    packed, absmax, a, b, bias = _nf4_layer(N, K, 64, rank, seed=41, dev=dev)
    x = _randn((M, K), seed=42)
    y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, bias.to(dev), lora_a=a.to(dev), lora_b=b.to(dev),
                       scaling=0.25)
    ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), bias, a, b, 0.25, N)
    _check(y, ref, TOL32)


def test_nf4_unaligned_rows_through_abi(dev):
    """x rows 2 bytes off a 16-byte boundary at M = 40 (the MFMA GEMM reads
    16 bytes at a time): the ABI runs the generic kernels."""
    M, K, N, rank = 40, 256, 192, 16
    packed, absmax, a, b, bias = _nf4_layer(N, K, 64, rank, seed=51, dev=dev)
    x = _randn((M, K), seed=52, dtype=torch.bfloat16)
    buf = torch.zeros(M * K + 1, dtype=torch.bfloat16, device=dev)
    xd = buf[1:].view(M, K)
    xd.copy_(x.to(dev))
    assert xd.data_ptr() % 16 != 0
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    import ctypes
    nb = ctypes.c_int64(0)
    nat.call("rq_nf4_linear_workspace_size", nat.dtype_code(torch.bfloat16), M, K, N, rank, ctypes.byref(nb))
    ws = torch.zeros(nb.value, dtype=torch.uint8, device=dev)
    ad, bd, biasd = a.to(dev), b.to(dev), bias.to(dev)
    nat.call("rq_nf4_linear", xd.data_ptr(), nat.dtype_code(torch.bfloat16), M, K, K,
             packed.data_ptr(), N, 64, absmax.data_ptr(), nat.dtype_code(absmax.dtype),
             None, nat.C2_FP8_E4M3FNUZ, 256, biasd.data_ptr(), nat.dtype_code(biasd.dtype),
             xd.data_ptr(), K, ad.data_ptr(), bd.data_ptr(), rank, nat.dtype_code(ad.dtype), rank, 0.5,
             y.data_ptr(), N, ws.data_ptr(), ws.numel(), nat.stream_handle(dev))
    ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), bias, a, b, 0.5, N)
    _check(y, ref, TOL16)


def _int8_weight(N, K, bs, seed):
    w = _randn((N, K), seed, scale=0.02)
    if bs == 0:
        q, s = R.quantize_int8(w, per_channel=True)
        return q, s, R.dequantize_int8(q, s)
    q, s = R.quantize_int8(w.flatten(), bs)
    return q, s, R.dequantize_int8(q, s, bs)[:N * K].reshape(N, K)


@pytest.mark.parametrize("dtype,K,bs", [(torch.float32, 512, 64), (torch.float32, 100, 0),
                                        (torch.bfloat16, 100, 64), (torch.float16, 96, 32),
                                        (torch.bfloat16, 512, 48)])
@pytest.mark.parametrize("M", [1, 40])
def test_int8_generic_forward(dev, dtype, K, bs, M):
    N = 136
    print(f"int8 {dtype} K={K} block={bs} M={M}", flush=True)
    q, s, wdq = _int8_weight(N, K, bs, seed=61)
    bias = _randn((N,), 62, scale=0.1)
    x = _randn((M, K), seed=63, dtype=dtype)
    y = ops.int8_linear(x.to(dev), q.to(dev), s.to(dev), N, bs, bias.to(dev))
    ref = F.linear(x, wdq.to(dtype), bias.to(dtype))
    _check(y, ref, _tol(dtype))


@pytest.mark.parametrize("dtype,K,bs", [(torch.bfloat16, 512, 64), (torch.float32, 512, 64),
                                        (torch.bfloat16, 100, 0), (torch.float16, 96, 32)])
def test_int8_dx(dev, dtype, K, bs):
    """INT8 backward dX = dY . RND(W_deq) (dequant_matmul.py:308-324), also
    through autograd."""
    N, M = 136, 24
    print(f"int8 dX {dtype} K={K} block={bs}", flush=True)
    q, s, wdq = _int8_weight(N, K, bs, seed=71)
    dy = _randn((M, N), seed=72, dtype=dtype)
    dx = ops.int8_linear_dx(dy.to(dev), q.to(dev), s.to(dev), K, bs)
    _check(dx, dy @ wdq.to(dtype), _tol(dtype))
    x = _randn((M, K), seed=73, dtype=dtype).to(dev).requires_grad_(True)
    w = dm.Int8Weight(q.to(dev), s.to(dev), N, K, bs)
    y = dm.int8_linear(x, w)
    y.backward(dy.to(dev))
    _check(x.grad, dy @ wdq.to(dtype), _tol(dtype))


@pytest.mark.parametrize("dtype,K", [(torch.float32, 512), (torch.float32, 100), (torch.bfloat16, 100),
                                     (torch.float16, 72)])
@pytest.mark.parametrize("M", [1, 40])
def test_fp8_generic(dev, dtype, K, M):
    """fp8_linear.py:27-60 with fp32 activations or a K the fp8 matrix cores
    do not take: x8 and w8 decoded and their fp32 products summed."""
    N = 96
    print(f"fp8 {dtype} K={K} M={M}", flush=True)
    w = _randn((N, K), seed=81, scale=0.05, dtype=dtype)
    bias = _randn((N,), 82, scale=0.1, dtype=dtype)
    x = _randn((M, K), seed=83, dtype=dtype)
    codes, scale = ops.fp8_quantize(w.to(dev))
    y = ops.fp8_linear(x.to(dev), codes, scale, bias.to(dev))
    ref = R.fp8_linear(x, w, bias)
    _check(y, ref, _tol(dtype))


def test_generic_calls_run_no_vendor_gemm(dev):
    """A profile of generic-path calls (NF4 LoRA forward and dX at 37 x 73,
    INT8 fp32 forward and dX, FP8 fp32) holds this library's kernels and
    torch's elementwise kernels only."""
    from torch.profiler import ProfilerActivity, profile
    ql = QuantLinear.from_linear(_linear(37, 73, seed=91).to(dev), bits=4)
    lora = LoRALinear(ql, r=8, lora_alpha=16)
    lora.lora_A.requires_grad_(False)
    lora.lora_B.requires_grad_(False)
    q8 = QuantLinear.from_linear(_linear(37, 73, seed=92).to(dev), bits=8)
    w8 = _randn((64, 100), 93, scale=0.05)
    codes, scale = ops.fp8_quantize(w8.to(dev))
    x = _randn((5, 37), 94).to(dev)
    torch.cuda.synchronize(dev)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        xg = x.clone().requires_grad_(True)
        lora(xg.to(torch.bfloat16)).float().sum().backward()
        x8 = x.clone().requires_grad_(True)
        dm.int8_linear(x8, q8.int8_weight(), q8.bias).sum().backward()
        ops.fp8_linear(_randn((5, 100), 95).to(dev), codes, scale)
        torch.cuda.synchronize(dev)
    names = sorted({e.name for e in prof.events() if e.device_type.name in ("CUDA", "PrivateUse1")})
    if not names:
        pytest.skip("the profiler recorded no GPU kernels on this system")
    ours = [n for n in names if "rq::" in n or n.startswith("_ZN2rq")]
    vendor = [n for n in names if n not in ours and any(k in n.lower() for k in ("cijk", "gemm", "rocblas",
                                                                                  "hipblas", "gemv"))]
    assert not vendor, f"vendor GEMM kernels ran: {vendor}"
    assert any("generic_linear_kernel" in n for n in ours), names
