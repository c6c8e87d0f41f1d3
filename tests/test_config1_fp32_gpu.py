"""Config 1: a single NF4 QuantLinear with LoRA (r = 16, alpha = 32) on fp32
activations, 4096 -> 4096, M in {1, 16} -- the reference's CPU-runnable case
(quant_linear.py:189-197 computes in fp32 for fp32 inputs, lora_layer.py:67
keeps the adapter in fp32).  The forward runs the fp32-MFMA kernels
(csrc/nf4_linear_f32.hip) and is checked against the oracle's fp32 CPU
restatement at rtol = atol = 1e-3.  Weights fp32 N(0, 0.02) quantized by the
NF4 quantizer with block 64 and fp32 absmax; A Kaiming-uniform(a = sqrt 5);
B N(0, 0.01); x N(0, 1); fixed seeds."""
import math

import pytest
import torch
import torch.nn as nn

from oracle import qlora_ref as R
from rocm_qlora import LoRALinear, QuantLinear
from rocm_qlora import ops

pytestmark = pytest.mark.gpu

TOL = 1e-3
K = N = 4096
RANK, ALPHA = 16, 32


def _check(got, ref, tol=TOL):
    got = got.detach().cpu().float()
    ref = ref.detach().float()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bad = err > tol + tol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


def _layer(dev, seed, bias):
    g = torch.Generator().manual_seed(seed)
    lin = nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    ql = QuantLinear.from_linear(lin.to(dev), bits=4, block_size=64)
    lora = LoRALinear(ql, r=RANK, lora_alpha=ALPHA)
    with torch.no_grad():
        a = torch.empty(RANK, K)
        nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
        lora.lora_A.copy_(a)
        lora.lora_B.copy_(torch.randn(N, RANK, generator=g) * 0.01)
    lora.eval()
    return ql, lora


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 16])
def test_config1_fp32_lora_linear(dev, M, bias):
    print(f"config 1 fp32 M={M} bias={bias}", flush=True)
    ql, lora = _layer(dev, seed=1 + M, bias=bias)
    assert ql.weight_scales.dtype == torch.float32  # fp32 master -> fp32 absmax
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(100 + M))
    with torch.no_grad():
        y = lora(x.to(dev))
    assert y.dtype == torch.float32
    ref = R.nf4_lora_linear(x, ql.weight_quant.cpu(), ql.weight_scales.cpu(),
                            ql.bias.cpu() if bias else None, lora.lora_A.detach().cpu(),
                            lora.lora_B.detach().cpu(), lora.scaling, N, 64)
    _check(y, ref)


@pytest.mark.parametrize("M", [1, 3, 16, 35, 37])
def test_fp32_base_and_double_quant(dev, M):
    """The base layer alone (no adapter) and after enable_double_quant
    (double_quant.py:160-200), against dequantize -> F.linear in fp32; M = 35
    and 37 run as 16-row blocks (tails of 3 and 5 rows: the vector-ALU and
    the MFMA kernel)."""
    ql, _ = _layer(dev, seed=5, bias=True)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(7 + M))
    w32 = R.dequantize_int4(ql.weight_quant.cpu(), ql.weight_scales.cpu(), 64)
    with torch.no_grad():
        y = ql(x.to(dev))
    _check(y, R.quant_linear_forward(x, w32, ql.bias.cpu(), N, K))
    assert ql.enable_double_quant()
    w2 = R.double_dequantize(ql.weight_quant.cpu(), ql.c2.cpu(), ql.c2_scales.cpu(), (N * K,), 64,
                             ql.blocksize_2, ql.use_fp8_c2)
    with torch.no_grad():
        y2 = ql(x.to(dev))
    _check(y2, R.quant_linear_forward(x, w2, ql.bias.cpu(), N, K))


@pytest.mark.parametrize("M", [2, 5])
def test_fp32_strided_activations_and_lora_input(dev, M):
    """Activation rows with a stride, bf16 LoRA weights widened to fp32, and a
    separate LoRA input (the dropout path) through ops.nf4_linear (M = 2: the
    vector-ALU kernel, M = 5: the MFMA kernel)."""
    ql, lora = _layer(dev, seed=9, bias=False)
    g = torch.Generator().manual_seed(3)
    big = torch.randn(M, K + 12, generator=g)
    x = big[:, 4:4 + K]
    xl = torch.randn(M, K, generator=g)
    a16 = lora.lora_A.detach().to(torch.bfloat16)
    b16 = lora.lora_B.detach().to(torch.bfloat16)
    y = ops.nf4_linear(x.to(dev), ql.weight_quant, ql.weight_scales, N, 64, lora_a=a16, lora_b=b16,
                       scaling=2.0, lora_x=xl.to(dev))
    base = R.quant_linear_forward(x, R.dequantize_int4(ql.weight_quant.cpu(), ql.weight_scales.cpu(), 64),
                                  None, N, K)
    ref = base + (xl @ a16.cpu().float().T @ b16.cpu().float().T * 2.0)
    _check(y, ref)


def test_fp32_call_leaves_sync_area_ready(dev, sync_ready):
    """An fp32 LoRA call shares the stream's rq_nf4_linear workspace with the
    bf16 decode GEMV, whose in-launch LoRA handshake needs the workspace's
    synchronization area in its ready state: the fp32 path keeps its LoRA
    operand after the area, so a bf16 call right after it gives the same bits
    as on a fresh stream."""
    ql, lora = _layer(dev, seed=12, bias=False)
    a, b = lora.lora_A.detach(), lora.lora_B.detach()
    x16 = torch.randn(2, K, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    fresh = torch.cuda.Stream(dev)
    with torch.cuda.stream(fresh):
        want = ops.nf4_linear(x16, ql.weight_quant, ql.weight_scales, N, 64, lora_a=a, lora_b=b, scaling=2.0)
    torch.cuda.synchronize(dev)
    x32 = torch.randn(16, K, generator=torch.Generator().manual_seed(5)).to(dev)
    ops.nf4_linear(x32, ql.weight_quant, ql.weight_scales, N, 64, lora_a=a, lora_b=b, scaling=2.0)
    got = ops.nf4_linear(x16, ql.weight_quant, ql.weight_scales, N, 64, lora_a=a, lora_b=b, scaling=2.0)
    torch.cuda.synchronize(dev)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    assert sync_ready(ops._LINEAR_WS[key])
    assert torch.equal(got, want)
