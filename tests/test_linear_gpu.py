"""GPU parity of the NF4 linear (decode GEMV, M <= 16): HIP kernels through
the C ABI vs the oracle's restatement of QuantLinear.forward +
LoRALinear.forward (quant_linear.py:182-197, lora_layer.py:60-70) on the
same seeded inputs.  Tolerance rtol = atol = 1e-2 in the activation dtype,
as the reference's own matmul checks allow (tests/v2/test_kernels.py:31-68
use 1e-4 for identical math).  The weight operand is bit-identical to the
reference's dequantized weight (test_gemv_weight_operand_bit_exact); only the
fp32 summation order differs, so outputs may differ by a bf16 ulp."""
import math

import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import ops
from rocm_qlora.quantization import quantize_int4, double_quantize

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2


def _inputs(N, K, M, dtype, seed, rank=16, bias=False):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    x = torch.randn(M, K, generator=g).to(dtype)
    a = torch.empty(rank, K)
    torch.nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
    b = torch.randn(N, rank, generator=g) * 0.01
    bvec = (torch.randn(N, generator=g) * 0.1) if bias else None
    return w, x, a, b, bvec


def _check(got, ref):
    got = got.cpu().float()
    ref = ref.float()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)])
def test_gemv_llama3_shapes_bf16(dev, M, K, N):
    """Config: decode dequant-GEMV at every Llama-3-8B projection shape, LoRA r=16 fused."""
    print(f"gemv bf16 K={K} N={N} M={M}", flush=True)
    w, x, a, b, _ = _inputs(N, K, M, torch.bfloat16, seed=K + N + M)
    packed, absmax = quantize_int4(w.to(dev), 64)
    y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=a.to(dev), lora_b=b.to(dev), scaling=2.0)
    ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), None, a, b, 2.0, N, 64)
    _check(y, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ["plain", "bias", "odd_n", "block128", "strided_x", "dropout_x", "no_lora",
                                  "k320", "k64", "rank96", "rank256", "bf16_lora"])
def test_gemv_variants(dev, dtype, case):
    N, K, M = (1000 if case == "odd_n" else 768), 512, 5
    K = {"k320": 320, "k64": 64}.get(case, K)
    rank = {"rank96": 96, "rank256": 256}.get(case, 16)
    bs = 128 if case == "block128" else 64
    print(f"gemv variant {case} {dtype}", flush=True)
    w, x, a, b, bvec = _inputs(N, K, M, dtype, seed=7, rank=rank, bias=(case == "bias"))
    if case == "bf16_lora":
        a, b = a.to(dtype), b.to(dtype)
    packed, absmax = quantize_int4(w.to(dev), bs)
    xd = x.to(dev)
    xl = None
    if case == "strided_x":
        big = torch.zeros(M, K + 64, dtype=dtype, device=dev)
        big[:, 32:32 + K] = xd
        xd = big[:, 32:32 + K]
    if case == "dropout_x":
        xl = (x * (torch.rand(x.shape, generator=torch.Generator().manual_seed(3)) > 0.3)).to(dtype)
    la, lb = (None, None) if case == "no_lora" else (a.to(dev), b.to(dev))
    y = ops.nf4_linear(xd, packed, absmax, N, bs, bias=None if bvec is None else bvec.to(dev),
                       lora_a=la, lora_b=lb, scaling=0.5, lora_x=None if xl is None else xl.to(dev))
    wf = R.dequantize_int4(packed.cpu(), absmax.cpu(), bs)
    base = R.quant_linear_forward(x, wf, bvec, N, K)
    if la is None:
        ref = base
    else:
        lx = x if xl is None else xl
        lora = lx @ a.to(dtype).T @ b.to(dtype).T * 0.5
        ref = base + lora.to(base.dtype)
    _check(y, ref)


@pytest.mark.parametrize("N,K,M,rank", [
    (8235, 512, 3, 64),     # 4 tiles per workgroup, the last workgroup with a tile past N, partial tile
    (4800, 512, 16, 16),    # 2 tiles per workgroup, all 16 activation rows
    (14336, 4096, 16, 64),  # 4 tiles per workgroup at M = 16 and rank 64 (largest LDS staging)
    (4800, 4160, 2, 16),    # K split in two with a partial last segment (split-K finisher)
])
def test_gemv_tiling_cases(dev, N, K, M, rank):
    """Tiles per workgroup 1, 2 and 4, dead tiles, K splits: bias + LoRA."""
    print(f"gemv tiling N={N} K={K} M={M} r={rank}", flush=True)
    w, x, a, b, bvec = _inputs(N, K, M, torch.bfloat16, seed=N + K, rank=rank, bias=True)
    packed, absmax = quantize_int4(w.to(dev), 64)
    y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, bias=bvec.to(dev), lora_a=a.to(dev), lora_b=b.to(dev),
                       scaling=0.25)
    wf = R.dequantize_int4(packed.cpu(), absmax.cpu(), 64)
    ref = R.lora_forward(x, R.quant_linear_forward(x, wf, bvec, N, K), a, b, 0.25)
    _check(y, ref)


@pytest.mark.parametrize("M,rank", [(4, 16), (16, 64), (8, 96)])
def test_gemv_k_splits(dev, M, rank):
    """K = 14336 at M > 2 runs as 4 K splits.  With rank <= 64 the last split
    of each workgroup column to count itself sums the splits' partials and
    runs the epilogue in the same launch (rank 96: the finisher launch).
    Bias + LoRA against the oracle; three calls bit-identical, whichever split
    counts itself last, which also shows the counters left at zero."""
    N, K = 4096, 14336
    print(f"gemv k splits M={M} r={rank}", flush=True)
    w, x, a, b, bvec = _inputs(N, K, M, torch.bfloat16, seed=M + rank, rank=rank, bias=True)
    packed, absmax = quantize_int4(w.to(dev), 64)
    args = (x.to(dev), packed, absmax, N, 64)
    kw = dict(bias=bvec.to(dev), lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.25)
    ys = [ops.nf4_linear(*args, **kw) for _ in range(3)]
    wf = R.dequantize_int4(packed.cpu(), absmax.cpu(), 64)
    ref = R.lora_forward(x, R.quant_linear_forward(x, wf, bvec, N, K), a, b, 0.25)
    _check(ys[0], ref)
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2])


def test_gemv_double_quant(dev):
    N, K, M = 2048, 4096, 3
    w, x, a, b, _ = _inputs(N, K, M, torch.bfloat16, seed=21)
    st = double_quantize(w.to(dev), 64, 256)
    y = ops.nf4_linear(x.to(dev), st.W_quant, None, N, 64, c2=st.c2, c2_scales=st.c2_scales,
                       blocksize_2=256, use_fp8_c2=True, lora_a=a.to(dev), lora_b=b.to(dev), scaling=2.0)
    wf = R.double_dequantize(st.W_quant.cpu(), st.c2.cpu(), st.c2_scales.cpu(), (N, K), 64, 256, True)
    base = R.quant_linear_forward(x, wf.reshape(-1), None, N, K)
    ref = R.lora_forward(x, base, a, b, 2.0)
    _check(y, ref)


def test_gemv_leading_dims_and_empty(dev):
    N, K = 256, 256
    w, x, a, b, _ = _inputs(N, K, 6, torch.bfloat16, seed=5)
    packed, absmax = quantize_int4(w.to(dev), 64)
    x3 = x.reshape(2, 3, K).to(dev)
    y = ops.nf4_linear(x3, packed, absmax, N, 64)
    assert y.shape == (2, 3, N) and y.dtype == torch.bfloat16
    ref = R.quant_linear_forward(x, R.dequantize_int4(packed.cpu(), absmax.cpu(), 64), None, N, K)
    _check(y.reshape(6, N), ref)
    e = ops.nf4_linear(torch.empty(0, K, dtype=torch.bfloat16, device=dev), packed, absmax, N, 64)
    assert e.shape == (0, N)


def test_gemv_deterministic(dev):
    N, K, M = 4096, 4096, 16
    w, x, a, b, _ = _inputs(N, K, M, torch.bfloat16, seed=9)
    packed, absmax = quantize_int4(w.to(dev), 64)
    args = (x.to(dev), packed, absmax, N, 64)
    kw = dict(lora_a=a.to(dev), lora_b=b.to(dev), scaling=2.0)
    y1 = ops.nf4_linear(*args, **kw)
    y2 = ops.nf4_linear(*args, **kw)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dq", [False, True])
def test_gemv_weight_operand_bit_exact(dev, dtype, dq):
    """One-hot activation rows pick single weights: y[m, n] = RND(W[n, k_m])
    must equal the reference's dequantize_int4(...).to(dtype) bit for bit
    (quant_ops.py:144-148, quant_linear.py:191-193; double_quant.py:108-118)."""
    N, K = 512, 1024
    g = torch.Generator().manual_seed(17)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    ks = torch.randperm(K, generator=g)[:16]
    x = torch.zeros(16, K, dtype=dtype)
    x[torch.arange(16), ks] = 1.0
    if dq:
        st = double_quantize(w.to(dev), 64, 256)
        y = ops.nf4_linear(x.to(dev), st.W_quant, None, N, 64, c2=st.c2, c2_scales=st.c2_scales)
        wf = R.double_dequantize(st.W_quant.cpu(), st.c2.cpu(), st.c2_scales.cpu(), (N, K), 64, 256, True)
    else:
        packed, absmax = quantize_int4(w.to(dev), 64)
        y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64)
        wf = R.dequantize_int4(packed.cpu(), absmax.cpu(), 64)[:N * K].reshape(N, K)
    ref = wf.to(dtype)[:, ks].T
    assert torch.equal(y.cpu().view(torch.int16), ref.contiguous().view(torch.int16))
