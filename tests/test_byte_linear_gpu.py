"""GPU parity of the INT8 and FP8 linears (HIP kernels through the C ABI) vs
the oracle's restatements: row-absmax / blockwise INT8 dequantize-then-
F.linear (quant_ops.py:17-78, quant_linear.py:193-197) and the FP8
_FP8LinearFunc recipe (fp8_linear.py:27-60).  Tolerance rtol = atol = 1e-2
in the activation dtype for outputs; the FP8 quantization (codes and scale)
and the INT8 weight operand are bit-exact.  Full Llama-3-70B MLP shapes
(K=8192, N=28672) are checked on every output element."""
import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import ops
from rocm_qlora.quantization import quantize_int8

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2


def _check(got, ref):
    got = got.cpu().float()
    ref = ref.float()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


def _weights(N, K, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * 0.02).to(dtype)


def _x(M, K, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(dtype)


@pytest.mark.parametrize("M", [1, 512, 4096])
def test_int8_row_absmax_llama70b_mlp(dev, M):
    """Config: INT8 per-output-row absmax weights (N(0,0.02)), bf16 x, K=8192, N=28672."""
    K, N = 8192, 28672
    print(f"int8 row-absmax M={M}", flush=True)
    w = _weights(N, K, seed=5).to(dev)
    q, s = quantize_int8(w, per_channel=True)
    x = _x(M, K, torch.bfloat16, seed=M)
    y = ops.int8_linear(x.to(dev), q, s, N, block_size=0)
    ref = R.int8_linear(x, q.cpu(), s.cpu())
    _check(y.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ["m1", "m5", "m16", "m17", "m300", "blockwise", "bias", "odd_n", "k64",
                                  "bf16_scales"])
def test_int8_variants(dev, dtype, case):
    N, K = 704, 512
    M = {"m1": 1, "m5": 5, "m16": 16, "m17": 17}.get(case, 300)
    N = 1000 if case == "odd_n" else N
    K = 64 if case == "k64" else K
    print(f"int8 variant {case} {dtype}", flush=True)
    w = _weights(N, K, seed=7).to(dev)
    if case == "bf16_scales":
        w = w.to(torch.bfloat16)
    block = 64 if case == "blockwise" else 0
    if block:
        q, s = quantize_int8(w, block_size=64)
    else:
        q, s = quantize_int8(w, per_channel=True)
    g = torch.Generator().manual_seed(3)
    bias = (torch.randn(N, generator=g) * 0.1) if case == "bias" else None
    x = _x(M, K, dtype, seed=11)
    y = ops.int8_linear(x.to(dev), q, s, N, block_size=block, bias=None if bias is None else bias.to(dev))
    if block:
        wf = R.dequantize_int8(q.cpu(), s.cpu(), 64)[:N * K].reshape(N, K)
    else:
        wf = R.dequantize_int8(q.cpu().reshape(N, K), s.cpu())
    ref = torch.nn.functional.linear(x, wf.to(dtype), None if bias is None else bias.to(dtype))
    _check(y, ref)


@pytest.mark.parametrize("M", [7, 300])
@pytest.mark.parametrize("block", [0, 64])
def test_int8_weight_operand_bit_exact(dev, M, block):
    """One-hot activation rows pick single weights: y[m, n] = RND(q * s) bit
    for bit (GEMV path for M <= 16, MFMA GEMM otherwise)."""
    N, K = 384, 1024
    w = _weights(N, K, seed=17).to(dev)
    q, s = quantize_int8(w, block_size=64) if block else quantize_int8(w, per_channel=True)
    g = torch.Generator().manual_seed(19)
    ks = torch.randint(0, K, (M,), generator=g)
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    x[torch.arange(M), ks] = 1.0
    y = ops.int8_linear(x.to(dev), q, s, N, block_size=block)
    if block:
        wf = R.dequantize_int8(q.cpu(), s.cpu(), 64)[:N * K].reshape(N, K)
    else:
        wf = R.dequantize_int8(q.cpu().reshape(N, K), s.cpu())
    ref = wf.to(torch.bfloat16)[:, ks].T
    assert torch.equal(y.cpu().view(torch.int16), ref.contiguous().view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fp8_quantize_bit_exact(dev, dtype):
    """Codes and scale of the per-tensor e4m3fnuz recipe (fp8_linear.py:33-42)
    equal the oracle's bit for bit; the absmax element encodes to 0x7F."""
    t = (torch.randn(257, 1000, generator=torch.Generator().manual_seed(23)) * 0.05).to(dtype)
    t[3, 7] = 0.9
    codes, scale = ops.fp8_quantize(t.to(dev))
    rc, rs = R.fp8_quantize_tensor(t)
    assert float(scale) == float(rs)
    assert torch.equal(codes.view(torch.uint8).cpu(), rc.view(torch.uint8))
    assert int(codes.view(torch.uint8)[3, 7]) == 0x7F


@pytest.mark.parametrize("M", [1, 512, 4096])
def test_fp8_llama70b_mlp(dev, M):
    """Config: FP8 e4m3 weights and activations with per-tensor fp32 scales,
    K=8192, N=28672, bf16 output vs dequantize-then-matmul."""
    K, N = 8192, 28672
    print(f"fp8 M={M}", flush=True)
    w = _weights(N, K, seed=29, dtype=torch.bfloat16)
    wc, ws = ops.fp8_quantize(w.to(dev))
    x = _x(M, K, torch.bfloat16, seed=31 + M)
    y = ops.fp8_linear(x.to(dev), wc, ws)
    # the oracle's recipe on the whole output
    x8, xs = R.fp8_quantize_tensor(x)
    w8, wsr = R.fp8_quantize_tensor(w)
    assert float(ws) == float(wsr)
    ref = ((x8.to(torch.float32) * xs) @ (w8.to(torch.float32) * wsr).T).to(torch.bfloat16)
    _check(y.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 16, 17, 333])
def test_fp8_variants(dev, dtype, M):
    N, K = 640, 768
    w = _weights(N, K, seed=37, dtype=dtype)
    x = _x(M, K, dtype, seed=41)
    g = torch.Generator().manual_seed(43)
    bias = (torch.randn(N, generator=g) * 0.1).to(dtype)
    wc, ws = ops.fp8_quantize(w.to(dev))
    y = ops.fp8_linear(x.to(dev), wc, ws, bias.to(dev))
    ref = R.fp8_linear(x, w, bias)
    _check(y, ref)


@pytest.mark.parametrize("K", [320, 384, 448])
def test_byte_k_step_tails(dev, K):
    """INT8 and FP8 MFMA paths (M > 16) with K / 64 = 5, 6, 7 k-steps: three
    calls in a row each within tolerance and bitwise equal to each other."""
    N, M = 384, 300
    w = _weights(N, K, seed=K)
    x = _x(M, K, torch.bfloat16, seed=K + 1)
    q, s = quantize_int8(w.to(dev), per_channel=True)
    ys = [ops.int8_linear(x.to(dev), q, s, N, block_size=0) for _ in range(3)]
    ref = R.int8_linear(x, q.cpu(), s.cpu())
    for y in ys:
        _check(y, ref)
        assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))
    wb = w.to(torch.bfloat16)
    wc, ws = ops.fp8_quantize(wb.to(dev))
    fs = [ops.fp8_linear(x.to(dev), wc, ws) for _ in range(3)]
    fref = R.fp8_linear(x, wb)
    for y in fs:
        _check(y, fref)
        assert torch.equal(y.view(torch.int16), fs[0].view(torch.int16))


def test_fp8_to_e4m3fn_matches_torch(dev):
    """rq_fp8_fnuz_to_e4m3fn (the fp8 matrix cores' operand encoding) equals
    torch's value conversion .to(torch.float8_e4m3fn) bit for bit: every code
    once, then a ragged random buffer (length not a multiple of 16)."""
    allc = torch.arange(256, dtype=torch.uint8)
    rnd = torch.randint(0, 256, (4099,), generator=torch.Generator().manual_seed(3), dtype=torch.uint8)
    for c in (allc, rnd):
        got = ops.fp8_to_e4m3fn(c.to(dev).view(torch.float8_e4m3fnuz)).view(torch.uint8).cpu()
        want = c.view(torch.float8_e4m3fnuz).to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(got, want)
    # exact except the 8 odd subnormal-range magnitudes (and their negatives)
    fz = allc.view(torch.float8_e4m3fnuz).float()
    fn = ops.fp8_to_e4m3fn(allc.to(dev).view(torch.float8_e4m3fnuz)).cpu().float()
    same = (fz == fn) | (fz.isnan() & fn.isnan())
    assert int((~same).sum()) == 16
    assert float((fz - fn)[~same].abs().max()) <= 2.0 ** -10


@pytest.mark.parametrize("M", [1, 7, 16, 40, 300])
def test_fp8_e4m3fn_weights_same_as_fnuz(dev, M):
    """A weight passed as e4m3fn codes (converted once) gives the same bits as
    the same weight passed as fnuz codes (converted per call), GEMV and GEMM."""
    N, K = 2048, 1024
    w = _weights(N, K, seed=51, dtype=torch.bfloat16)
    x = _x(M, K, torch.bfloat16, seed=52)
    wc, ws = ops.fp8_quantize(w.to(dev))
    y1 = ops.fp8_linear(x.to(dev), wc, ws)
    y2 = ops.fp8_linear(x.to(dev), ops.fp8_to_e4m3fn(wc), ws)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    _check(y1, R.fp8_linear(x, w))


@pytest.mark.parametrize("K", [64, 128, 192, 1088])
@pytest.mark.parametrize("M", [3, 16, 70])
def test_fp8_short_and_ragged_k(dev, M, K):
    """K shorter than the GEMM's load pipeline (1 to 3 stages of 64 k) and K
    not a multiple of the GEMV's 128-k step, with a bias."""
    N = 320
    w = _weights(N, K, seed=K + 60, dtype=torch.bfloat16)
    x = _x(M, K, torch.bfloat16, seed=K + 61)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(62)) * 0.1).to(torch.bfloat16)
    wc, ws = ops.fp8_quantize(w.to(dev))
    y = ops.fp8_linear(x.to(dev), wc, ws, bias.to(dev))
    _check(y, R.fp8_linear(x, w, bias))
