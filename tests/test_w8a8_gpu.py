"""GPU parity of the W8A8 INT8 mode (int8 activations quantized per row x
int8 per-row weights on the int8 matrix cores, through the C ABI) against
the oracle's restatement (oracle.qlora_ref.quantize_rows_int8 /
w8a8_linear).  The mode has no counterpart in the reference; its activation
recipe is quantize_int8's per-row one (quant_ops.py:29-35) in fp32.

Everything here is integer arithmetic plus a fixed chain of fp32 roundings,
so the bar is bit-exact: codes, scales and outputs.  Full Llama-3-70B MLP
shapes (K=8192, N=28672) are checked on every column of seeded output rows
(rows are independent: each is quantized on its own)."""
import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import W8A8Linear, ops, torch_ops
from rocm_qlora.quantization import quantize_int8

pytestmark = pytest.mark.gpu


def _x(M, K, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, K, generator=g) * scale).to(dtype)


def _w(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(N, K, generator=g) * 0.02


def _equal(got, want, what=""):
    got = got.cpu()
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.is_floating_point():
        diff = got.view(torch.int16 if got.element_size() == 2 else torch.int32) != \
            want.view(torch.int16 if want.element_size() == 2 else torch.int32)
    else:
        diff = got != want
    assert not diff.any(), f"{what}: {int(diff.sum())} of {diff.numel()} differ"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(1, 8), (3, 200), (16, 4096), (64, 8192), (65, 520), (300, 1024)])
def test_quantize_rows_bit_exact(dev, dtype, M, K):
    print(f"w8a8 quantize rows M={M} K={K} {dtype}", flush=True)
    x = _x(M, K, dtype, seed=M * 7 + K, scale=4.0)
    if M > 2:
        x[1] = 0          # zero row: scale 1e-12, codes 0
        x[2, 3] = 1e-30   # a row whose absmax underflows the clamp
        x[2, 4:] = 0
    q, s = ops.int8_quantize_rows(x.to(dev))
    qr, sr = R.quantize_rows_int8(x)
    _equal(s, sr, "scales")
    _equal(q, qr, "codes")


def _half_integer_rows(dtype, n_rows=16, K=64):
    """Rows whose largest value m sets s = RN32(m / 127) and whose other
    values x give quotients that round (rint) differently as RN32(x / s) and
    as RN32(x * RN32(1 / s)): quotients on or within a few fp32 ulps of a
    half-integer, found by brute force over every finite value of dtype."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(dtype).float()
    vals = bits[torch.isfinite(bits)]
    rows = []
    for mx in vals[(vals >= 0.5) & (vals <= 8.0)].tolist():
        s = torch.tensor(mx, dtype=torch.float32) / 127.0
        rs = 1.0 / s
        x = vals[vals.abs() < mx]
        bad = x[torch.round(x / s) != torch.round(x * rs)]  # round half to even, as rint
        if len(bad) == 0:
            continue
        row = torch.zeros(K)
        row[0] = mx
        row[1:1 + min(len(bad), K - 1)] = bad[:K - 1]
        rows.append(row)
        if len(rows) == n_rows:
            break
    assert len(rows) >= 4
    return torch.stack(rows).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quantize_rows_half_integer_quotients(dev, dtype):
    """Rows made of values whose quotients x / s lie on or within a few fp32
    ulps of a half-integer, where a quotient through RN32(1 / s) would round
    to the other integer: the kernel's codes match the oracle's true
    division bit for bit."""
    print(f"w8a8 quantize rows at half-integer quotients {dtype}", flush=True)
    x = _half_integer_rows(dtype)
    q, s = ops.int8_quantize_rows(x.to(dev))
    qr, sr = R.quantize_rows_int8(x)
    _equal(s, sr, "scales")
    _equal(q, qr, "codes")


def test_quantize_rows_strided_input(dev):
    x = _x(40, 640, torch.bfloat16, seed=3)
    xs = x[:, 64:576]  # row stride 640, 16-byte aligned rows
    q, s = ops.int8_quantize_rows(xs.to(dev))
    qr, sr = R.quantize_rows_int8(xs)
    _equal(s, sr, "scales")
    _equal(q, qr, "codes")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 2, 5, 16, 17, 64, 300, 512])
@pytest.mark.parametrize("N,K", [(96, 64), (704, 512), (200, 192), (4096, 4096)])
def test_w8a8_linear_bit_exact(dev, dtype, M, N, K):
    """GEMV (M <= 16) and GEMM paths, K below / at / past one 128-k step,
    ragged N, bias on odd cases."""
    print(f"w8a8 linear M={M} N={N} K={K} {dtype}", flush=True)
    w = _w(N, K, seed=N + K)
    q, ws = R.quantize_int8(w, per_channel=True)
    x = _x(M, K, dtype, seed=M + 11)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(M)) * 0.1) if M % 2 else None
    y = ops.int8_linear_w8a8(x.to(dev), q.to(dev), ws.to(dev), bias.to(dev) if bias is not None else None)
    _equal(y, R.w8a8_linear(x, q, ws, bias), f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1, 512, 4096])
def test_w8a8_llama70b_mlp_rows(dev, M):
    """K=8192, N=28672, weights N(0,0.02) per-row int8 (bf16 scales, as
    quantize_int8 returns them for a bf16 weight), bf16 x N(0,1)."""
    K, N = 8192, 28672
    print(f"w8a8 llama70b mlp M={M}", flush=True)
    w = _w(N, K, seed=5).to(torch.bfloat16).to(dev)
    q, s = quantize_int8(w, per_channel=True)
    x = _x(M, K, torch.bfloat16, seed=M)
    y = ops.int8_linear_w8a8(x.to(dev), q, s).cpu()
    # every column of 64 seeded rows (the first and last included): the
    # oracle's exact integer sums run in float64 on the CPU
    g = torch.Generator().manual_seed(M + 1)
    rows = torch.unique(torch.cat([torch.randperm(M, generator=g)[:64], torch.tensor([0, M - 1])]))
    want = R.w8a8_linear(x[rows], q.cpu(), s.cpu())
    _equal(y[rows], want, f"M={M}")


def test_w8a8_close_to_w8a16(dev):
    """The activation rounding costs little: W8A8 stays within 1 % (relative
    Frobenius) of the W8A16 INT8 linear on the same per-row weights."""
    K, N, M = 4096, 2048, 256
    w = _w(N, K, seed=8).to(dev)
    q, s = quantize_int8(w, per_channel=True)
    x = _x(M, K, torch.bfloat16, seed=9).to(dev)
    a = ops.int8_linear_w8a8(x, q, s).float()
    b = ops.int8_linear(x, q, s, N).float()
    assert float((a - b).norm() / b.norm()) < 0.01


def test_w8a8_rejects_blockwise_scales_and_bad_k(dev):
    q = torch.zeros(64, 128, dtype=torch.int8, device=dev)
    x = torch.zeros(2, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):
        ops.int8_linear_w8a8(x, q, torch.ones(128, device=dev))  # blockwise scales count
    with pytest.raises(RuntimeError):
        ops.int8_linear_w8a8(x[:, :96], q.reshape(-1)[:64 * 96].reshape(64, 96), torch.ones(64, device=dev))


def test_w8a8_linear_module_and_custom_op(dev):
    torch.manual_seed(12)
    lin = torch.nn.Linear(512, 384).to(dev)
    m = W8A8Linear.from_linear(lin)
    x = torch.randn(3, 7, 512, device=dev, dtype=torch.bfloat16)
    y = m(x)
    assert y.shape == (3, 7, 384) and y.dtype == torch.bfloat16
    q, s = R.quantize_int8(lin.weight.detach().float().cpu(), per_channel=True)
    _equal(m.weight_quant, q, "weight codes")
    want = R.w8a8_linear(x.cpu().reshape(-1, 512), q, s, lin.bias.detach().cpu()).reshape(3, 7, 384)
    _equal(y, want, "module")
    torch.library.opcheck(torch_ops.int8_linear_w8a8, (x, m.weight_quant, m.weight_scales, m.bias))
