"""GPU parity of the NF4 prefill/training GEMM (M > 16 activation rows): HIP
MFMA kernel through the C ABI vs the oracle's restatement of
QuantLinear.forward + LoRALinear.forward (quant_linear.py:182-197,
lora_layer.py:60-70) on the same seeded inputs.  Tolerance rtol = atol = 1e-2
in the activation dtype.  The full-size Llama-3-8B cases check every output
element against the oracle."""
import math

import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import ops
from rocm_qlora.quantization import quantize_int4, double_quantize

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2


def _inputs(N, K, M, dtype, seed, rank=64, bias=False):
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


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)])
def test_gemm_llama3_shapes_bf16(dev, K, N):
    """Config: prefill dequant-GEMM, M=2048 bf16 tokens, LoRA r=64 alpha=16 fused."""
    M, rank = 2048, 64
    print(f"gemm bf16 K={K} N={N} M={M}", flush=True)
    w, x, a, b, _ = _inputs(N, K, M, torch.bfloat16, seed=K + N)
    packed, absmax = quantize_int4(w.to(dev), 64)
    y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=a.to(dev), lora_b=b.to(dev),
                       scaling=16.0 / rank)
    ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), None, a, b, 16.0 / rank, N, 64)
    _check(y.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ["plain", "bias", "odd_n", "odd_m", "m17", "block128", "strided_x",
                                  "dropout_x", "no_lora", "k64", "k320", "rank8", "rank12", "rank16", "rank24",
                                  "rank96", "rank256",
                                  "bf16_lora", "tiles8", "strided_b"])
def test_gemm_variants(dev, dtype, case):
    N, K, M = 640, 512, 300
    N = {"odd_n": 1000, "tiles8": 512}.get(case, N)
    M = {"odd_m": 777, "m17": 17, "tiles8": 512}.get(case, M)
    K = {"k64": 64, "k320": 320}.get(case, K)
    rank = {"rank8": 8, "rank12": 12, "rank16": 16, "rank24": 24, "rank96": 96, "rank256": 256}.get(case, 64)
    bs = 128 if case == "block128" else 64
    print(f"gemm variant {case} {dtype}", flush=True)
    w, x, a, b, bvec = _inputs(N, K, M, dtype, seed=11, rank=rank, bias=(case == "bias"))
    if case == "bf16_lora":
        a, b = a.to(dtype), b.to(dtype)
    packed, absmax = quantize_int4(w.to(dev), bs)
    xd = x.to(dev)
    xl = None
    if case == "strided_x":
        big = torch.zeros(M, K + 72, dtype=dtype, device=dev)
        big[:, 40:40 + K] = xd
        xd = big[:, 40:40 + K]
    if case == "dropout_x":
        xl = (x * (torch.rand(x.shape, generator=torch.Generator().manual_seed(3)) > 0.3)).to(dtype)
    la, lb = (None, None) if case == "no_lora" else (a.to(dev), b.to(dev))
    if case == "strided_b":
        # rows of B 4 * (rank + 3) bytes apart: no 16-byte loads of them
        wide = torch.zeros(N, rank + 3, dtype=b.dtype, device=dev)
        wide[:, 1:1 + rank] = lb
        lb = wide[:, 1:1 + rank]
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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [320, 384, 448])
@pytest.mark.parametrize("lora", [False, True])
def test_gemm_k_step_tails(dev, dtype, K, lora):
    """K / 64 = 5, 6, 7 k-steps (1, 2, 3 past the loop's groups of four):
    three calls in a row each equal the oracle and each other bit for bit
    (a tail step once read its activations before they had landed, which
    only a repeated call exposed)."""
    N, M = 384, 300
    w, x, a, b, _ = _inputs(N, K, M, dtype, seed=K + 1, rank=16)
    packed, absmax = quantize_int4(w.to(dev), 64)
    kw = dict(lora_a=a.to(dev), lora_b=b.to(dev), scaling=2.0) if lora else {}
    ys = [ops.nf4_linear(x.to(dev), packed, absmax, N, 64, **kw) for _ in range(3)]
    ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), None, a if lora else None, b if lora else None, 2.0,
                            N, 64)
    for y in ys:
        _check(y, ref)
        assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))


def test_gemm_double_quant(dev):
    N, K, M = 1024, 2048, 512
    w, x, a, b, _ = _inputs(N, K, M, torch.bfloat16, seed=23)
    st = double_quantize(w.to(dev), 64, 256)
    y = ops.nf4_linear(x.to(dev), st.W_quant, None, N, 64, c2=st.c2, c2_scales=st.c2_scales,
                       blocksize_2=256, use_fp8_c2=True, lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.25)
    wf = R.double_dequantize(st.W_quant.cpu(), st.c2.cpu(), st.c2_scales.cpu(), (N, K), 64, 256, True)
    base = R.quant_linear_forward(x, wf.reshape(-1), None, N, K)
    ref = R.lora_forward(x, base, a, b, 0.25)
    _check(y, ref)


def test_gemm_deterministic(dev):
    N, K, M = 2048, 2048, 1024
    w, x, a, b, _ = _inputs(N, K, M, torch.bfloat16, seed=9)
    packed, absmax = quantize_int4(w.to(dev), 64)
    args = (x.to(dev), packed, absmax, N, 64)
    kw = dict(lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.25)
    y1 = ops.nf4_linear(*args, **kw)
    y2 = ops.nf4_linear(*args, **kw)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dq", [False, True])
def test_gemm_weight_operand_bit_exact(dev, dtype, dq):
    """One-hot activation rows pick single weights: y[m, n] = RND(W[n, k_m])
    must equal the reference's dequantized weight cast to x's dtype bit for
    bit (quant_ops.py:144-148, quant_linear.py:191-193; double_quant.py:108-118).
    300 rows cover two 256-row tiles and every k position mod 64."""
    N, K, M = 384, 1024, 300
    g = torch.Generator().manual_seed(19)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    ks = torch.randint(0, K, (M,), generator=g)
    ks[:64] = torch.arange(64) + 128
    x = torch.zeros(M, K, dtype=dtype)
    x[torch.arange(M), ks] = 1.0
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


def test_gemm_k_splits_and_shared_workspace(dev, sync_ready):
    """Shapes with few tiles run as K splits whose last split of each tile sums
    the others (tile counters in the workspace's zeroed synchronization area).
    Calls of split GEMMs, an unsplit GEMM and a decode GEMV with in-launch
    LoRA share one workspace in a row; each matches the oracle, repeated
    calls give the same bits, and the area is zero again afterwards."""
    K, rank = 2048, 16
    cases = [(1024, 512), (768, 2048), (2048, 2048), (1024, 3)]
    layers = {}
    for N, M in cases:
        if N not in layers:
            w, _, a, b, _ = _inputs(N, K, 1, torch.bfloat16, seed=N, rank=rank)
            packed, absmax = quantize_int4(w.to(dev), 64)
            layers[N] = (packed, absmax, a, b)
    for rep in range(2):
        for i, (N, M) in enumerate(cases):
            packed, absmax, a, b = layers[N]
            x = _inputs(N, K, M, torch.bfloat16, seed=100 + i)[1]
            print(f"k-split case N={N} M={M} rep={rep}", flush=True)
            y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.5)
            y2 = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.5)
            assert torch.equal(y, y2)
            ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), None, a, b, 0.5, N, 64)
            _check(y, ref)
    torch.cuda.synchronize(dev)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    assert sync_ready(ops._LINEAR_WS[key])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank,lora_dt", [(64, torch.float32), (24, torch.float32), (64, torch.bfloat16)])
def test_gemm_lora_operand_paths_match(dev, dtype, rank, lora_dt):
    """The epilogue's LoRA operands are read into registers during the
    kernel's prologue when B's rows allow 16-byte loads (rank <= 64, a
    multiple of 8), and staged from memory after the main loop otherwise.
    The same values as a strided view of B (rows not 16-byte aligned) take
    the second path and give the same bits."""
    N, K, M = 640, 512, 300
    print(f"gemm lora operand paths rank={rank} {lora_dt} {dtype}", flush=True)
    w, x, a, b, _ = _inputs(N, K, M, dtype, seed=19, rank=rank)
    packed, absmax = quantize_int4(w.to(dev), 64)
    a, b = a.to(lora_dt).to(dev), b.to(lora_dt).to(dev)
    wide = torch.zeros(N, rank + 3, dtype=b.dtype, device=dev)
    wide[:, 1:1 + rank] = b
    y_regs = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=a, lora_b=b, scaling=0.5)
    y_mem = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=a, lora_b=wide[:, 1:1 + rank], scaling=0.5)
    assert torch.equal(y_regs.view(torch.int16), y_mem.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_output_strides(dev, dtype):
    """The epilogue stores whole tiles through LDS as 128-byte row pieces
    when the output rows are 16-byte aligned, four-output runs when they are
    8-byte aligned, and single values otherwise.  Output row strides N, N + 4
    and N + 3 (through the C ABI) give the same bits in the N columns and
    leave the padding as it was; the forward at N = 1001 (a partial column
    tile, rows not 8-byte aligned) matches the oracle."""
    import ctypes
    from rocm_qlora import _native as nat
    M, K, N, rank = 300, 512, 512, 16
    print(f"gemm output strides {dtype}", flush=True)
    w, x, a, b, bvec = _inputs(N, K, M, dtype, seed=23, rank=rank, bias=True)
    packed, absmax = quantize_int4(w.to(dev), 64)
    xd, ad, bd, biasd = x.to(dev), a.to(dev), b.to(dev), bvec.to(dtype).to(dev)
    nb = ctypes.c_int64(0)
    nat.call("rq_nf4_linear_workspace_size", nat.dtype_code(dtype), M, K, N, rank, ctypes.byref(nb))
    outs = []
    for ld in (N, N + 4, N + 3):
        ws = torch.zeros(nb.value, dtype=torch.uint8, device=dev)
        y = torch.full((M, ld), -7.0, dtype=dtype, device=dev)
        nat.call("rq_nf4_linear", xd.data_ptr(), nat.dtype_code(dtype), M, K, K,
                 packed.data_ptr(), N, 64, absmax.data_ptr(), nat.dtype_code(absmax.dtype),
                 None, nat.C2_FP8_E4M3FNUZ, 256, biasd.data_ptr(), nat.dtype_code(biasd.dtype),
                 xd.data_ptr(), K, ad.data_ptr(), bd.data_ptr(), rank, nat.dtype_code(ad.dtype), rank, 0.5,
                 y.data_ptr(), ld, ws.data_ptr(), ws.numel(), nat.stream_handle(dev))
        torch.cuda.synchronize(dev)
        assert bool((y[:, N:] == -7.0).all()), f"ldy={ld}: padding written"
        outs.append(y[:, :N].contiguous())
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    wf = R.dequantize_int4(packed.cpu(), absmax.cpu(), 64)
    ref = R.quant_linear_forward(x, wf, bvec, N, K) + \
        (x @ a.to(dtype).T @ b.to(dtype).T * 0.5).to(dtype)
    _check(outs[0], ref)
    N2 = 1001
    w2, x2, a2, b2, _ = _inputs(N2, K, M, dtype, seed=29, rank=rank)
    p2, s2 = quantize_int4(w2.to(dev), 64)
    y2 = ops.nf4_linear(x2.to(dev), p2, s2, N2, 64, lora_a=a2.to(dev), lora_b=b2.to(dev), scaling=0.5)
    ref2 = R.quant_linear_forward(x2, R.dequantize_int4(p2.cpu(), s2.cpu(), 64), None, N2, K) + \
        (x2 @ a2.to(dtype).T @ b2.to(dtype).T * 0.5).to(dtype)
    _check(y2, ref2)
