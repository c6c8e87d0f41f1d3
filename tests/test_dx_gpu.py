"""GPU parity of the NF4 dX backward (dX = dY . W_deq + ((dY * s) . B) . A):
HIP MFMA kernel through the C ABI vs the oracle's restatement of
_FusedNF4MatmulFunc.backward (dequant_matmul.py:338-351) plus the adapter's
input gradient (lora_layer.py:67 differentiated), on the same seeded inputs.
Tolerance rtol = atol = 1e-2 in dY's dtype.  The full-size Llama-3-8B cases
check every output element."""
import math

import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import ops
from rocm_qlora.quantization import quantize_int4, double_quantize

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2


def _inputs(N, K, M, dtype, seed, rank=64):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    dy = (torch.randn(M, N, generator=g) * 1e-2).to(dtype)
    a = torch.empty(rank, K)
    torch.nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
    b = torch.randn(N, rank, generator=g) * 0.01
    return w, dy, a, b


def _check(got, ref):
    got = got.cpu().float()
    ref = ref.float()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)])
def test_dx_llama3_shapes_bf16(dev, K, N):
    """Config: training backward dX, M=2048 bf16, dY ~ N(0, 1e-2), LoRA r=64 alpha=16."""
    M, rank = 2048, 64
    print(f"dx bf16 K={K} N={N} M={M}", flush=True)
    w, dy, a, b = _inputs(N, K, M, torch.bfloat16, seed=K + 3 * N)
    packed, absmax = quantize_int4(w.to(dev), 64)
    dx = ops.nf4_linear_dx(dy.to(dev), packed, absmax, K, 64, lora_a=a.to(dev), lora_b=b.to(dev),
                           scaling=16.0 / rank)
    ref = R.nf4_dx(dy, packed.cpu(), absmax.cpu(), N, K, a, b, 16.0 / rank, 64)
    _check(dx.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ["plain", "no_lora", "m1", "m5", "m17", "odd_m", "k_tail", "block128",
                                  "rank8", "rank16", "rank24", "rank96", "rank256", "bf16_lora", "strided_dy",
                                  "n64", "strided_b"])
def test_dx_variants(dev, dtype, case):
    N, K, M = 512, 640, 300
    M = {"m1": 1, "m5": 5, "m17": 17, "odd_m": 777}.get(case, M)
    K = {"k_tail": 320}.get(case, K)
    N = {"n64": 64}.get(case, N)
    rank = {"rank8": 8, "rank16": 16, "rank24": 24, "rank96": 96, "rank256": 256}.get(case, 64)
    bs = 128 if case == "block128" else 64
    print(f"dx variant {case} {dtype}", flush=True)
    w, dy, a, b = _inputs(N, K, M, dtype, seed=13, rank=rank)
    if case == "bf16_lora":
        a, b = a.to(dtype), b.to(dtype)
    packed, absmax = quantize_int4(w.to(dev), bs)
    dyd = dy.to(dev)
    if case == "strided_dy":
        big = torch.zeros(M, N + 64, dtype=dtype, device=dev)
        big[:, 32:32 + N] = dyd
        dyd = big[:, 32:32 + N]
    la, lb = (None, None) if case == "no_lora" else (a.to(dev), b.to(dev))
    if case == "strided_b":
        # rows of B 4 * (rank + 3) bytes apart: no 16-byte loads of them
        wide = torch.zeros(N, rank + 3, dtype=b.dtype, device=dev)
        wide[:, 1:1 + rank] = lb
        lb = wide[:, 1:1 + rank]
    dx = ops.nf4_linear_dx(dyd, packed, absmax, K, bs, lora_a=la, lora_b=lb, scaling=0.5)
    ref = R.nf4_dx(dy, packed.cpu(), absmax.cpu(), N, K,
                   None if la is None else a, None if lb is None else b, 0.5, bs)
    _check(dx, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N", [320, 384, 448])
@pytest.mark.parametrize("lora", [False, True])
def test_dx_k_step_tails(dev, dtype, N, lora):
    """Reduction over N = 5, 6, 7 k-steps: three calls in a row each equal
    the oracle and each other bit for bit (regression: a tail step read its
    activations before they had landed)."""
    K, M = 512, 300
    w, dy, a, b = _inputs(N, K, M, dtype, seed=N + 5, rank=16)
    packed, absmax = quantize_int4(w.to(dev), 64)
    kw = dict(lora_a=a.to(dev), lora_b=b.to(dev), scaling=2.0) if lora else {}
    dxs = [ops.nf4_linear_dx(dy.to(dev), packed, absmax, K, 64, **kw) for _ in range(3)]
    ref = R.nf4_dx(dy, packed.cpu(), absmax.cpu(), N, K, a if lora else None, b if lora else None, 2.0, 64)
    for dx in dxs:
        _check(dx, ref)
        assert torch.equal(dx.view(torch.int16), dxs[0].view(torch.int16))


def test_dx_double_quant(dev):
    N, K, M = 1024, 2048, 512
    w, dy, a, b = _inputs(N, K, M, torch.bfloat16, seed=29)
    st = double_quantize(w.to(dev), 64, 256)
    dx = ops.nf4_linear_dx(dy.to(dev), st.W_quant, None, K, 64, c2=st.c2, c2_scales=st.c2_scales,
                           lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.25)
    wf = R.double_dequantize(st.W_quant.cpu(), st.c2.cpu(), st.c2_scales.cpu(), (N, K), 64, 256, True)
    base = torch.mm(dy, wf.reshape(N, K).to(dy.dtype))
    g = (dy * 0.25) @ b.to(dy.dtype)
    ref = base + (g @ a.to(dy.dtype)).to(base.dtype)
    _check(dx, ref)


def test_dx_deterministic(dev):
    N, K, M = 2048, 2048, 1024
    w, dy, a, b = _inputs(N, K, M, torch.bfloat16, seed=31)
    packed, absmax = quantize_int4(w.to(dev), 64)
    args = (dy.to(dev), packed, absmax, K, 64)
    kw = dict(lora_a=a.to(dev), lora_b=b.to(dev), scaling=0.25)
    assert torch.equal(ops.nf4_linear_dx(*args, **kw), ops.nf4_linear_dx(*args, **kw))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dq", [False, True])
def test_dx_weight_operand_bit_exact(dev, dtype, dq):
    """One-hot dY rows pick single weight rows: dX[m, :] = RND(W[n_m, :]) must
    equal the reference's dequantized weight cast to dY's dtype bit for bit
    (quant_ops.py:144-148, double_quant.py:108-118): pins the transposing
    dequantizer's index mapping."""
    N, K, M = 256, 640, 300
    g = torch.Generator().manual_seed(37)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    ns = torch.randint(0, N, (M,), generator=g)
    ns[:64] = torch.arange(64) + 64
    dy = torch.zeros(M, N, dtype=dtype)
    dy[torch.arange(M), ns] = 1.0
    if dq:
        st = double_quantize(w.to(dev), 64, 256)
        dx = ops.nf4_linear_dx(dy.to(dev), st.W_quant, None, K, 64, c2=st.c2, c2_scales=st.c2_scales)
        wf = R.double_dequantize(st.W_quant.cpu(), st.c2.cpu(), st.c2_scales.cpu(), (N, K), 64, 256, True)
    else:
        packed, absmax = quantize_int4(w.to(dev), 64)
        dx = ops.nf4_linear_dx(dy.to(dev), packed, absmax, K, 64)
        wf = R.dequantize_int4(packed.cpu(), absmax.cpu(), 64)[:N * K]
    ref = wf.reshape(N, K).to(dtype)[ns]
    assert torch.equal(dx.cpu().view(torch.int16), ref.contiguous().view(torch.int16))


def _dx_call(dev, dy, packed, scales, K, block, ws_bytes, c2=None, a=None, b=None, rank=0, scaling=0.25):
    """rq_nf4_linear_dx through the C ABI with a workspace of ws_bytes."""
    from rocm_qlora import _native as nat
    M, N = dy.shape
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    dx = torch.empty(M, K, dtype=dy.dtype, device=dev)
    nat.call("rq_nf4_linear_dx", dy.data_ptr(), nat.dtype_code(dy.dtype), M, N, N, packed.data_ptr(), K, block,
             scales.data_ptr(), nat.dtype_code(scales.dtype), nat.ptr(c2), nat.C2_FP8_E4M3FNUZ, 256,
             nat.ptr(a), nat.ptr(b), rank, nat.dtype_code(a.dtype) if a is not None else 0, rank, scaling,
             None, 0, 1.0, dx.data_ptr(), K, ws.data_ptr(), ws_bytes, nat.stream_handle(dev))
    torch.cuda.synchronize()
    return dx


@pytest.mark.parametrize("N,K,case", [(512, 4096, "f32"), (512, 4096, "bf16"), (512, 4096, "dq"),
                                      (512, 64, "f32"), (256, 64, "bf16"), (512, 1024, "lora"),
                                      (512, 1024, "lora64"), (256, 1024, "lora12"), (256, 1024, "lora96")])
def test_dx_transposed_scales_match_direct(dev, N, K, case):
    """With room in the workspace a launch before the dX kernel decodes and
    transposes the scales ([blocks][rows] fp32, a step's scales contiguous)
    and, with LoRA, writes RND(A)^T as 16-bit rows (the epilogue's operand,
    read into registers during the kernel's prologue for ranks up to 64 that
    are multiples of 8); with less room, the scales transposed and A read in
    place; with less still, the absmax (or c2 codes and their scales)
    directly.  All give the same bits: fp32 and bf16 absmax, double
    quantization, one block per row (K == block size, where the two rows a
    thread dequantizes have adjacent scales), and LoRA ranks 16, 64, 12 and
    96."""
    import ctypes
    from rocm_qlora import _native as nat
    M = 300
    print(f"dx transposed scales N={N} K={K} {case}", flush=True)
    g = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    dy = (torch.randn(M, N, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    c2 = None
    if case == "dq":
        st = double_quantize(w.to(dev), 64, 256)
        packed, scales, c2 = st.W_quant.reshape(-1), st.c2_scales, st.c2.reshape(-1).view(torch.uint8)
    else:
        packed, scales = quantize_int4(w.to(dev).to(torch.bfloat16 if case == "bf16" else torch.float32), 64)
    rank = {"lora": 16, "lora64": 64, "lora12": 12, "lora96": 96}.get(case, 0)
    a = (torch.randn(rank, K, generator=g) * 0.05).to(dev) if rank else None
    b = (torch.randn(N, rank, generator=g) * 0.05).to(dev) if rank else None
    nb = ctypes.c_int64(0)
    nat.call("rq_nf4_linear_dx_workspace_size", nat.dtype_code(dy.dtype), M, N, K, rank, ctypes.byref(nb))
    # the workspace ends with the transposed scales, then RND(A)^T
    st_bytes = (N * (K // 64) * 4 + 255) // 256 * 256
    at_bytes = (K * ((rank + 15) // 16 * 16) * 2 + 255) // 256 * 256 if rank else 0
    assert nb.value >= st_bytes + at_bytes
    full = _dx_call(dev, dy, packed, scales, K, 64, nb.value, c2, a, b, rank)
    if rank:
        scales_only = _dx_call(dev, dy, packed, scales, K, 64, nb.value - at_bytes, c2, a, b, rank)
        assert torch.equal(full.view(torch.int16), scales_only.view(torch.int16))
    direct = _dx_call(dev, dy, packed, scales, K, 64, nb.value - at_bytes - st_bytes, c2, a, b, rank)
    assert torch.equal(full.view(torch.int16), direct.view(torch.int16))
    if case in ("f32", "bf16"):
        ref = R.nf4_dx(dy.cpu(), packed.cpu(), scales.cpu(), N, K, None, None, 0.0, 64)
        _check(full.cpu(), ref)
    if rank:
        ref = R.nf4_dx(dy.cpu(), packed.cpu(), scales.cpu(), N, K, a.cpu(), b.cpu(), 0.25, 64)
        _check(full.cpu(), ref)


def test_dx_down_deterministic(dev):
    """At the Llama-3-8B down shape (dX output 14336 columns, reduction over
    4096: the transposed scales span 224 blocks per row) three calls give the
    same bits, and the output is within rtol = atol = 1e-2 of the oracle."""
    N, K, M, rank = 4096, 14336, 2048, 64
    print("dx down deterministic", flush=True)
    w, dy, a, b = _inputs(N, K, M, torch.bfloat16, seed=77)
    packed, absmax = quantize_int4(w.to(dev), 64)
    args = (dy.to(dev), packed, absmax, K, 64)
    kw = dict(lora_a=a.to(dev), lora_b=b.to(dev), scaling=16.0 / rank)
    outs = [ops.nf4_linear_dx(*args, **kw) for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = R.nf4_dx(dy, packed.cpu(), absmax.cpu(), N, K, a, b, 16.0 / rank, 64)
    _check(outs[0].cpu(), ref)
