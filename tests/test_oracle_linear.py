"""Pins the oracle's linear compositions (oracle/qlora_ref.py:
quant_linear_forward, lora_forward, nf4_lora_linear, nf4_dx, int8_linear,
fp8_linear, lora_linear_grads) against closed forms and float64 finite
differences, chosen so that a dropped term, a wrong sign, a transposed
operand or a misplaced scaling fails one of them.  CPU only."""
import math

import pytest
import torch

from oracle import qlora_ref as R


def _lora(N, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.empty(r, K)
    torch.nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
    b = torch.randn(N, r, generator=g) * 0.1
    return a, b


def test_one_hot_rows_pick_weight_columns_bias_and_adapter():
    """x = e_k: base = W[:, k] + bias; the adapter adds s * B @ A[:, k]."""
    N, K, r, s = 96, 128, 8, 0.75
    g = torch.Generator().manual_seed(1)
    w = torch.randn(N, K, generator=g) * 0.02
    packed, absmax = R.quantize_int4(w, 64)
    wf = R.dequantize_int4(packed, absmax, 64)[:N * K].view(N, K)
    bias = torch.randn(N, generator=g)
    a, b = _lora(N, K, r, 2)
    ks = torch.tensor([0, 5, 127])
    x = torch.zeros(3, K)
    x[torch.arange(3), ks] = 1.0
    base = R.quant_linear_forward(x, wf.reshape(-1), bias, N, K)
    assert torch.equal(base, (wf[:, ks] + bias[:, None]).T)
    y = R.nf4_lora_linear(x, packed, absmax, bias, a, b, s, N, 64)
    expect = base + s * (b @ a[:, ks]).T
    assert torch.allclose(y, expect, rtol=1e-6, atol=1e-7)
    assert torch.equal(R.lora_forward(x, base, a, torch.zeros_like(b), s), base)


def test_nf4_dx_is_the_transposed_product():
    """dX[m, k] = sum_n dY[m, n] W[n, k] + s sum_n dY[m, n] (B A)[n, k], in float64."""
    N, K, r, s = 64, 192, 4, 1.5
    g = torch.Generator().manual_seed(3)
    w = torch.randn(N, K, generator=g) * 0.02
    packed, absmax = R.quantize_int4(w, 64)
    wf = R.dequantize_int4(packed, absmax, 64)[:N * K].view(N, K).double()
    a, b = _lora(N, K, r, 4)
    dy = torch.randn(5, N, generator=g)
    dx = R.nf4_dx(dy, packed, absmax, N, K, a, b, s, 64).double()
    expect = dy.double() @ wf + s * dy.double() @ (b.double() @ a.double())
    assert torch.allclose(dx, expect, rtol=1e-5, atol=1e-6)


def test_nf4_dx_matches_the_autograd_grads():
    """nf4_dx (the dX kernel's restatement) against the dX that
    lora_linear_grads, pinned by central differences below, gives for the
    same quantized layer: float64 operands, so both are the exact product
    up to summation order; an nf4_dx with a dropped LoRA term or B and A
    swapped fails here."""
    N, K, r, M, s = 48, 128, 8, 7, 0.75
    g = torch.Generator().manual_seed(13)
    w = torch.randn(N, K, generator=g) * 0.02
    packed, absmax = R.quantize_int4(w, 64)
    wq = R.dequantize_int4(packed, absmax, 64)[:N * K]
    a, b = _lora(N, K, r, 6)
    a, b = a.double(), b.double()
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    dy = torch.randn(M, N, generator=g, dtype=torch.float64)
    _, dx_auto, _, _ = R.lora_linear_grads(x, wq.double(), None, a, b, s, dy)
    dx = R.nf4_dx(dy, packed, absmax, N, K, a, b, s, 64)
    assert dx.dtype == torch.float64
    assert torch.allclose(dx, dx_auto, rtol=1e-12, atol=1e-14)
    # the base and the adapter term are both present (neither is negligible)
    base_only = R.nf4_dx(dy, packed, absmax, N, K, None, None, 0.0, 64)
    assert (dx - base_only).abs().max() > 1e-3 * dx.abs().max()


def test_lora_grads_match_finite_differences():
    """Gradients of L = sum(dY * y) for y = x W^T + b + s (x A^T) B^T, by
    central differences in float64 on a tiny case."""
    N, K, r, M, s = 6, 8, 3, 2, 0.5
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    w = torch.randn(N, K, generator=g, dtype=torch.float64) * 0.3
    bias = torch.randn(N, generator=g, dtype=torch.float64)
    a = torch.randn(r, K, generator=g, dtype=torch.float64)
    b = torch.randn(N, r, generator=g, dtype=torch.float64)
    dy = torch.randn(M, N, generator=g, dtype=torch.float64)
    _, dx, da, db = R.lora_linear_grads(x, w.reshape(-1), bias, a, b, s, dy)

    def loss(xx, aa, bb):
        y = xx @ w.T + bias + s * (xx @ aa.T) @ bb.T
        return float((dy * y).sum())

    h = 1e-6
    for t, grad, which in ((x, dx, 0), (a, da, 1), (b, db, 2)):
        num = torch.zeros_like(t)
        for i in range(t.numel()):
            tp, tm = t.clone(), t.clone()
            tp.view(-1)[i] += h
            tm.view(-1)[i] -= h
            args_p = [x, a, b]
            args_m = [x, a, b]
            args_p[which], args_m[which] = tp, tm
            num.view(-1)[i] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        assert torch.allclose(grad.double(), num, rtol=1e-6, atol=1e-8), which


def test_int8_linear_per_row_scales():
    """Row-absmax INT8: y = x (q * s[:, None])^T; a row scale multiplies its output column."""
    g = torch.Generator().manual_seed(6)
    w = torch.randn(40, 64, generator=g) * 0.02
    q, s = R.quantize_int8(w, per_channel=True)
    x = torch.randn(3, 64, generator=g)
    y = R.int8_linear(x, q, s)
    assert torch.allclose(y.double(), x.double() @ (q.double() * s.double()[:, None]).T, rtol=1e-5, atol=1e-7)
    y2 = R.int8_linear(x, q, s * 2)
    assert torch.allclose(y2, 2 * y, rtol=1e-6, atol=1e-7)


def test_fp8_linear_is_decode_then_matmul_with_both_scales():
    """y = (x8 * sx) @ (w8 * sw)^T + bias, the scales applied once each."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, 32, generator=g).to(torch.bfloat16)
    w = (torch.randn(16, 32, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(16, generator=g).to(torch.bfloat16)
    y = R.fp8_linear(x, w, bias)
    x8, sx = R.fp8_quantize_tensor(x)
    w8, sw = R.fp8_quantize_tensor(w)
    core = (x8.double() * float(sx)) @ (w8.double() * float(sw)).T
    assert torch.allclose(y.double(), (core.to(torch.bfloat16) + bias).double(), rtol=0, atol=0)
    # and close to the unquantized product (e4m3 keeps ~3 bits)
    assert torch.allclose(y.float(), (x.float() @ w.float().T + bias.float()), rtol=0.15, atol=0.15)


def test_lora_grads_with_dropout_mask():
    """The oracle's LoRA dropout (lora_layer.py:67, drop(x) = x * mask / (1 - p)):
    in float64 the gradients match central differences of the loss with the
    dropped input; an all-kept mask at p = 0 gives the no-dropout results bit
    for bit; in bf16 the dropped input is x * scale rounded once."""
    N, K, r, M, s, p = 6, 8, 3, 2, 0.5, 0.25
    g = torch.Generator().manual_seed(9)
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    w = torch.randn(N, K, generator=g, dtype=torch.float64) * 0.3
    bias = torch.randn(N, generator=g, dtype=torch.float64)
    a = torch.randn(r, K, generator=g, dtype=torch.float64)
    b = torch.randn(N, r, generator=g, dtype=torch.float64)
    dy = torch.randn(M, N, generator=g, dtype=torch.float64)
    mask = torch.rand(M, K, generator=g) > p
    y, dx, da, db = R.lora_linear_grads(x, w.reshape(-1), bias, a, b, s, dy, dropout_mask=mask, dropout_p=p)
    keep = mask.to(torch.float64) / (1 - p)

    def fwd(xx, aa, bb):
        return xx @ w.T + bias + s * ((xx * keep) @ aa.T) @ bb.T

    assert torch.allclose(y, fwd(x, a, b), rtol=1e-12, atol=1e-12)
    h = 1e-6
    for t, grad, which in ((x, dx, 0), (a, da, 1), (b, db, 2)):
        num = torch.zeros_like(t)
        for i in range(t.numel()):
            tp, tm = t.clone(), t.clone()
            tp.view(-1)[i] += h
            tm.view(-1)[i] -= h
            ap, am = [x, a, b], [x, a, b]
            ap[which], am[which] = tp, tm
            num.view(-1)[i] = (float((dy * fwd(*ap)).sum()) - float((dy * fwd(*am)).sum())) / (2 * h)
        assert torch.allclose(grad, num, rtol=1e-6, atol=1e-6), which
    ones = torch.ones(M, K, dtype=torch.bool)
    got = R.lora_linear_grads(x, w.reshape(-1), bias, a, b, s, dy, dropout_mask=ones, dropout_p=0.0)
    want = R.lora_linear_grads(x, w.reshape(-1), bias, a, b, s, dy)
    assert all(torch.equal(u, v) for u, v in zip(got, want))
    xb = torch.randn(64, generator=g).to(torch.bfloat16)
    mk = torch.rand(64, generator=g) > 0.1
    dropped = R._DropoutWithMask.apply(xb, mk, 1.0 / 0.9)
    assert torch.equal(dropped, (xb.float() * mk.float() * (1.0 / 0.9)).to(torch.bfloat16))


def _dyadic(shape, g, scale_pow):
    """Integers in [-8, 8] times 2^-scale_pow: products and rank sums stay
    exact in fp32, so the delta does not depend on the summation order."""
    return torch.randint(-8, 9, shape, generator=g).to(torch.float32) * 2.0 ** -scale_pow


def test_merge_and_export_restatements_pinned():
    """merge_lora_weight rounds W + d once to fp16; export_dequant_layer
    rounds W and d to fp16 and adds them (float64 sum of two fp16 values,
    rounded once).  Zero adapters give the dequantized weight cast to fp16."""
    g = torch.Generator().manual_seed(81)
    N, K, r, s = 24, 128, 5, 2.0
    w = torch.randn(N * K, generator=g) * 0.02
    a, b = _dyadic((r, K), g, 6), _dyadic((N, r), g, 7)
    d64 = (b.double() @ a.double()) * s                       # exact, as is the fp32 product
    want_merge = (w.double().reshape(N, K) + d64).float().to(torch.float16)
    assert torch.equal(R.merge_lora_weight(w, a, b, s, N, K).view(torch.int16), want_merge.view(torch.int16))
    w16 = w.reshape(N, K).to(torch.float16)
    want_export = (w16.double() + d64.to(torch.float16).double()).to(torch.float16)
    assert torch.equal(R.export_dequant_layer(w, a, b, s, N, K).view(torch.int16), want_export.view(torch.int16))
    z = torch.zeros(N, r)
    for fn in (R.merge_lora_weight, R.export_dequant_layer):
        assert torch.equal(fn(w, a, z, s, N, K), w16)


def test_w8a8_activation_codes_are_the_per_row_recipe():
    """quantize_rows_int8 is quantize_int8(per_channel=True) on fp32 rows
    (that function is pinned against the C restatement)."""
    g = torch.Generator().manual_seed(51)
    x = (torch.randn(7, 96, generator=g) * 3).to(torch.bfloat16)
    x[2] = 0
    q, s = R.quantize_rows_int8(x)
    q2, s2 = R.quantize_int8(x.float(), per_channel=True)
    assert torch.equal(q, q2) and torch.equal(s, s2.reshape(-1))
    assert float(s[2]) == pytest.approx(1e-12) and int(q[2].abs().max()) == 0
    assert int(q.abs().max()) == 127


def test_w8a8_integer_sum_brute_force():
    """The integer core of w8a8_linear against a Python-int brute force, and
    the scales applied to it in fp32, each rounding once."""
    g = torch.Generator().manual_seed(52)
    x = torch.randn(3, 64, generator=g).to(torch.bfloat16)
    q = torch.randint(-127, 128, (5, 64), generator=g).to(torch.int8)
    ws = torch.rand(5, generator=g) * 0.01 + 1e-3
    qx, sx = R.quantize_rows_int8(x)
    y = R.w8a8_linear(x, q, ws)
    for m in range(3):
        for n in range(5):
            acc = sum(int(qx[m, k]) * int(q[n, k]) for k in range(64))
            want = torch.tensor(float(acc), dtype=torch.float32) * sx[m] * ws[n]
            assert y[m, n] == want.to(torch.bfloat16)


def test_w8a8_power_of_two_scales_equal_the_w8a16_product():
    """Rows of x with absmax 127 * 2^-j (scales 2^-j, codes exact) and weights
    with power-of-two row scales: every step is exact, so W8A8 equals the
    reference's INT8 linear (x times dequantized weights) bit for bit."""
    g = torch.Generator().manual_seed(53)
    M, N, K = 4, 6, 128
    kx = torch.randint(-127, 128, (M, K), generator=g)
    kx[:, 5] = 127
    x = (kx.double() * 2.0 ** -torch.arange(3, 3 + M).double()[:, None]).to(torch.bfloat16)
    q = torch.randint(-127, 128, (N, K), generator=g).to(torch.int8)
    ws = 2.0 ** -torch.randint(4, 9, (N,), generator=g).float()
    bias = (torch.randint(-64, 64, (N,), generator=g).float() / 8).to(torch.bfloat16)
    y = R.w8a8_linear(x, q, ws, bias)
    want = (R.int8_linear(x.float(), q, ws)).to(torch.bfloat16) + bias
    assert torch.equal(y, want)
    exact = (x.double() @ (q.double() * ws.double()[:, None]).T).to(torch.bfloat16) + bias
    assert torch.equal(y, exact)


def test_w8a8_close_to_float64_of_its_codes():
    """General scales: within one bf16 ulp of the float64 product of the
    decoded codes (three fp32 roundings, then one to bf16)."""
    g = torch.Generator().manual_seed(54)
    x = torch.randn(9, 256, generator=g).to(torch.bfloat16)
    w = torch.randn(33, 256, generator=g) * 0.02
    q, ws = R.quantize_int8(w, per_channel=True)
    y = R.w8a8_linear(x, q, ws)
    qx, sx = R.quantize_rows_int8(x)
    exact = (qx.double() * sx.double()[:, None]) @ (q.double() * ws.double()[:, None]).T
    ulp = (exact.abs().to(torch.bfloat16).double().abs() * 2.0 ** -7).clamp_min(2.0 ** -133)
    assert bool(((y.double() - exact).abs() <= ulp).all())
    # and close to the unquantized product
    assert torch.allclose(y.float(), x.float() @ w.T, rtol=0.05, atol=0.05)
