"""The oracle's PagedAdamW step (oracle.qlora_ref.paged_adamw_step,
optim/paged_adamw.py:84-113) pinned against torch.optim.AdamW, zero and
constant gradients; its restatement with the GPU kernels' roundings
(paged_adamw_step_device) and the exact fp32 fused multiply-add it uses
(fma32, against rational arithmetic); and the optimizer's host logic
(construction, state layout, statistics) without a GPU."""
from fractions import Fraction

import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora.optim import PagedAdamW
from rocm_qlora.optim.paged_adamw import ADAMW_CHUNK


def _tensors(seed, shapes):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g) * 0.05 for s in shapes]


def test_oracle_matches_torch_adamw():
    """Same update rule as torch.optim.AdamW (decoupled decay, bias
    corrections, eps outside the square root); torch's own implementation
    rounds its first moment through lerp_, so within a few ulps after five
    steps; a wrong bias correction, decay or eps placement moves p by far
    more (lr = 1e-2 per step)."""
    shapes = [(16, 64), (64, 16), (7,)]
    ps = _tensors(1, shapes)
    qs = [p.clone().requires_grad_(True) for p in ps]
    opt = torch.optim.AdamW(qs, lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, foreach=False)
    ms = [torch.zeros_like(p) for p in ps]
    vs = [torch.zeros_like(p) for p in ps]
    for t in range(1, 6):
        gs = _tensors(10 + t, shapes)
        for q, g in zip(qs, gs):
            q.grad = g.clone()
        opt.step()
        R.paged_adamw_step(ps, gs, ms, vs, [t] * 3, lr=1e-2, weight_decay=0.01)
    for p, q in zip(ps, qs):  # a few fp32 ulps of |p| ~ 0.05
        assert float((p - q.detach()).abs().max()) <= 5e-8
    for m, q in zip(ms, qs):
        assert float((m - opt.state[q]["exp_avg"]).abs().max()) <= 2e-8  # |m| < 0.04


def test_oracle_zero_gradient_is_pure_decay():
    p = _tensors(2, [(1000,)])[0]
    want = p.clone()
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    for t in range(1, 4):
        R.paged_adamw_step([p], [torch.zeros_like(p)], [m], [v], [t], lr=1e-3, weight_decay=0.1)
        want = want * torch.tensor(1 - 1e-3 * 0.1, dtype=torch.float32)
    assert torch.equal(p, want)
    assert not m.any() and not v.any()


def test_oracle_constant_gradient_closed_form():
    """With a constant gradient the bias-corrected moments are g and g^2, so
    each step moves p by lr * g / (|g| + eps) (no decay)."""
    g = torch.tensor([1e-3, -2e-2, 0.5, -3.0])
    p = torch.zeros(4)
    m, v = torch.zeros(4), torch.zeros(4)
    for t in range(1, 11):
        R.paged_adamw_step([p], [g], [m], [v], [t], lr=1e-2, eps=1e-8, weight_decay=0.0)
    want = -10 * 1e-2 * g.double() / (g.double().abs() + 1e-8)
    assert torch.allclose(p.double(), want, rtol=1e-5, atol=0)


def test_oracle_exact_sqrt_variant():
    """exact_sqrt changes only the square root: same moments, parameters
    within an ulp of the update per step, and its root is the float64 root
    rounded once."""
    shapes = [(4096,)]
    p1, p2 = _tensors(4, shapes)[0], None
    p2 = p1.clone()
    m1, v1, m2, v2 = (torch.zeros(4096) for _ in range(4))
    for t in range(1, 4):
        g = _tensors(20 + t, shapes)[0] * 0.01
        R.paged_adamw_step([p1], [g], [m1], [v1], [t], lr=1e-3)
        R.paged_adamw_step([p2], [g], [m2], [v2], [t], lr=1e-3, exact_sqrt=True)
    assert torch.equal(m1, m2) and torch.equal(v1, v2)
    assert float((p1 - p2).abs().max()) <= 3 * (2 ** -23) * 1e-3 * 4
    r = v2.double().sqrt().float().double()
    assert bool(((r - v2.double().sqrt()).abs() <= (r.abs() * 2.0 ** -24)).all())


def _rn32(x: Fraction) -> float:
    """x rounded to the nearest fp32, ties to even, decided in rationals."""
    f = torch.tensor(float(x), dtype=torch.float64).float()
    cands = [torch.nextafter(f, torch.tensor(-float("inf"))), f, torch.nextafter(f, torch.tensor(float("inf")))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - x), int(c.view(torch.int32)) & 1))
    return float(best)


def test_fma32_against_rationals():
    """fma32 equals a * b + c rounded once, in exact rationals, on random
    triples over wide exponent ranges (cancellation included) and on sums
    whose float64 rounding lands on an fp32 midpoint -- where rounding the
    float64 sum again gives the wrong neighbour."""
    g = torch.Generator().manual_seed(5)
    n = 3000
    a = (torch.randn(n, generator=g) * torch.exp2(torch.randint(-30, 30, (n,), generator=g).float())).float()
    b = (torch.randn(n, generator=g) * torch.exp2(torch.randint(-30, 30, (n,), generator=g).float())).float()
    c = (torch.randn(n, generator=g) * torch.exp2(torch.randint(-60, 60, (n,), generator=g).float())).float()
    c[:300] = (-(a[:300].double() * b[:300].double())).float()  # near-total cancellation
    e = 2.0 ** -23
    ties = [((1 + e), 2 * (1 - e), 2.0 ** 25 + 4),      # float64 sum on the midpoint 2^25 + 6
            (-(1 + e), 2 * (1 - e), -(2.0 ** 25 + 4)),
            ((1 + e), (1 + e) * 2 ** -24, 1.0)]
    ta = torch.tensor([t[0] for t in ties], dtype=torch.float32)
    tb = torch.tensor([t[1] for t in ties], dtype=torch.float32)
    tc = torch.tensor([t[2] for t in ties], dtype=torch.float32)
    got_t = R.fma32(ta, tb, tc)
    naive = (ta.double() * tb.double() + tc.double()).float()
    assert float(got_t[0]) == 2.0 ** 25 + 4 and float(naive[0]) == 2.0 ** 25 + 8
    a, b, c = torch.cat([a, ta]), torch.cat([b, tb]), torch.cat([c, tc])
    got = R.fma32(a, b, c)
    for i in range(a.numel()):
        want = _rn32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert float(got[i]) == want, (i, float(a[i]), float(b[i]), float(c[i]))


def _ulp32(x: torch.Tensor) -> torch.Tensor:
    f = x.float()
    return (torch.nextafter(f.abs(), torch.full_like(f, float("inf"))) - f.abs()).double()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_device_restatement_close_to_cpu_ops(dtype):
    """paged_adamw_step_device differs from the torch-CPU restatement only in
    where it rounds (v: alpha * RND(g * g) against RND(alpha * g) * g; the
    denominator: a multiply by the double reciprocal against a division; p:
    one fused multiply-add against RND(RND(-step m) / d) then an add): the
    first moment is bit-equal, the second within an ulp, the parameters
    within a few ulps of p plus of the update per step."""
    shapes = [(4096,)]
    p1 = _tensors(6, shapes)[0].to(dtype)
    p2 = p1.clone()
    m1, v1, m2, v2 = (torch.zeros(4096) for _ in range(4))
    for t in range(1, 6):
        gr = (_tensors(30 + t, shapes)[0] * 0.02).to(dtype)
        R.paged_adamw_step([p1], [gr], [m1], [v1], [t], lr=1e-3, exact_sqrt=True)
        R.paged_adamw_step_device([p2], [gr], [m2], [v2], [t], lr=1e-3)
    assert torch.equal(m1, m2)
    assert bool(((v1.double() - v2.double()).abs() <= 5 * _ulp32(v1)).all())
    mant = 23 if dtype == torch.float32 else 7
    bound = 5 * (2.0 ** -mant * p1.double().abs() + 4 * 2.0 ** -23 * 1e-3) + 1e-30
    assert bool(((p1.double() - p2.double()).abs() <= bound).all())
    assert not torch.equal(v1, v2) or not torch.equal(p1, p2)  # the roundings do differ somewhere


def test_device_restatement_closed_forms():
    """Zero gradients: exactly p * RND(1 - lr wd) per step, moments stay 0; a
    constant gradient: p moves by lr * t * g / (|g| + eps) (no decay)."""
    p = _tensors(2, [(1000,)])[0]
    want = p.clone()
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    for t in range(1, 4):
        R.paged_adamw_step_device([p], [torch.zeros_like(p)], [m], [v], [t], lr=1e-3, weight_decay=0.1)
        want = want * torch.tensor(1 - 1e-3 * 0.1, dtype=torch.float32)
    assert torch.equal(p, want) and not m.any() and not v.any()
    g = torch.tensor([1e-3, -2e-2, 0.5, -3.0])
    p = torch.zeros(4)
    m, v = torch.zeros(4), torch.zeros(4)
    for t in range(1, 11):
        R.paged_adamw_step_device([p], [g], [m], [v], [t], lr=1e-2, eps=1e-8, weight_decay=0.0)
    want = -10 * 1e-2 * g.double() / (g.double().abs() + 1e-8)
    assert torch.allclose(p.double(), want, rtol=1e-5, atol=0)


def test_oracle_skips_parameters_without_gradient():
    p = _tensors(3, [(10,)])[0]
    before = p.clone()
    R.paged_adamw_step([p], [None], [torch.zeros(10)], [torch.zeros(10)], [1])
    assert torch.equal(p, before)


def test_paged_adamw_host_layout_and_stats():
    """States are chunk-aligned views of two flat fp32 buffers (host memory
    without a GPU), shaped like their parameters; the statistics follow
    paged_adamw.py:129-151."""
    lin = torch.nn.Linear(10, 10)
    opt = PagedAdamW(lin.parameters(), lr=1e-3)
    st_w, st_b = opt.state[lin.weight], opt.state[lin.bias]
    assert st_w["exp_avg"].shape == lin.weight.shape and st_b["exp_avg_sq"].shape == lin.bias.shape
    assert st_w["exp_avg"].device.type == "cpu" and st_w["step"] == 0
    assert st_b["exp_avg"].data_ptr() - st_w["exp_avg"].data_ptr() == 4 * ADAMW_CHUNK
    stats = opt.get_memory_stats()
    assert stats["num_params"] == 2
    assert stats["cpu_pinned_mb"] == pytest.approx(110 * 4 * 2 / 2 ** 20)
    with pytest.raises(ValueError):
        PagedAdamW(lin.parameters(), lr=-1.0)
    with pytest.raises(ValueError):
        PagedAdamW(lin.parameters(), betas=(1.0, 0.999))


def test_paged_adamw_refuses_cpu_step():
    lin = torch.nn.Linear(4, 2)
    opt = PagedAdamW(lin.parameters())
    lin(torch.randn(1, 4)).sum().backward()
    with pytest.raises(RuntimeError):
        opt.step()
