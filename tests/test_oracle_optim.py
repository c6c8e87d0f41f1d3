"""The oracle's PagedAdamW step (oracle.qlora_ref.paged_adamw_step,
optim/paged_adamw.py:84-113) pinned against torch.optim.AdamW, zero and
constant gradients; and the optimizer's host logic (construction, state
layout, statistics) without a GPU."""
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
