"""GPU parity of the fused AdamW step (rq_adamw_step behind PagedAdamW)
against the oracle's restatement of PagedAdamW.step
(oracle.qlora_ref.paged_adamw_step, optim/paged_adamw.py:84-113).

Bar: bit-exact -- parameters, m and v -- against the oracle with a
correctly rounded square root (exact_sqrt=True: the reference's op order
with the multiply-adds fused where torch's CPU kernels fuse them); against
the plain torch-CPU restatement, m and v bit-exact and the parameters within,
per step, one ulp of p plus four ulps of the update's size (lr): torch's
vectorized CPU sqrt is one ulp off for some inputs (0.07 % to 1.2 % of them,
depending on the host's SIMD path), and an ulp of the denominator moves the
update by about an ulp of the update -- near p = 0 many ulps of p."""
import copy

import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import LoRALinear, QuantLinear
from rocm_qlora.optim import PagedAdamW

pytestmark = pytest.mark.gpu

SHAPES = [(1,), (7,), (2047,), (2048,), (2049,), (300001,), (16, 4096), (4096, 16)]


def _ulps32(a, b):
    return (a.view(torch.int32).long() - b.view(torch.int32).long()).abs()


def _check_params(got, want, steps, lr, mant_bits):
    """|got - want| <= steps * (ulp(want) + 4 ulp(lr))."""
    got, want = got.double(), want.double()
    ulp = 2.0 ** -mant_bits
    bound = steps * (ulp * want.abs() + 4 * ulp * lr) + 1e-30
    err = (got - want).abs()
    assert bool((err <= bound).all()), f"max err {float(err.max()):.3g}, worst ratio {float((err / bound).max()):.2f}"


def _bits_equal(a, b):
    return torch.equal(a.contiguous().view(torch.int8), b.contiguous().view(torch.int8))


def _run(dev, dtype, offload, steps=5, page_mb=1, none_every=3, groups=False, exact_sqrt=True):
    g = torch.Generator().manual_seed(7)
    init = [(torch.randn(s, generator=g) * 0.05).to(dtype) for s in SHAPES]
    params = [torch.nn.Parameter(t.clone().to(dev)) for t in init]
    if groups:
        pg = [{"params": params[:4], "lr": 1e-3, "weight_decay": 0.0},
              {"params": params[4:], "lr": 3e-4, "weight_decay": 0.05, "betas": (0.8, 0.99), "eps": 1e-6}]
        opt = PagedAdamW(pg, page_size_mb=page_mb, offload_states=offload)
    else:
        opt = PagedAdamW(params, lr=1e-3, weight_decay=0.01, page_size_mb=page_mb, offload_states=offload)
    ref_p = [t.clone() for t in init]
    ref_m = [torch.zeros(s) for s in SHAPES]
    ref_v = [torch.zeros(s) for s in SHAPES]
    ref_steps = [0] * len(SHAPES)
    for t in range(1, steps + 1):
        grads = []
        for i, s in enumerate(SHAPES):
            if none_every and (i + t) % none_every == 0:
                grads.append(None)  # skipped this step (paged_adamw.py:86-87)
            else:
                grads.append((torch.randn(s, generator=g) * 1e-3).to(dtype))
        for p, gr in zip(params, grads):
            p.grad = gr.to(dev) if gr is not None else None
        opt.step()
        for i, gr in enumerate(grads):
            if gr is None:
                continue
            ref_steps[i] += 1
            grp = opt.param_groups[0 if not groups or i < 4 else 1]
            R.paged_adamw_step([ref_p[i]], [gr], [ref_m[i]], [ref_v[i]], [ref_steps[i]], lr=grp["lr"],
                               betas=grp["betas"], eps=grp["eps"], weight_decay=grp["weight_decay"],
                               exact_sqrt=exact_sqrt)
    return opt, params, ref_p, ref_m, ref_v, ref_steps


@pytest.mark.parametrize("offload", [False, True])
@pytest.mark.parametrize("groups", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_adamw_bit_exact_vs_oracle(dev, offload, groups, dtype):
    print(f"adamw {dtype} offload={offload} groups={groups}", flush=True)
    opt, params, ref_p, ref_m, ref_v, ref_steps = _run(dev, dtype, offload, groups=groups)
    for i, p in enumerate(params):
        st = opt.state[p]
        assert st["step"] == ref_steps[i]
        assert _bits_equal(st["exp_avg"].cpu(), ref_m[i]), f"m of tensor {i}"
        assert _bits_equal(st["exp_avg_sq"].cpu(), ref_v[i]), f"v of tensor {i}"
        assert _bits_equal(p.detach().cpu(), ref_p[i]), f"p of tensor {i}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adamw_vs_torch_cpu_restatement(dev, dtype):
    print(f"adamw vs torch-cpu sqrt {dtype}", flush=True)
    opt, params, ref_p, ref_m, ref_v, ref_steps = _run(dev, dtype, False, exact_sqrt=False)
    for i, p in enumerate(params):
        st = opt.state[p]
        assert _bits_equal(st["exp_avg"].cpu(), ref_m[i]), f"m of tensor {i}"
        assert _bits_equal(st["exp_avg_sq"].cpu(), ref_v[i]), f"v of tensor {i}"
        _check_params(p.detach().cpu(), ref_p[i], ref_steps[i], 1e-3, 23 if dtype == torch.float32 else 7)


def test_adamw_offloaded_states_stay_pinned_on_host(dev):
    """Between steps the states are pinned host tensors (paged_adamw.py:46-61),
    and the offloaded and resident modes give the same bits."""
    a = _run(dev, torch.float32, offload=True, steps=3, page_mb=1)
    b = _run(dev, torch.float32, offload=False, steps=3)
    for pa, pb in zip(a[1], b[1]):
        sa, sb = a[0].state[pa], b[0].state[pb]
        assert sa["exp_avg"].device.type == "cpu" and sa["exp_avg"].is_pinned()
        assert sb["exp_avg"].device.type == "cuda"
        assert torch.equal(pa.detach(), pb.detach())
        assert torch.equal(sa["exp_avg_sq"], sb["exp_avg_sq"].cpu())
    stats = a[0].get_memory_stats()
    assert stats["num_params"] == len(SHAPES) and stats["cpu_pinned_mb"] > 0


def test_adamw_state_dict_roundtrip(dev):
    opt, params, *_ = _run(dev, torch.float32, offload=True, steps=2)
    sd = opt.state_dict()
    new = PagedAdamW(params, lr=1e-3, weight_decay=0.01, page_size_mb=1)
    new.load_state_dict(sd)
    for p in params:
        a, b = opt.state[p], new.state[p]
        assert b["exp_avg"].device.type == "cpu" and b["exp_avg"].is_pinned()
        assert torch.equal(a["exp_avg"], b["exp_avg"]) and a["step"] == b["step"]
    # both continue identically
    for p in params:
        p.grad = torch.full_like(p, 1e-3)
    snapshot = [p.detach().clone() for p in params]
    new.step()
    after_new = [p.detach().clone() for p in params]
    with torch.no_grad():
        for p, s in zip(params, snapshot):
            p.copy_(s)
    opt.step()
    for p, s in zip(params, after_new):
        assert torch.equal(p.detach(), s)


def test_adamw_trains_lora_and_matches_torch_adamw(dev):
    """A LoRA layer on an NF4 base trained a few steps: loss falls, and the
    adapters stay within 1e-5 of torch.optim.AdamW run on a copy (the same
    update rule; torch's first moment goes through lerp_)."""
    torch.manual_seed(3)
    base = torch.nn.Linear(256, 128).to(dev)
    layers = []
    for _ in range(2):
        ql = QuantLinear.from_linear(copy.deepcopy(base), bits=4, block_size=64)
        lora = LoRALinear(ql, r=8, lora_alpha=16)
        with torch.no_grad():
            lora.lora_B.normal_(0, 0.01)
        layers.append(lora)
    layers[1].lora_A.data.copy_(layers[0].lora_A.data)
    layers[1].lora_B.data.copy_(layers[0].lora_B.data)
    opt_a = PagedAdamW([layers[0].lora_A, layers[0].lora_B], lr=1e-2, offload_states=False)
    opt_b = torch.optim.AdamW([layers[1].lora_A, layers[1].lora_B], lr=1e-2, weight_decay=0.01, foreach=False)
    x = torch.randn(32, 256, device=dev, dtype=torch.bfloat16)
    target = torch.randn(32, 128, device=dev)
    losses = []
    for _ in range(5):
        for lora, opt in ((layers[0], opt_a), (layers[1], opt_b)):
            opt.zero_grad()
            loss = torch.nn.functional.mse_loss(lora(x).float(), target)
            loss.backward()
            opt.step()
            if opt is opt_a:
                losses.append(float(loss.detach()))
    assert losses[-1] < losses[0]
    for pa, pb in ((layers[0].lora_A, layers[1].lora_A), (layers[0].lora_B, layers[1].lora_B)):
        assert float((pa - pb).abs().max()) < 1e-5
