"""GPU parity of the fused AdamW step (rq_adamw_step behind PagedAdamW).

The reference updates on the parameter's device (optim/paged_adamw.py:98-113
moves the states there), so its arithmetic is that of torch's GPU kernels.
Bar: bit-exact -- parameters, m and v -- against the oracle's restatement of
those roundings (oracle.qlora_ref.paged_adamw_step_device, on the CPU), and
that restatement bit-exact against the reference's ops themselves run by
torch on the GPU (paged_adamw_step on device tensors).  Against the torch-CPU
restatement (paged_adamw_step), m bit-exact, v within an ulp and the
parameters within, per step, a few ulps of p plus of the update's size (lr):
torch's CPU kernels round v's product, the denominator's division and the
parameter update at other points, and an ulp of the denominator moves the
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


def _run(dev, dtype, offload, steps=5, page_mb=1, none_every=3, groups=False, ref="device"):
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
            kw = dict(lr=grp["lr"], betas=grp["betas"], eps=grp["eps"], weight_decay=grp["weight_decay"])
            if ref == "device":
                R.paged_adamw_step_device([ref_p[i]], [gr], [ref_m[i]], [ref_v[i]], [ref_steps[i]], **kw)
            else:
                R.paged_adamw_step([ref_p[i]], [gr], [ref_m[i]], [ref_v[i]], [ref_steps[i]], **kw)
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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_device_restatement_is_torch_on_the_gpu(dev, dtype):
    """The reference's ops (paged_adamw_step: mul_, add_, addcmul_, sqrt, /,
    add_, addcdiv_) run by torch on the GPU give the oracle's device
    restatement bit for bit, over five steps on every shape."""
    print(f"adamw torch-gpu ops vs device restatement {dtype}", flush=True)
    g = torch.Generator().manual_seed(11)
    for s in SHAPES:
        p_cpu = (torch.randn(s, generator=g) * 0.05).to(dtype)
        p_dev = p_cpu.to(dev)
        m_cpu, v_cpu = torch.zeros(s), torch.zeros(s)
        m_dev, v_dev = m_cpu.to(dev), v_cpu.to(dev)
        for t in range(1, 6):
            gr = (torch.randn(s, generator=g) * 1e-3).to(dtype)
            R.paged_adamw_step_device([p_cpu], [gr], [m_cpu], [v_cpu], [t], lr=1e-3, weight_decay=0.01)
            R.paged_adamw_step([p_dev], [gr.to(dev)], [m_dev], [v_dev], [t], lr=1e-3, weight_decay=0.01)
        assert _bits_equal(m_dev.cpu(), m_cpu), s
        assert _bits_equal(v_dev.cpu(), v_cpu), s
        assert _bits_equal(p_dev.cpu(), p_cpu), s


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adamw_vs_torch_cpu_restatement(dev, dtype):
    print(f"adamw vs torch-cpu ops {dtype}", flush=True)
    opt, params, ref_p, ref_m, ref_v, ref_steps = _run(dev, dtype, False, ref="cpu")
    for i, p in enumerate(params):
        st = opt.state[p]
        assert _bits_equal(st["exp_avg"].cpu(), ref_m[i]), f"m of tensor {i}"
        v, want_v = st["exp_avg_sq"].cpu().double(), ref_v[i].double()
        assert bool(((v - want_v).abs() <= ref_steps[i] * 2.0 ** -23 * want_v.abs()).all()), f"v of tensor {i}"
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
        assert float((pa - pb).detach().abs().max()) < 1e-5
