"""The decode GEMV with the LoRA down-projection u = x A^T computed inside the
same launch (one wave per K-split job, in the workgroups themselves, hands its
partials to every workgroup through a partial region of the workspace's
synchronization area; the launch's last job readies the other region for the
next launch).  Checked against the oracle's
QuantLinear.forward + LoRALinear.forward (quant_linear.py:182-197,
lora_layer.py:60-70) at rtol = atol = 1e-2 in the activation dtype, and
against the library's own other paths bit for bit:

- calls in a row on one stream (the area is left ready after each);
- the workgroups' own computation of u when the jobs' partials are not
  awaited (wait forced to 0) or awaited only briefly (a wait of a few
  microseconds, after which some workgroups give up and others do not),
  which must give the same bits;
- replays of a captured HIP graph with new inputs, against eager calls;
- operands the jobs cannot read 16 bytes at a time, which run the
  down-projection as its own kernel.
"""
import math

import pytest
import torch

from oracle import qlora_ref as R
from rocm_qlora import _native as nat
from rocm_qlora import ops
from rocm_qlora.quantization import quantize_int4

pytestmark = pytest.mark.gpu

RTOL = ATOL = 1e-2


def _layer(N, K, rank, seed, dev, lora_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    a = torch.empty(rank, K)
    torch.nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
    b = torch.randn(N, rank, generator=g) * 0.01
    packed, absmax = quantize_int4(w.to(dev), 64)
    return packed, absmax, a.to(lora_dtype), b.to(lora_dtype)


def _x(M, K, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(dtype)


def _check(got, ref):
    got = got.cpu().float()
    ref = ref.float()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} outside tol; max err {float(err.max()):.4g}"


def _sync_words_ready(dev, sync_ready):
    torch.cuda.synchronize(dev)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    ws = ops._LINEAR_WS.get(key)
    assert ws is not None
    assert sync_ready(ws)


@pytest.mark.parametrize("K,N,M,rank", [
    (4096, 4096, 1, 16),     # q / o: 256 workgroups, 32 jobs
    (4096, 14336, 1, 16),    # gate / up
    (14336, 4096, 1, 16),    # down: 112 jobs, partials summed by 8 threads per rank
    (4096, 1024, 2, 16),     # k / v
    (4096, 4096, 5, 8),      # activations as register operands
    (4096, 1024, 16, 64),    # four rank groups, jobs of four chunks
    (1024, 512, 3, 32),
])
def test_calls_in_a_row(dev, sync_ready, K, N, M, rank):
    print(f"in-launch lora K={K} N={N} M={M} rank={rank}", flush=True)
    packed, absmax, a, b = _layer(N, K, rank, seed=K + N + rank, dev=dev)
    ad, bd = a.to(dev), b.to(dev)
    for i in range(3):
        x = _x(M, K, seed=100 * i + M)
        y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
        ref = R.nf4_lora_linear(x, packed.cpu(), absmax.cpu(), None, a, b, 2.0, N, 64)
        _check(y, ref)
    _sync_words_ready(dev, sync_ready)


def test_mixed_shapes_share_one_workspace(dev, sync_ready):
    """Launches of different extents (K splits x M x rank) in a row on one
    stream, twice round: each leaves its partials in one region and readies
    the other for the next launch, so every call gives the bits of the same
    call on a fresh workspace (a stream of its own) and the area is ready
    after each one."""
    specs = [(4096, 4096, 1, 16), (4096, 1024, 16, 64), (14336, 4096, 1, 16), (1024, 512, 3, 32),
             (4096, 14336, 2, 16), (2048, 768, 1, 8)]
    layers = [(K, N, M, r) + _layer(N, K, r, seed=K + N + r + M, dev=dev) for K, N, M, r in specs]
    for rnd in range(2):
        for i, (K, N, M, r, packed, absmax, a, b) in enumerate(layers):
            print(f"mixed round {rnd} call {i}: K={K} N={N} M={M} rank={r}", flush=True)
            x = _x(M, K, seed=10 * rnd + i).to(dev)
            ad, bd = a.to(dev), b.to(dev)
            got = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
            _sync_words_ready(dev, sync_ready)
            fresh = torch.cuda.Stream(dev)
            fresh.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(fresh):
                want = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
            torch.cuda.synchronize(dev)
            ops._LINEAR_WS.pop((dev.index if dev.index is not None else torch.cuda.current_device(),
                                fresh.cuda_stream), None)
            assert torch.equal(got, want), f"call {i} of round {rnd} differs from a fresh workspace"


@pytest.mark.parametrize("K,N,M,rank,lora_dtype", [
    (4096, 4096, 1, 16, torch.float32),
    (4096, 1024, 4, 64, torch.float32),
    (2048, 768, 2, 16, torch.bfloat16),
])
def test_workgroups_own_u_same_bits(dev, sync_ready, K, N, M, rank, lora_dtype):
    """Wait forced to 0: every workgroup computes u itself, job by job as
    the job waves do, so y is bit-identical to the awaited path."""
    print(f"own-u K={K} N={N} M={M} rank={rank} {lora_dtype}", flush=True)
    packed, absmax, a, b = _layer(N, K, rank, seed=7 + K, dev=dev, lora_dtype=lora_dtype)
    x = _x(M, K, seed=3).to(dev)
    ad, bd = a.to(dev), b.to(dev)
    y0 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
    old = nat.set_gemv_wait_us(0)
    try:
        y1 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
        y2 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
    finally:
        nat.set_gemv_wait_us(old)
    y3 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
    assert torch.equal(y0, y1) and torch.equal(y0, y2) and torch.equal(y0, y3)
    _sync_words_ready(dev, sync_ready)
    ref = R.nf4_lora_linear(x.cpu(), packed.cpu(), absmax.cpu(), None, a, b, 0.5, N, 64)
    _check(y1, ref)


@pytest.mark.parametrize("wait_us", [1, 3])
def test_short_wait_same_bits(dev, sync_ready, wait_us):
    """A wait bounded at a few microseconds of the device's real-time
    counter: workgroups that give up compute u themselves, the others take
    the jobs' partials; either way y has the same bits, over several calls
    in a row, and the area is left ready for the default wait."""
    K, N, M, rank = 14336, 4096, 1, 64
    print(f"short wait {wait_us} us K={K} N={N} M={M} rank={rank}", flush=True)
    packed, absmax, a, b = _layer(N, K, rank, seed=91, dev=dev)
    x = _x(M, K, seed=13).to(dev)
    ad, bd = a.to(dev), b.to(dev)
    y0 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
    old = nat.set_gemv_wait_us(wait_us)
    try:
        ys = [ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5) for _ in range(4)]
    finally:
        nat.set_gemv_wait_us(old)
    y5 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=0.5)
    for i, y in enumerate(ys + [y5]):
        assert torch.equal(y0, y), f"call {i} after a {wait_us} us wait differs"
    _sync_words_ready(dev, sync_ready)
    ref = R.nf4_lora_linear(x.cpu(), packed.cpu(), absmax.cpu(), None, a, b, 0.5, N, 64)
    _check(y5, ref)


def test_graph_replays_match_eager(dev, sync_ready):
    K, N, M, rank = 4096, 4096, 1, 16
    packed, absmax, a, b = _layer(N, K, rank, seed=11, dev=dev)
    ad, bd = a.to(dev), b.to(dev)
    xs = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(2):  # warm the allocator and the kernels outside the capture
            ops.nf4_linear(xs, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ys = ops.nf4_linear(xs, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
    for i in range(4):
        x = _x(M, K, seed=50 + i).to(dev)
        xs.copy_(x)
        graph.replay()
        got = ys.clone()
        torch.cuda.synchronize(dev)
        want = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
        torch.cuda.synchronize(dev)
        assert torch.equal(got, want), f"replay {i} differs from the eager call"
    _sync_words_ready(dev, sync_ready)


def test_two_graphs_replayed_in_turn(dev):
    """Two captures take workspaces of their own (spares zeroed by eager
    calls beforehand); replays of either, in turn, match eager calls."""
    K, M, rank = 4096, 2, 16
    shapes = [(4096, 11), (14336, 12)]
    layers = [(N,) + _layer(N, K, rank, seed=s, dev=dev) for N, s in shapes]
    xs = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream(dev)
    graphs, outs, operands = [], [], []
    for N, packed, absmax, a, b in layers:
        ad, bd = a.to(dev), b.to(dev)
        operands.append((ad, bd))  # a graph does not keep its inputs alive
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            ops.nf4_linear(xs, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
        torch.cuda.current_stream(dev).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(ops.nf4_linear(xs, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0))
        graphs.append(g)
    for i in range(6):
        j = i % 2
        N, packed, absmax, a, b = layers[j]
        x = _x(M, K, seed=70 + i).to(dev)
        xs.copy_(x)
        graphs[j].replay()
        got = outs[j].clone()
        want = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=a.to(dev), lora_b=b.to(dev), scaling=2.0)
        torch.cuda.synchronize(dev)
        assert torch.equal(got, want), f"replay {i} of graph {j} differs from the eager call"


@pytest.mark.parametrize("case", ["lora_x_offset", "a_offset", "bf16_a_offset", "strided_b"])
def test_unaligned_operands_run_separate_kernel(dev, case):
    K, N, M, rank = 1024, 1024, 2, 16
    lora_dtype = torch.bfloat16 if case == "bf16_a_offset" else torch.float32
    packed, absmax, a, b = _layer(N, K, rank, seed=21, dev=dev, lora_dtype=lora_dtype)
    x = _x(M, K, seed=5)
    xl = _x(M, K, seed=6)
    if case == "lora_x_offset":
        # rows 8 bytes off a 16-byte boundary
        buf = torch.zeros(M * K + 4, dtype=torch.bfloat16, device=dev)
        xld = buf[4:].view(M, K)
        xld.copy_(xl.to(dev))
        ad = a.to(dev)
    else:
        xld = xl.to(dev)
        buf = torch.zeros(rank * K + 2, dtype=lora_dtype, device=dev)
        ad = buf[2:].view(rank, K)
        ad.copy_(a.to(dev))
    bd = b.to(dev)
    if case == "strided_b":
        # rows of B 4 * (rank + 3) bytes apart: the LoRA term is added by the
        # split-K finisher, which reads B by element
        wide = torch.zeros(N, rank + 3, dtype=lora_dtype, device=dev)
        wide[:, 1:1 + rank] = bd
        bd = wide[:, 1:1 + rank]
    y = ops.nf4_linear(x.to(dev), packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0, lora_x=xld)
    base = R.quant_linear_forward(x, R.dequantize_int4(packed.cpu(), absmax.cpu(), 64), None, N, K)
    ref = R.lora_forward(xl, base, a, b, 2.0)
    _check(y, ref)


def test_capture_forking_side_streams(dev, sync_ready):
    """A capture that forks two side streams, each running fused-LoRA M = 1
    GEMVs (the in-launch handshake) and a GEMM with K splits: each branch
    gets a workspace of its own, and every replay matches eager calls bit
    for bit; the eager workspace's synchronization area is left ready."""
    K, M, rank = 4096, 1, 16
    specs = [(4096, 31), (1024, 32)]
    layers = [(N,) + _layer(N, K, rank, seed=s, dev=dev) for N, s in specs]
    ops_dev = [(N, p, s_, a.to(dev), b.to(dev)) for N, p, s_, a, b in layers]
    xs = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    xg = torch.zeros(64, K, dtype=torch.bfloat16, device=dev)

    def run(x, x64):
        out = []
        for N, p, s_, ad, bd in ops_dev:
            out.append(ops.nf4_linear(x, p, s_, N, 64, lora_a=ad, lora_b=bd, scaling=2.0))
        N, p, s_, ad, bd = ops_dev[1]
        out.append(ops.nf4_linear(x64, p, s_, N, 64, lora_a=ad, lora_b=bd, scaling=2.0))
        return out

    run(xs, xg)  # eager warm-up
    torch.cuda.synchronize(dev)
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        main = torch.cuda.current_stream(dev)
        s1.wait_stream(main)
        s2.wait_stream(main)
        with torch.cuda.stream(s1):
            o1 = run(xs, xg)
        with torch.cuda.stream(s2):
            o2 = run(xs, xg)
        main.wait_stream(s1)
        main.wait_stream(s2)
    for i in range(4):
        xs.copy_(_x(M, K, seed=90 + i).to(dev))
        xg.copy_(_x(64, K, seed=95 + i).to(dev))
        graph.replay()
        got = [t.clone() for t in o1 + o2]
        want = run(xs, xg)
        torch.cuda.synchronize(dev)
        for g, w in zip(got, want + want):
            assert torch.equal(g, w), f"replay {i} differs from the eager calls"
    _sync_words_ready(dev, sync_ready)


def test_captured_gemm_holds_no_fill_node(dev):
    """A capture preceded by an eager call of the same work takes a
    pre-zeroed workspace of the size it needs (here the M = 2048 GEMM's with
    its K-split partials, larger than the pool's first entries), so its
    replays run the library's kernels only -- no fill node -- and give the
    eager call's bits."""
    from torch.profiler import ProfilerActivity, profile
    K, N, M, rank = 4096, 1024, 2048, 16
    print(f"captured GEMM K={K} N={N} M={M} rank={rank}", flush=True)
    packed, absmax, a, b = _layer(N, K, rank, seed=111, dev=dev)
    ad, bd = a.to(dev), b.to(dev)
    x = _x(M, K, seed=112).to(dev)
    y0 = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=ad, lora_b=bd, scaling=2.0)
    graph.replay()
    torch.cuda.synchronize(dev)
    assert torch.equal(y, y0)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        graph.replay()
        torch.cuda.synchronize(dev)
    assert torch.equal(y, y0)
    names = sorted({e.name for e in prof.events() if e.device_type.name in ("CUDA", "PrivateUse1")})
    if not names:
        pytest.skip("the profiler recorded no GPU kernels of the replay on this system")
    foreign = [n for n in names if "rq::" not in n and not n.startswith("_ZN2rq")]
    assert not foreign, f"the replay ran kernels outside the library: {foreign}"
