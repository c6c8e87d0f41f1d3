#!/usr/bin/env python3
"""Benchmark of the MI355X NF4 quantized-linear path at Llama-3-8B projection shapes.

Headline (`value`, GB/s): one step is one Llama-3-8B decoder layer's seven
NF4 projections (q, k, v, o, gate, up, down; in x out = 4096x4096,
4096x1024 twice, 4096x4096, 4096x14336 twice, 14336x4096) run as decode
dequant-GEMVs with the LoRA term fused (M = 1 token by default, bf16
activations N(0,1), weights N(0,0.02) quantized to NF4 block 64 with fp32
absmax, LoRA r = 16, alpha = 32).  `value` is the step's algorithmic HBM
bytes divided by its time, with every input resident in HBM.  Weights rotate
over enough layer copies (> 512 MB) that the 256 MB MALL cannot serve them.
The step is captured once per layer copy as a HIP graph and replayed.

Also reported:
  config        p10 / p50 / p90 of the headline's per-step times, from a
                second pass with an event after every step (which adds about
                4 us per step; `value` comes from the uninstrumented pass).
  roofline      the dominant kernel as the headline step runs it (the GEMV at
                the gate/up shape with the LoRA term fused), timed with HIP
                events over back-to-back launches on the stream they run on;
                algorithmic bytes / average launch time vs 8 TB/s.  `traffic`
                is the HBM bytes per launch that the committed counter
                profile (profiles/nf4_gemv_kernel_traffic.md) holds for the
                same kernel, mode and shape, or null.
  decode_m      the same decode step at the configuration's other batch sizes
                (M in {1, 4, 8, 16}), 50 steps each.
  decode_per_shape
                per projection at the headline M: median launch time with the
                LoRA term fused and without it, and a minimal launch (a 4-byte
                fill) of the same graph structure.
  config1       one NF4 4096x4096 QuantLinear with LoRA r = 16 on fp32
                activations (M = 1 and 16), the fp32-MFMA path, rotating 60
                weight copies (565 MB).
  gemm          the prefill/training shapes: the same seven projections at
                M = 2048 tokens with LoRA r = 64, alpha = 16, forward and dX
                backward, TFLOP/s and fraction of the 2.5 PFLOP/s bf16 MFMA peak.
  codec         NF4 + double quantization of an 11008x4096 bf16 weight (N(0,0.02)
                with 0.1 % outliers at +-8 sigma, blocks 64 / 256): quantize ->
                pack -> double-quantize the absmax, and double-dequantize ->
                bf16, over 5 weight copies (565 MB); algorithmic bytes / time
                vs 8 TB/s.
  byte_linears  INT8 (per-row absmax: W8A16 on the bf16 MFMA, and the
                separate W8A8 mode on the int8 MFMA) and FP8 (e4m3
                per-tensor scales, fp8 MFMA) linears at the Llama-3-70B MLP
                shape 8192 -> 28672, M = 1 (HBM: bytes / time, two weight
                copies rotating) and M = 512, 4096 (TFLOP/s against the bf16,
                int8 and fp8 MFMA peaks, 2.5, 5.0 and 5.0 P/s), plus W8A8's
                relative deviation from W8A16 at M = 512.
  optimizer     the fused AdamW step over the LoRA adapters of a whole
                Llama-3-8B (r = 16, 7 projections x 32 layers, 41.9 M fp32
                parameters): kernel time vs 8 TB/s (28 bytes per parameter),
                and PagedAdamW.step() wall time with the states resident and
                offloaded to pinned host memory.
  cpu_baseline  the oracle's restatement of the reference's CPU path on the
                host cores: the headline decode step whole (`value`), and per
                configuration (fp32 config 1, codec, GEMM forward / dX, INT8 /
                FP8, the AdamW update) on stated samples, each beside the GPU time of the same
                work; 2 warm-ups, median of 10 runs, thread count, core count
                and CPU model reported.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m M] [--no-gemm] [--no-extra] [--no-cpu]
    python bench.py --summarize-profile DIR   # per-kernel, per-grid rocprofv3 kernel-trace table
    python bench.py --counters [gemv|fp8_gemm|int8_gemm|nf4_gemm]   # short eager run for rocprofv3 --pmc passes
    python bench.py --summarize-counters DIR [DIR ...]   # per-kernel counter means; for the gemv run,
                                                         # HBM bytes per launch per (shape, mode)
"""
import argparse
import csv
import glob
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rocm-qlora_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "NF4 dequant-GEMV GB/s + GEMM TFLOP/s (% roofline), Llama-3-8B proj shapes"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0       # MI355X dense fp8 MFMA
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA (TOP/s)

# (name, in_features K, out_features N)
LLAMA3_8B_PROJ = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
                  ("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096)]
RANK, ALPHA, BLOCK = 16, 32, 64
SCALING = ALPHA / RANK
GEMM_M, GEMM_RANK, GEMM_ALPHA = 2048, 64, 16
CONFIG1_COPIES = 60            # 4096x4096 NF4 weights: 60 x 9.4 MB = 565 MB
CODEC_COPIES = 5               # 11008x4096 bf16 weights and their codes: 5 x 113 MB = 565 MB

# The counter profile of the decode GEMV: `bench.py --summarize-counters`
# output for `bench.py --counters` (FETCH_SIZE and WRITE_SIZE passes), whose
# table rows "| nf4_gemv_kernel | shape | mode | M | K | N | fetch | write |
# total | algorithmic | ratio |" give the HBM bytes per launch.
GEMV_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "nf4_gemv_kernel_traffic.md")
COPY_BYTES = 512 << 20         # calibration copy: 512 MiB read + 512 MiB written
# (shape, LoRA fused) of the counter run, in launch order
GEMV_COUNTER_CONFIGS = [("gate", False, 1), ("gate", True, 1), ("k", False, 1), ("k", True, 1),
                        ("gate", False, 16), ("gate", True, 16), ("k", False, 16), ("k", True, 16)]


def profiled_traffic(shape, mode, M, K, N, path=GEMV_TRAFFIC_PROFILE):
    """HBM bytes per launch of nf4_gemv_kernel for (shape, mode, M, K, N) from
    the committed counter profile, or None when it holds no such row."""
    try:
        with open(path) as fh:
            for line in fh:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 9 and cells[0] == "nf4_gemv_kernel" and cells[1:6] == \
                        [shape, mode, str(M), str(K), str(N)]:
                    return int(cells[8].replace(",", ""))
    except OSError:
        return None
    return None


def gemv_bytes(M, N, K, rank=RANK, scale_bytes=4):
    """Algorithmic HBM bytes of one fused NF4 LoRA linear: packed codes,
    absmax, activations in and out, LoRA A and B (bf16 accounting)."""
    return N * K // 2 + (N * K // BLOCK) * scale_bytes + M * K * 2 + M * N * 2 + (rank * K + N * rank) * 2


def kernel_bytes(M, N, K, scale_bytes=4):
    """Algorithmic bytes of one plain GEMV launch (no LoRA)."""
    return N * K // 2 + (N * K // BLOCK) * scale_bytes + M * K * 2 + M * N * 2


def gemm_flops(M, N, K, rank):
    """2MNK + 2Mr(K + N): base product plus the two LoRA products."""
    return 2 * M * N * K + 2 * M * rank * (K + N)


def make_layer(dev, seed, rank=RANK):
    import torch
    from rocm_qlora.quantization import quantize_int4
    g = torch.Generator(device=dev).manual_seed(seed)
    layer = {}
    for name, K, N in LLAMA3_8B_PROJ:
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        packed, absmax = quantize_int4(w, BLOCK)
        del w
        a = (torch.rand(rank, K, generator=g, device=dev) * 2 - 1) / math.sqrt(K)  # kaiming_uniform(a=sqrt 5)
        b = torch.randn(N, rank, generator=g, device=dev) * 0.01
        layer[name] = (packed, absmax, a, b, N, K)
    return layer


class _Range:
    """A roctx range (rocprofv3 --marker-trace) naming a timed region, so a
    profile can attribute kernel launches to it; a no-op where torch has no
    range support."""

    def __init__(self, name):
        self.name = name

    def __enter__(self):
        import torch
        try:
            torch.cuda.nvtx.range_push(self.name)
            self.ok = True
        except Exception:
            self.ok = False
        return self

    def __exit__(self, *exc):
        import torch
        if self.ok:
            torch.cuda.nvtx.range_pop()


def _time_graph(graph, reps):
    """ms per replay, HIP events on the stream the replays run on."""
    import torch
    cur = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    graph.replay()
    torch.cuda.synchronize()
    t0.record(cur)
    for _ in range(reps):
        graph.replay()
    t1.record(cur)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def _time_graph_stats(graph, reps):
    """ms per replay of `reps` back-to-back replays on the current stream:
    "mean" from HIP events around all of them; p10 / median / p90 from a
    second pass with an event after each replay (those events add a few us
    per replay, so the mean is taken without them)."""
    import torch
    cur = torch.cuda.current_stream()
    graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(cur)
    for _ in range(reps):
        graph.replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record(cur)
    for i in range(reps):
        graph.replay()
        ev[i + 1].record(cur)
    torch.cuda.synchronize()
    d = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
    return {"mean": t0.elapsed_time(t1) / reps, "p10": _pct(d, 10), "p50": _pct(d, 50), "p90": _pct(d, 90)}


def _pct(sorted_vals, q):
    """Nearest-rank percentile of an ascending list."""
    i = min(len(sorted_vals) - 1, max(0, math.ceil(q / 100 * len(sorted_vals)) - 1))
    return sorted_vals[i]


def _capture(fn, stream):
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            fn()
    torch.cuda.synchronize()
    return g


def _cpu_threads():
    """Host threads for the CPU leg: the process's OpenMP share (the GPU box
    gives one GPU's job a share of its cores through OMP_NUM_THREADS), else
    every core os.cpu_count() reports."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cpu_time(fn, runs=10, warmup=2):
    """time.perf_counter() median (and p10 / p90) of `runs` calls after
    `warmup` calls, in seconds."""
    for _ in range(warmup):
        fn()
    d = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        d.append(time.perf_counter() - t0)
    d.sort()
    return {"median": d[len(d) // 2], "p10": _pct(d, 10), "p90": _pct(d, 90), "runs": runs}


def cpu_baselines(layer_cpu, xs_cpu, M, gpu):
    """The oracle's CPU restatement of the reference's CPU path (dequantize ->
    .to(x.dtype) -> F.linear + LoRA; the NF4 / double-quant codec; INT8 and
    FP8 dequantize-then-matmul), timed on this host's cores: 2 warm-up calls,
    median of 10.  Config 3 (the headline decode step) runs whole; the other
    configurations run a sample of whole rows or blocks (every operation is
    per row or per block, so time scales with the sample), stated in each
    entry.  `gpu` holds the GPU time of the same work where bench.py measured
    it."""
    import torch
    from oracle import qlora_ref as R
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(2024)
    out = {"threads": torch.get_num_threads(), "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model(),
           "timing": "time.perf_counter, 2 warm-ups, median (p10 / p90) of 10 runs", "seed": 2024}

    def entry(t, work, unit, gpu_s=None, note=""):
        e = {"cpu_ms": round(t["median"] * 1e3, 3), "cpu_ms_p10": round(t["p10"] * 1e3, 3),
             "cpu_ms_p90": round(t["p90"] * 1e3, 3), unit: round(work / t["median"] / (1e9 if unit == "gbs" else 1e12), 4)}
        if gpu_s:
            e["gpu_us"] = round(gpu_s * 1e6, 3)
            e["speedup"] = round(t["median"] / gpu_s, 1)
        if note:
            e["sample"] = note
        return e

    # config 3: one decode step of the seven projections (headline)
    def step():
        for name, K, N in LLAMA3_8B_PROJ:
            packed, absmax, a, b, _, _ = layer_cpu[name]
            R.nf4_lora_linear(xs_cpu[K], packed, absmax, None, a, b, SCALING, N, BLOCK)
    step_bytes = sum(gemv_bytes(M, N, K) for _, K, N in LLAMA3_8B_PROJ)
    t3 = _cpu_time(step)
    out["config3_decode_step"] = entry(t3, step_bytes, "gbs", gpu.get("decode_step_s"),
                                       f"whole step, M={M}")
    # config 1: fp32 4096x4096 NF4 + LoRA r=16, M in {1, 16}
    K1 = N1 = 4096
    w1 = torch.randn(N1, K1, generator=g) * 0.02
    p1, s1 = R.quantize_int4(w1, 64)
    a1 = (torch.rand(RANK, K1, generator=g) * 2 - 1) / math.sqrt(K1)
    b1 = torch.randn(N1, RANK, generator=g) * 0.01
    for m in (1, 16):
        x1 = torch.randn(m, K1, generator=g)
        t = _cpu_time(lambda: R.nf4_lora_linear(x1, p1, s1, None, a1, b1, SCALING, N1, 64))
        out[f"config1_m{m}"] = entry(t, gemv_bytes(m, N1, K1), "gbs", gpu.get(f"config1_m{m}_s"), "whole call, fp32")
    del w1, p1, s1
    # config 2: codec on 1376 of the 11008 rows (1/8 of the blocks)
    rows, K2 = 1376, 4096
    w2 = torch.randn(rows, K2, generator=g) * 0.02
    n_out = rows * K2 // 1000
    idx = torch.randperm(rows * K2, generator=g)[:n_out]
    w2.view(-1)[idx] = (torch.randint(0, 2, (n_out,), generator=g).float() * 2 - 1) * 0.16
    w2 = w2.to(torch.bfloat16)
    numel2 = rows * K2
    codec_bytes = 2 * numel2 + numel2 // 2 + numel2 // 64 + 4 * numel2 // 16384
    state = {}

    def enc():
        state["dq"] = R.double_quantize(w2, 64, 256, True)

    t = _cpu_time(enc)
    frac = numel2 / (11008 * 4096)
    out["config2_encode"] = entry(t, codec_bytes, "gbs", gpu["codec_encode_s"] * frac if gpu.get("codec_encode_s") else None,
                                  f"{rows} of 11008 rows; gpu_us scaled to the same rows")
    pk, c2, c2s, fp8 = state["dq"]
    t = _cpu_time(lambda: R.double_dequantize(pk, c2, c2s, (numel2,), 64, 256, fp8).to(torch.bfloat16))
    out["config2_decode"] = entry(t, codec_bytes, "gbs", gpu["codec_decode_s"] * frac if gpu.get("codec_decode_s") else None,
                                  f"{rows} of 11008 rows; gpu_us scaled to the same rows")
    del w2, state
    # config 4: q projection (4096 -> 4096) forward and dX at M = 2048, r = 64
    K4 = N4 = 4096
    w4 = torch.randn(N4, K4, generator=g) * 0.02
    p4, s4 = R.quantize_int4(w4, 64)
    a4 = (torch.rand(GEMM_RANK, K4, generator=g) * 2 - 1) / math.sqrt(K4)
    b4 = torch.randn(N4, GEMM_RANK, generator=g) * 0.01
    x4 = torch.randn(GEMM_M, K4, generator=g).to(torch.bfloat16)
    dy4 = (torch.randn(GEMM_M, N4, generator=g) * 1e-2).to(torch.bfloat16)
    sc4 = GEMM_ALPHA / GEMM_RANK
    fl = gemm_flops(GEMM_M, N4, K4, GEMM_RANK)
    t = _cpu_time(lambda: R.nf4_lora_linear(x4, p4, s4, None, a4, b4, sc4, N4, 64), runs=10)
    out["config4_q_fwd"] = entry(t, fl, "tflops", gpu.get("gemm_q_fwd_s"), "q projection only")
    t = _cpu_time(lambda: R.nf4_dx(dy4, p4, s4, N4, K4, a4, b4, sc4), runs=10)
    out["config4_q_dx"] = entry(t, fl, "tflops", gpu.get("gemm_q_dx_s"), "q projection only")
    del w4, p4, s4, x4, dy4
    # config 5: 1792 of the 28672 output rows, M = 1
    K5, N5, n5 = 8192, 28672, 1792
    w5 = (torch.randn(n5, K5, generator=g) * 0.02).to(torch.bfloat16)
    x5 = torch.randn(1, K5, generator=g).to(torch.bfloat16)
    q5, sc5 = R.quantize_int8(w5, per_channel=True)
    b5 = n5 * K5 + 4 * n5 + 2 * K5 + 2 * n5
    f = n5 / N5
    t = _cpu_time(lambda: R.int8_linear(x5, q5, sc5))
    out["config5_int8_m1"] = entry(t, b5, "gbs", gpu["int8_m1_s"] * f if gpu.get("int8_m1_s") else None,
                                   f"{n5} of {N5} rows; gpu_us scaled to the same rows")
    t = _cpu_time(lambda: R.fp8_linear(x5, w5))
    out["config5_fp8_m1"] = entry(t, b5, "gbs", gpu["fp8_m1_s"] * f if gpu.get("fp8_m1_s") else None,
                                  f"{n5} of {N5} rows, W quantized per call as the reference does; "
                                  f"gpu_us scaled to the same rows")
    del w5, x5, q5
    # optimizer: the PagedAdamW update on the adapters of 4 of the 32 layers
    shapes = lora_param_shapes(layers=4)
    ps = [torch.randn(sh, generator=g) * 0.02 for sh in shapes]
    gs = [torch.randn(sh, generator=g) * 1e-3 for sh in shapes]
    ms = [torch.zeros(sh) for sh in shapes]
    vs = [torch.zeros(sh) for sh in shapes]
    cnt = [0]

    def opt_step():
        cnt[0] += 1
        R.paged_adamw_step(ps, gs, ms, vs, [cnt[0]] * len(ps), lr=2e-4, weight_decay=0.01)
    n_opt = sum(a * b for a, b in shapes)
    t = _cpu_time(opt_step)
    f = 4 / ADAMW_LAYERS
    out["optimizer_adamw_step"] = entry(t, 28 * n_opt, "gbs",
                                        gpu["adamw_step_s"] * f if gpu.get("adamw_step_s") else None,
                                        f"LoRA adapters of 4 of the 32 Llama-3-8B layers ({n_opt} fp32 parameters), "
                                        f"the update alone (no host/device copies); gpu_us scaled to the same "
                                        f"parameters")
    return out, t3


def bench_config1(dev, stream):
    """Config 1 on the GPU: one NF4 QuantLinear 4096 -> 4096 with LoRA r = 16,
    alpha = 32 on fp32 activations (the fp32-MFMA path), M in {1, 16}; fp32
    weights N(0,0.02) quantized with block 64 and fp32 absmax, 20 replays of
    a graph of 60 calls over 60 weight copies (565 MB of codes and scales,
    past the 256 MB MALL)."""
    import torch
    from rocm_qlora import ops
    from rocm_qlora.quantization import quantize_int4
    K = N = 4096
    g = torch.Generator(device=dev).manual_seed(13)
    ws = []
    for _ in range(CONFIG1_COPIES):
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        p, s_ = quantize_int4(w, BLOCK)
        a = (torch.rand(RANK, K, generator=g, device=dev) * 2 - 1) / math.sqrt(K)
        b = torch.randn(N, RANK, generator=g, device=dev) * 0.01
        ws.append((p, s_, a, b))
        del w
    wbytes = len(ws) * (N * K // 2 + N * K // BLOCK * 4)
    out = {"workload": f"NF4 {K}x{N} fp32 activations, LoRA r={RANK} alpha={ALPHA}, block {BLOCK} fp32 absmax",
           "rotation": f"{len(ws)} weight copies, {wbytes / 1e6:.0f} MB of codes and scales"}
    for m in (1, 16):
        x = torch.randn(m, K, generator=g, device=dev)
        gr = _capture(lambda: [ops.nf4_linear(x, p, s_, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING)
                               for p, s_, a, b in ws], stream)
        with _Range(f"rq-config1 fp32 M={m}"):
            t = _time_graph_stats(gr, 20)
        del gr
        us = t["mean"] * 1e3 / len(ws)
        out[f"m{m}"] = {"us": round(us, 2), "gbs": round(gemv_bytes(m, N, K) / (us * 1e-6) / 1e9, 1),
                        "frac": round(gemv_bytes(m, N, K) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def bench_gemm(dev, stream):
    """Config: M = 2048 bf16 tokens N(0,1), LoRA r = 64, alpha = 16, dY
    N(0,1e-2); per-shape forward and dX graphs, 20 replays each."""
    import torch
    from rocm_qlora import ops
    layer = make_layer(dev, 4242, rank=GEMM_RANK)
    s = GEMM_ALPHA / GEMM_RANK
    g = torch.Generator(device=dev).manual_seed(11)
    xs = {K: torch.randn(GEMM_M, K, generator=g, device=dev).to(torch.bfloat16) for K in (4096, 14336)}
    per = {}
    tot = {"fwd": [0.0, 0.0], "dx": [0.0, 0.0]}
    for name, K, N in LLAMA3_8B_PROJ:
        packed, absmax, a, b, _, _ = layer[name]
        dy = (torch.randn(GEMM_M, N, generator=g, device=dev) * 1e-2).to(torch.bfloat16)
        x = xs[K]
        gf = _capture(lambda: ops.nf4_linear(x, packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=s),
                      stream)
        gd = _capture(lambda: ops.nf4_linear_dx(dy, packed, absmax, K, BLOCK, lora_a=a, lora_b=b, scaling=s),
                      stream)
        fl = gemm_flops(GEMM_M, N, K, GEMM_RANK)
        with _Range(f"rq-gemm-fwd {name} M={GEMM_M} K={K} N={N}"):
            ms_f = _time_graph(gf, 20)
        with _Range(f"rq-gemm-dx {name} M={GEMM_M} K={K} N={N}"):
            ms_d = _time_graph(gd, 20)
        per[name] = {"fwd_us": round(ms_f * 1e3, 2), "fwd_tflops": round(fl / ms_f / 1e9, 1),
                     "dx_us": round(ms_d * 1e3, 2), "dx_tflops": round(fl / ms_d / 1e9, 1)}
        tot["fwd"][0] += fl
        tot["fwd"][1] += ms_f
        tot["dx"][0] += fl
        tot["dx"][1] += ms_d
        del gf, gd, dy
    fwd = tot["fwd"][0] / tot["fwd"][1] / 1e9
    dx = tot["dx"][0] / tot["dx"][1] / 1e9
    return {"workload": f"Llama-3-8B 7 NF4 projections, M={GEMM_M} bf16, LoRA r={GEMM_RANK} alpha={GEMM_ALPHA} "
                        f"fused, forward Y and backward dX",
            "fwd_tflops": round(fwd, 1), "fwd_frac": round(fwd / BF16_PEAK_TFLOPS, 4),
            "dx_tflops": round(dx, 1), "dx_frac": round(dx / BF16_PEAK_TFLOPS, 4),
            "peak_tflops": BF16_PEAK_TFLOPS, "per_shape": per}


def bench_codec(dev, stream):
    """NF4 + double quantization of the down-projection weight (11008 x 4096
    bf16, 0.1 % outliers at +-8 sigma), blocks 64 / 256, over CODEC_COPIES
    weight copies (each call encodes or decodes all of them, 565 MB, past the
    256 MB MALL), 10 graph replays each way.  Algorithmic bytes (each way,
    per copy): 2 numel (bf16 W) + numel / 2 (packed) + numel / 64 (c2 codes)
    + 4 numel / 16384 (c2 scales)."""
    import torch
    from rocm_qlora.quantization import quantize_int4
    from rocm_qlora.quantization.double_quant import dq_quantize_absmax, dq_dequantize_to
    N, K = 11008, 4096
    numel = N * K
    g = torch.Generator(device=dev).manual_seed(5)
    ws = []
    for _ in range(CODEC_COPIES):
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        n_out = numel // 1000
        idx = torch.randperm(numel, generator=g, device=dev)[:n_out]
        sign = torch.randint(0, 2, (n_out,), generator=g, device=dev).float() * 2 - 1
        w.view(-1)[idx] = sign * 0.16
        ws.append(w.to(torch.bfloat16))
        del w, idx, sign
    states = [{} for _ in ws]

    def encode():
        for w, st in zip(ws, states):
            packed, c1 = quantize_int4(w, 64)
            c2, c2s = dq_quantize_absmax(c1, 256, True)
            st.update(packed=packed, c2=c2, c2s=c2s)

    encode()
    ge = _capture(encode, stream)
    codes = [(st["packed"], st["c2"], st["c2s"]) for st in states]
    gd = _capture(lambda: [dq_dequantize_to(p, c2, c2s, 64, 256, True, torch.bfloat16, numel)
                           for p, c2, c2s in codes], stream)
    nbytes = 2 * numel + numel // 2 + numel // 64 + 4 * numel // 16384
    with _Range(f"rq-codec encode {N}x{K} x{CODEC_COPIES}"):
        ms_e = _time_graph(ge, 10) / CODEC_COPIES
    with _Range(f"rq-codec decode {N}x{K} x{CODEC_COPIES}"):
        ms_d = _time_graph(gd, 10) / CODEC_COPIES
    del ge, gd
    enc, dec = nbytes / ms_e / 1e6, nbytes / ms_d / 1e6
    return {"workload": f"NF4 + double quantization (blocks 64/256, fp8 c2) of a {N}x{K} bf16 weight with "
                        f"0.1% outliers at +-8 sigma",
            "rotation": f"{CODEC_COPIES} weight copies, {CODEC_COPIES * nbytes / 1e6:.0f} MB per pass",
            "bytes": nbytes, "encode_us": round(ms_e * 1e3, 2), "encode_gbs": round(enc, 1),
            "encode_frac": round(enc / HBM_PEAK_GBS, 4), "decode_us": round(ms_d * 1e3, 2),
            "decode_gbs": round(dec, 1), "decode_frac": round(dec / HBM_PEAK_GBS, 4)}


def bench_int8_codec(w, qs, stream):
    """INT8 weight codec on one bf16 weight: per-row quantization (bytes: 2
    numel read, numel codes + 2 N scales written) and its fp32 reconstruction
    (numel codes + 2 N scales read, 4 numel written), 10 graph replays each."""
    from rocm_qlora.quantization import dequantize_int8, quantize_int8
    N, K = w.shape
    q, s = qs
    gq = _capture(lambda: quantize_int8(w, per_channel=True), stream)
    with _Range(f"rq-int8-codec quantize {N}x{K}"):
        tq = _time_graph(gq, 10)
    del gq
    gd = _capture(lambda: dequantize_int8(q, s), stream)
    with _Range(f"rq-int8-codec dequantize {N}x{K}"):
        td = _time_graph(gd, 10)
    del gd
    bq = 3 * N * K + 2 * N
    bd = 5 * N * K + 2 * N
    return {"workload": f"per-row INT8 quantize / fp32 dequantize of a {N}x{K} bf16 weight",
            "quantize_us": round(tq * 1e3, 2), "quantize_gbs": round(bq / tq / 1e6, 1),
            "quantize_frac": round(bq / tq / 1e6 / HBM_PEAK_GBS, 4),
            "dequantize_us": round(td * 1e3, 2), "dequantize_gbs": round(bd / td / 1e6, 1),
            "dequantize_frac": round(bd / td / 1e6 / HBM_PEAK_GBS, 4)}


def bench_byte_linears(dev, stream):
    """INT8 per-row-absmax (W8A16 on bf16 MFMA; W8A8 on int8 MFMA) and FP8 (e4m3, fp8 MFMA)
    linears at 8192 -> 28672 with
    bf16 activations N(0,1), weights N(0,0.02); M = 1 rotates two weight
    copies (470 MB each kind, past the MALL), M = 512 and 4096 one copy."""
    import torch
    from rocm_qlora import ops
    from rocm_qlora.quantization import quantize_int8
    K, N = 8192, 28672
    g = torch.Generator(device=dev).manual_seed(9)
    int8_w, fp8_w = [], []
    out = {}
    for c in range(2):
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        int8_w.append(quantize_int8(w, per_channel=True))
        if c == 0:
            out["int8_codec"] = bench_int8_codec(w, int8_w[0], stream)
        codes, scale = ops.fp8_quantize(w)
        fp8_w.append((ops.fp8_to_e4m3fn(codes), scale))  # as FP8LinearWrapper caches it
        del codes
        del w
    for M in (1, 512, 4096):
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        copies = 2 if M == 1 else 1
        for kind in ("int8", "int8_w8a8", "fp8"):
            if kind == "int8":
                fn = lambda: [ops.int8_linear(x, q, s, N) for q, s in int8_w[:copies]]
            elif kind == "int8_w8a8":
                fn = lambda: [ops.int8_linear_w8a8(x, q, s) for q, s in int8_w[:copies]]
            else:
                fn = lambda: [ops.fp8_linear(x, cw, sc) for cw, sc in fp8_w[:copies]]
            gr = _capture(fn, stream)
            with _Range(f"rq-{kind}-linear M={M} K={K} N={N}"):
                t = _time_graph_stats(gr, 20)
            del gr
            us = t["mean"] * 1e3 / copies
            pct = {"p10_us": round(t["p10"] * 1e3 / copies, 2), "p90_us": round(t["p90"] * 1e3 / copies, 2)}
            if M == 1:
                nb = N * K + 4 * N + 2 * M * K + 2 * M * N
                gbs = nb / us / 1e3
                out[f"{kind}_m{M}"] = {"us": round(us, 2), "gbs": round(gbs, 1),
                                        "frac": round(gbs / HBM_PEAK_GBS, 4), "bound": "hbm", **pct}
            else:
                tf = 2 * M * N * K / us / 1e6
                peak, bound = {"int8": (BF16_PEAK_TFLOPS, "bf16 mfma"),
                               "int8_w8a8": (INT8_PEAK_TOPS, "int8 mfma"),
                               "fp8": (FP8_PEAK_TFLOPS, "fp8 mfma")}[kind]
                out[f"{kind}_m{M}"] = {"us": round(us, 2), "tflops": round(tf, 1),
                                        "frac": round(tf / peak, 4), "bound": bound, **pct}
        if M == 512:
            # what the activation rounding of W8A8 costs against the W8A16 path
            q, s = int8_w[0]
            ref = ops.int8_linear(x, q, s, N).float()
            d = (ops.int8_linear_w8a8(x, q, s).float() - ref).norm() / ref.norm()
            out["int8_w8a8_rel_dev_vs_w8a16"] = round(float(d), 5)
        del x
    return {"workload": f"INT8 per-row (W8A16 and W8A8) and FP8 per-tensor linears, K={K} N={N}, "
                        "bf16 activations", **out}


ADAMW_LAYERS = 32  # Llama-3-8B


def lora_param_shapes(layers=ADAMW_LAYERS, rank=RANK):
    """LoRA A [r, K] and B [N, r] of the seven projections of `layers` layers."""
    out = []
    for _ in range(layers):
        for _, K, N in LLAMA3_8B_PROJ:
            out += [(rank, K), (N, rank)]
    return out


def bench_optimizer(dev, stream):
    """The fused AdamW step (rq_adamw_step behind PagedAdamW) over the LoRA
    adapters of a whole Llama-3-8B: r = 16 on the seven projections of 32
    layers, 448 fp32 tensors, 41.9 M parameters, gradients N(0, 1e-3);
    algorithmic bytes 28 per parameter (p, m, v read and written, g read).
    `kernel_us`: back-to-back rq_adamw_step calls (a 32 KB descriptor copy and
    one launch each), HIP events on the launch stream, mean of 50;
    `step_resident_ms` / `step_offload_ms`: wall time of PagedAdamW.step()
    with the states resident in HBM / in pinned host memory paged through
    256 MB device pages (the reference's memory behaviour; PCIe-bound),
    median of 20 and 5."""
    import torch
    from rocm_qlora import _native as nat
    from rocm_qlora.optim import PagedAdamW
    shapes = lora_param_shapes()
    n_params = sum(a * b for a, b in shapes)
    nbytes = 28 * n_params
    g = torch.Generator(device=dev).manual_seed(77)
    params = [torch.nn.Parameter(torch.randn(s, generator=g, device=dev) * 0.02) for s in shapes]
    for p in params:
        p.grad = torch.randn(p.shape, generator=g, device=dev) * 1e-3
    out = {"workload": f"AdamW step over Llama-3-8B LoRA adapters (r={RANK}, 7 projections x "
                       f"{ADAMW_LAYERS} layers, {len(shapes)} fp32 tensors)",
           "params": n_params, "bytes_per_step": nbytes}
    with torch.cuda.stream(stream):
        opt = PagedAdamW(params, lr=2e-4, weight_decay=0.01, offload_states=False)
        opt.step()
        table, keep, _ = opt._table(dev)
        nch = opt._total // 2048
        call = lambda: nat.call("rq_adamw_step", table.ctypes.data, len(table), opt._dev_table.data_ptr(),
                                opt._dev_table.numel(), 0, nch, opt._m.data_ptr(), opt._v.data_ptr(),
                                stream.cuda_stream)
        for _ in range(5):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 50
        e0.record(stream)
        for _ in range(reps):
            call()
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        gbs = nbytes / us / 1e3
        out.update({"kernel_us": round(us, 2), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
        t = []
        for _ in range(20):
            stream.synchronize()
            t0 = time.perf_counter()
            opt.step()
            stream.synchronize()
            t.append(time.perf_counter() - t0)
        t.sort()
        out["step_resident_ms"] = round(t[len(t) // 2] * 1e3, 3)
        del opt, keep
        opt = PagedAdamW(params, lr=2e-4, weight_decay=0.01, offload_states=True, page_size_mb=256)
        opt.step()
        t = []
        for _ in range(5):
            t0 = time.perf_counter()
            opt.step()  # ends with a synchronization, as the reference's step
            t.append(time.perf_counter() - t0)
        t.sort()
        out["step_offload_ms"] = round(t[len(t) // 2] * 1e3, 3)
        out["offload_pcie_gbs"] = round(16 * n_params / t[len(t) // 2] / 1e9, 1)
    del opt, params
    return out


def _short(name, n=70):
    return name if len(name) <= n else name[:n - 3] + "..."


def summarize_profile(path):
    """From a rocprofv3 CSV trace (`-f csv`): count / average / min kernel
    duration per (kernel, grid), and, when a marker trace is present, per
    kernel inside each of bench.py's named ranges (rq-...), which is how the
    roofline launches are told apart from the other launches of the same
    kernel."""
    files = glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        sys.exit(f"no *kernel_trace.csv under {path}")
    launches = []
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                launches.append((row["Kernel_Name"], int(row.get("Grid_Size_X", row.get("Grid_Size", 0)) or 0),
                                 int(row.get("Workgroup_Size_X", row.get("Workgroup_Size", 0)) or 0),
                                 int(row["Start_Timestamp"]), int(row["End_Timestamp"])))
    groups = {}
    for name, gx, wx, t0, t1 in launches:
        groups.setdefault((name, gx, wx), []).append((t1 - t0) / 1e3)
    print(f"{'kernel':<70} {'grid_x':>9} {'wg_x':>5} {'n':>6} {'avg_us':>10} {'min_us':>10}")
    for (name, gx, wx), ds in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        print(f"{_short(name):<70} {gx:>9} {wx:>5} {len(ds):>6} {sum(ds) / len(ds):>10.2f} {min(ds):>10.2f}")
    ranges = []
    for f in glob.glob(os.path.join(path, "**", "*marker_api_trace.csv"), recursive=True):
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                msg = row.get("Function", "") or row.get("Message", "")
                if msg.startswith("rq-"):
                    ranges.append((msg, int(row["Start_Timestamp"]), int(row["End_Timestamp"])))
    if ranges:
        print()
        print(f"{'range / kernel':<70} {'n':>6} {'avg_us':>10} {'min_us':>10} {'sum_us':>10}")
        for msg, r0, r1 in sorted(ranges, key=lambda r: r[1]):
            print(msg)
            per = {}
            for name, gx, wx, t0, t1 in launches:
                if r0 <= t0 <= r1:
                    per.setdefault(name, []).append((t1 - t0) / 1e3)
            for name, ds in sorted(per.items(), key=lambda kv: -sum(kv[1])):
                print(f"  {_short(name, 68):<68} {len(ds):>6} {sum(ds) / len(ds):>10.2f} {min(ds):>10.2f} "
                      f"{sum(ds):>10.1f}")


def run_counters_kernel(which, reps=4):
    """Eager launches of one MFMA kernel for counter passes (rocprofv3 --pmc):
    "fp8_gemm" -- the FP8 linear at M = 4096, K = 8192, N = 28672 (weights
    N(0,0.02) quantized per tensor, e4m3fn codes cached); "int8_gemm" -- the
    W8A8 INT8 linear at the same shape (weights quantized per row);
    "nf4_gemm" -- the
    NF4 forward and dX at the gate shape, M = 2048, K = 4096, N = 14336, LoRA
    r = 64, alpha = 16."""
    import torch
    from rocm_qlora import ops
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(9)
    if which == "fp8_gemm":
        K, N, M = 8192, 28672, 4096
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        codes, scale = ops.fp8_quantize(w)
        wf = ops.fp8_to_e4m3fn(codes)
        del w, codes
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        for _ in range(reps):
            ops.fp8_linear(x, wf, scale)
    elif which == "int8_gemm":
        from rocm_qlora.quantization import quantize_int8
        K, N, M = 8192, 28672, 4096
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q, s = quantize_int8(w, per_channel=True)
        del w
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        for _ in range(reps):
            ops.int8_linear_w8a8(x, q, s)
    else:
        layer = make_layer(dev, 4242, rank=GEMM_RANK)
        packed, absmax, a, b, N, K = layer["gate"]
        x = torch.randn(GEMM_M, K, generator=g, device=dev).to(torch.bfloat16)
        dy = (torch.randn(GEMM_M, N, generator=g, device=dev) * 1e-2).to(torch.bfloat16)
        s = GEMM_ALPHA / GEMM_RANK
        for _ in range(reps):
            ops.nf4_linear(x, packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=s)
            ops.nf4_linear_dx(dy, packed, absmax, K, BLOCK, lora_a=a, lora_b=b, scaling=s)
    torch.cuda.synchronize()
    print(f"counters: {reps} rounds of {which}", flush=True)


def run_counters(reps=4):
    """Eager launches for counter collection: one plain device copy of
    COPY_BYTES (calibration: its FETCH_SIZE / WRITE_SIZE readings against the
    bytes it must move), then the decode GEMV for each (shape, LoRA, M) of
    GEMV_COUNTER_CONFIGS in turn -- the gate/up shape (K = 4096, N = 14336)
    over the gate and up weights of six layer copies, the k/v shape (K =
    4096, N = 1024) over the k and v weights, plain and with the LoRA term
    fused (r = 16), at M = 1 and 16 -- `reps` rounds over the 12 weights
    each, so every launch reads its weights from HBM (past the 256 MB
    MALL)."""
    import torch
    from rocm_qlora import ops
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    layers = [make_layer(dev, 1000 + c) for c in range(6)]
    xs = {m: torch.randn(m, 4096, device=dev).to(torch.bfloat16) for m in sorted({c[2] for c in GEMV_COUNTER_CONFIGS})}
    src = torch.randint(0, 255, (COPY_BYTES,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    names = {"gate": ("gate", "up"), "k": ("k", "v")}
    for shape, lora, m in GEMV_COUNTER_CONFIGS:
        x = xs[m]
        ws = [layer[nm] for layer in layers for nm in names[shape]]
        for _ in range(reps):
            for packed, absmax, a, b, N, K in ws:
                if lora:
                    ops.nf4_linear(x, packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING)
                else:
                    ops.nf4_linear(x, packed, absmax, N, BLOCK)
        torch.cuda.synchronize()
        print(f"counters: {reps * len(ws)} launches {shape} {'lora' if lora else 'plain'} M={m}", flush=True)
    print(f"counters: copy {COPY_BYTES} B, then {GEMV_COUNTER_CONFIGS}", flush=True)


def summarize_counters(paths):
    """Per-kernel mean of each counter over the dispatches in rocprofv3 CSV
    counter files (`-f csv`).  For a `--counters gemv` run, also per (shape,
    mode, M) of GEMV_COUNTER_CONFIGS: the dispatches after the calibration copy
    are taken in dispatch order, the library's kernels only (a LoRA operand
    kernel counts with the GEMV launch that follows it), and each counter's
    mean per launch printed; FETCH_SIZE and WRITE_SIZE (KiB per dispatch)
    become HBM bytes per launch by dividing by what the same counter reads
    per byte for the calibration copy, printed as the table rows
    profiled_traffic reads."""
    files = []
    for p in paths:
        files += glob.glob(os.path.join(p, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        sys.exit(f"no *counter_collection.csv under {paths}")
    per = {}   # (kernel, counter) -> {dispatch: value}
    seq = {}   # file -> {dispatch id: (kernel, {counter: value})}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                key = (row["Kernel_Name"], row["Counter_Name"])
                d = per.setdefault(key, {})
                did = int(row.get("Dispatch_Id", row.get("Correlation_Id")) or 0)
                d[(f, did)] = d.get((f, did), 0.0) + float(row["Counter_Value"])
                ent = seq.setdefault(f, {}).setdefault(did, (row["Kernel_Name"], {}))
                ent[1][row["Counter_Name"]] = ent[1].get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    for (kname, cname), d in sorted(per.items()):
        vals = list(d.values())
        print(f"{_short(kname):<70} {cname:<24} n={len(vals):<4} mean={sum(vals) / len(vals):.1f}")
    # per (shape, mode) of the gemv run
    acc = {}    # (config index, counter) -> [sum, launches]
    factor = {}
    for f, disp in seq.items():
        order = sorted(disp.items())
        copies = [i for i, (_, (k, _)) in enumerate(order) if "copy" in k.lower()]
        if not copies:
            continue
        i0 = copies[-1]
        for cname, v in order[i0][1][1].items():
            factor[cname] = v * 1024.0 / COPY_BYTES
        gemv, pending = 0, {}
        launches = [(k, c) for _, (k, c) in order[i0 + 1:] if "rq::" in k or k.startswith("_ZN2rq")]
        n_gemv = sum(1 for k, _ in launches if "nf4_gemv_kernel" in k)
        per_cfg = n_gemv // len(GEMV_COUNTER_CONFIGS) if n_gemv else 0
        for k, c in launches:
            for cname, v in c.items():
                pending[cname] = pending.get(cname, 0.0) + v
            if "nf4_gemv_kernel" not in k:
                continue
            ci = min(gemv // per_cfg, len(GEMV_COUNTER_CONFIGS) - 1) if per_cfg else 0
            for cname, v in pending.items():
                a = acc.setdefault((ci, cname), [0.0, 0])
                a[0] += v
                a[1] += 1
            pending = {}
            gemv += 1
    if not acc:
        return
    print()
    shapes = {"gate": (4096, 14336), "k": (4096, 1024)}
    counters = sorted({c for _, c in acc})
    print("| config | " + " | ".join(counters) + " |")
    for ci, (shape, lora, m) in enumerate(GEMV_COUNTER_CONFIGS):
        cells = []
        for cname in counters:
            a = acc.get((ci, cname))
            cells.append(f"{a[0] / a[1]:,.0f}" if a else "-")
        print(f"| {shape} {'lora' if lora else 'plain'} M={m} | " + " | ".join(cells) + " |")
    if "FETCH_SIZE" in factor and "WRITE_SIZE" in factor:
        print()
        print(f"calibration: FETCH_SIZE factor {factor['FETCH_SIZE']:.4f}, WRITE_SIZE factor "
              f"{factor['WRITE_SIZE']:.4f} (counter bytes per copied byte)")
        print("| kernel | shape | mode | M | K | N | fetch B | write B | total B | algorithmic B | ratio |")
        print("|---|---|---|---|---|---|---|---|---|---|---|")
        for ci, (shape, lora, m) in enumerate(GEMV_COUNTER_CONFIGS):
            fe, wr = acc.get((ci, "FETCH_SIZE")), acc.get((ci, "WRITE_SIZE"))
            if not fe or not wr:
                continue
            K, N = shapes[shape]
            fb = fe[0] / fe[1] * 1024.0 / factor["FETCH_SIZE"]
            wb = wr[0] / wr[1] * 1024.0 / factor["WRITE_SIZE"]
            alg = gemv_bytes(m, N, K) if lora else kernel_bytes(m, N, K)
            print(f"| nf4_gemv_kernel | {shape} | {'lora' if lora else 'plain'} | {m} | {K} | {N} | {fb:,.0f} | "
                  f"{wb:,.0f} | {fb + wb:,.0f} | {alg:,} | {(fb + wb) / alg:.3f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--m", type=int, default=1, help="decode tokens per step (activation rows)")
    ap.add_argument("--no-gemm", action="store_true", help="skip the M=2048 GEMM section")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the codec and INT8/FP8 sections")
    ap.add_argument("--summarize-profile", metavar="DIR", help="summarize a rocprofv3 CSV kernel trace and exit")
    ap.add_argument("--counters", nargs="?", const="gemv", choices=["gemv", "fp8_gemm", "int8_gemm", "nf4_gemm"],
                    help="short eager run for rocprofv3 --pmc passes (default: the roofline GEMV and a copy)")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="HBM bytes per launch from rocprofv3 --pmc CSV output and exit")
    args = ap.parse_args()
    if args.summarize_profile:
        summarize_profile(args.summarize_profile)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.counters:
        if args.counters == "gemv":
            run_counters()
        else:
            run_counters_kernel(args.counters)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path is built and measured on a single MI355X; "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    from rocm_qlora import ops
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    M = args.m
    print(f"bench: decode GEMV M={M}", file=sys.stderr, flush=True)

    layer_bytes = sum(N * K // 2 + (N * K // BLOCK) * 4 for _, K, N in LLAMA3_8B_PROJ)
    n_copies = max(2, math.ceil(520e6 / layer_bytes / 2) * 2)
    layers = [make_layer(dev, 1000 + c) for c in range(n_copies)]
    gx = torch.Generator(device=dev).manual_seed(7)
    stream = torch.cuda.Stream()

    def decode_graphs(m):
        xs = {K: torch.randn(m, K, generator=gx, device=dev).to(torch.bfloat16) for K in (4096, 14336)}

        def step(layer):
            for name, K, N in LLAMA3_8B_PROJ:
                packed, absmax, a, b, _, _ = layer[name]
                ops.nf4_linear(xs[K], packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING)

        return xs, [_capture(lambda L=layer: step(L), stream) for layer in layers]

    def time_steps(graphs, steps, warmup):
        """`steps` back-to-back step replays (rotating layer copies) between
        two synchronizations, timed by an event before and after them (total
        ms); then the same number again with an event after each step (the
        per-step ms, sorted, for percentiles: recording those events adds
        about 4 us to each step, so they are kept out of the total)."""
        for i in range(warmup):
            graphs[i % n_copies].replay()
        torch.cuda.synchronize()
        cur = torch.cuda.current_stream()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(cur)
        for i in range(steps):
            graphs[i % n_copies].replay()
        t1.record(cur)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record(cur)
        for i in range(steps):
            graphs[i % n_copies].replay()
            ev[i + 1].record(cur)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1), sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))

    xs, graphs = decode_graphs(M)
    with _Range("rq-decode-step"):
        total_ms, per = time_steps(graphs, args.steps, args.warmup)
    ms_step = total_ms / args.steps
    step_bytes = sum(gemv_bytes(M, N, K) for _, K, N in LLAMA3_8B_PROJ)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    step_pct = {"p10_us": round(_pct(per, 10) * 1e3, 2), "p50_us": round(_pct(per, 50) * 1e3, 2),
                "p90_us": round(_pct(per, 90) * 1e3, 2)}
    del graphs

    # the other decode batch sizes of the configuration (M in {1, 4, 8, 16})
    decode_m = {}
    for m in (1, 4, 8, 16):
        if m == M:
            continue
        _, gm = decode_graphs(m)
        with _Range(f"rq-decode-step M={m}"):
            tm, pm = time_steps(gm, 50, 10)
        b = sum(gemv_bytes(m, N, K) for _, K, N in LLAMA3_8B_PROJ)
        decode_m[f"m{m}"] = {"us_per_step": round(tm / 50 * 1e3, 2), "gbs": round(b / (tm / 50 * 1e-3) / 1e9, 1),
                             "frac": round(b / (tm / 50 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "p10_us": round(_pct(pm, 10) * 1e3, 2), "p90_us": round(_pct(pm, 90) * 1e3, 2)}
        del gm
    print("bench: decode " + ", ".join(f"{k} {v['us_per_step']} us" for k, v in decode_m.items()),
          file=sys.stderr, flush=True)

    # per projection at M: launches of one shape over every layer copy, with
    # and without the fused LoRA term, beside a minimal launch (a 4-byte fill)
    per_shape = {}
    tiny = torch.zeros(1, device=dev)
    gt = _capture(lambda: [tiny.zero_() for _ in range(n_copies)], stream)
    with _Range("rq-minimal-launch"):
        t_min = _time_graph_stats(gt, 20)
    del gt
    for name, K, N in LLAMA3_8B_PROJ:
        ws = [layer[name] for layer in layers]
        x = xs[K]
        gl = _capture(lambda: [ops.nf4_linear(x, p, s_, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING)
                               for p, s_, a, b, _, _ in ws], stream)
        gp = _capture(lambda: [ops.nf4_linear(x, p, s_, N, BLOCK) for p, s_, _, _, _, _ in ws], stream)
        with _Range(f"rq-shape {name} lora M={M} K={K} N={N}"):
            tl = _time_graph_stats(gl, 20)
        with _Range(f"rq-shape {name} plain M={M} K={K} N={N}"):
            tp = _time_graph_stats(gp, 20)
        del gl, gp
        nl = len(ws)
        per_shape[name] = {"lora_us": round(tl["mean"] * 1e3 / nl, 2), "plain_us": round(tp["mean"] * 1e3 / nl, 2),
                           "lora_gbs": round(gemv_bytes(M, N, K) / (tl["mean"] * 1e-3 / nl) / 1e9, 1),
                           "plain_gbs": round(kernel_bytes(M, N, K) / (tp["mean"] * 1e-3 / nl) / 1e9, 1)}
    per_shape["minimal_launch_us"] = round(t_min["mean"] * 1e3 / n_copies, 2)

    # roofline of the dominant kernel as the step runs it: the GEMV at the
    # gate/up shape with the LoRA term fused (and, beside it, plain)
    K, N = 4096, 14336
    roof_w = [layer[nm][:4] for layer in layers for nm in ("gate", "up")]
    x_roof = xs[K]

    def roof_pass(lora):
        for packed, absmax, a, b in roof_w:
            if lora:
                ops.nf4_linear(x_roof, packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING)
            else:
                ops.nf4_linear(x_roof, packed, absmax, N, BLOCK)

    # 150 replays (1800 launches): single batches of a few replays vary by
    # +-5 % from one to the next on the same machine
    reps = 150
    rg = _capture(lambda: roof_pass(True), stream)
    with _Range(f"rq-roofline nf4_gemv_kernel lora M={M} K={K} N={N}"):
        us_launch = _time_graph(rg, reps) * 1e3 / len(roof_w)
    del rg
    rg = _capture(lambda: roof_pass(False), stream)
    with _Range(f"rq-roofline nf4_gemv_kernel plain M={M} K={K} N={N}"):
        us_plain = _time_graph(rg, reps) * 1e3 / len(roof_w)
    del rg
    kb = gemv_bytes(M, N, K)
    achieved = kb / (us_launch * 1e-6) / 1e9
    print(f"bench: decode {ms_step * 1e3:.1f} us/step, {value:.0f} GB/s; gate/up GEMV {us_launch:.2f} us",
          file=sys.stderr, flush=True)

    gpu_s = {"decode_step_s": ms_step * 1e-3}
    cfg1 = bench_config1(dev, stream)
    for k, v in cfg1.items():
        if isinstance(v, dict):
            gpu_s[f"config1_{k}_s"] = v["us"] * 1e-6

    gemm = None
    if not args.no_gemm:
        del layers
        torch.cuda.empty_cache()
        gemm = bench_gemm(dev, stream)
        print(f"bench: GEMM fwd {gemm['fwd_tflops']} TF/s, dX {gemm['dx_tflops']} TF/s", file=sys.stderr,
              flush=True)
        gpu_s["gemm_q_fwd_s"] = gemm["per_shape"]["q"]["fwd_us"] * 1e-6
        gpu_s["gemm_q_dx_s"] = gemm["per_shape"]["q"]["dx_us"] * 1e-6
        layer0 = make_layer(dev, 1000)
    else:
        layer0 = layers[0]

    codec = byte = optim = None
    if not args.no_extra:
        codec = bench_codec(dev, stream)
        print(f"bench: codec encode {codec['encode_gbs']} GB/s, decode {codec['decode_gbs']} GB/s",
              file=sys.stderr, flush=True)
        gpu_s["codec_encode_s"] = codec["encode_us"] * 1e-6
        gpu_s["codec_decode_s"] = codec["decode_us"] * 1e-6
        torch.cuda.empty_cache()
        byte = bench_byte_linears(dev, stream)
        print("bench: byte linears " + ", ".join(f"{k} {v['us']} us" for k, v in byte.items()
                                                  if isinstance(v, dict) and "us" in v), file=sys.stderr, flush=True)
        ic = byte["int8_codec"]
        print(f"bench: int8 codec quantize {ic['quantize_gbs']} GB/s, dequantize {ic['dequantize_gbs']} GB/s",
              file=sys.stderr, flush=True)
        gpu_s["int8_m1_s"] = byte["int8_m1"]["us"] * 1e-6
        gpu_s["fp8_m1_s"] = byte["fp8_m1"]["us"] * 1e-6
        torch.cuda.empty_cache()
        optim = bench_optimizer(dev, stream)
        print(f"bench: AdamW step {optim['kernel_us']} us ({optim['gbs']} GB/s), resident step "
              f"{optim['step_resident_ms']} ms, offloaded step {optim['step_offload_ms']} ms",
              file=sys.stderr, flush=True)
        gpu_s["adamw_step_s"] = optim["kernel_us"] * 1e-6
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        layer_cpu = {nm: tuple(t.cpu() if torch.is_tensor(t) else t for t in v) for nm, v in layer0.items()}
        xs_cpu = {k: v.cpu() for k, v in xs.items()}
        configs, t3 = cpu_baselines(layer_cpu, xs_cpu, M, gpu_s)
        cpu = {"value": round(step_bytes / t3["median"] / 1e9, 3), "unit": "GB/s",
               "cores": configs["threads"], "kind": "port",
               "sample": f"whole decode steps of one 7-projection Llama-3-8B layer (M={M}, LoRA r={RANK}) "
                         f"through the oracle's torch CPU restatement of dequantize_int4 -> .to(bf16) -> "
                         f"F.linear + LoRA; median of 10 after 2 warm-ups, "
                         f"{t3['median'] * 1e3:.1f} ms/step; {configs['threads']} threads of "
                         f"{configs['os_cpu_count']} cores ({configs['cpu_model']})",
               "configs": configs}
        print(f"bench: cpu decode step {t3['median'] * 1e3:.1f} ms", file=sys.stderr, flush=True)

    traffic = profiled_traffic("gate", "lora", M, K, N)
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"Llama-3-8B decoder layer, 7 NF4 projections, decode dequant-GEMV "
                               f"M={M}, LoRA r={RANK} fused, block {BLOCK} fp32 absmax",
                   "tokens": M, "layer_copies": n_copies, "step_bytes": step_bytes, **step_pct},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "nf4_gemv_kernel", "mode": f"LoRA r={RANK} fused",
                     "shape": f"M={M} K={K} N={N}", "bytes_per_launch": kb,
                     "us_per_launch": round(us_launch, 3),
                     "plain": {"us_per_launch": round(us_plain, 3), "bytes_per_launch": kernel_bytes(M, N, K),
                               "frac": round(kernel_bytes(M, N, K) / (us_plain * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                               "traffic": profiled_traffic("gate", "plain", M, K, N)}},
        "decode_m": decode_m,
        "decode_per_shape": per_shape,
        "config1": cfg1,
        "gemm": gemm,
        "codec": codec,
        "byte_linears": byte,
        "optimizer": optim,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
