#!/usr/bin/env python3
"""Benchmark of the MI355X NF4 quantized-linear path at Llama-3-8B projection shapes.

One step is one Llama-3-8B decoder layer's seven NF4 projections (q, k, v,
o, gate, up, down; in x out = 4096x4096, 4096x1024 twice, 4096x4096,
4096x14336 twice, 14336x4096) run as decode dequant-GEMVs with the LoRA term
fused (M = 1 token, bf16 activations, NF4 block 64 with fp32 absmax, LoRA
r = 16, alpha = 32).  `value` is the whole step's algorithmic HBM bytes
divided by its time, with every input resident in HBM.  Weights rotate over
enough layer copies (> 512 MB) that the 256 MB MALL cannot serve them.  The
step is captured once per layer copy as a HIP graph and replayed.

Alongside: the roofline of the dominant kernel (the GEMV at the gate/up
shape, timed with HIP events over back-to-back launches on the stream it
runs on), and the CPU baseline: the oracle's restatement of the reference's
CPU path (dequantize_int4 -> .to(bf16) -> F.linear + LoRA) over a bounded
sample of the same step on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rocm-qlora_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA

# (name, in_features K, out_features N)
LLAMA3_8B_PROJ = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
                  ("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096)]
RANK, ALPHA, BLOCK = 16, 32, 64
SCALING = ALPHA / RANK


def gemv_bytes(M, N, K, rank=RANK, scale_bytes=4):
    """Algorithmic HBM bytes of one fused NF4 LoRA linear: packed codes, absmax,
    activations in and out, LoRA A and B (bf16 accounting)."""
    return N * K // 2 + (N * K // BLOCK) * scale_bytes + M * K * 2 + M * N * 2 + (rank * K + N * rank) * 2


def kernel_bytes(M, N, K, scale_bytes=4):
    """Algorithmic bytes of one plain GEMV launch (no LoRA)."""
    return N * K // 2 + (N * K // BLOCK) * scale_bytes + M * K * 2 + M * N * 2


def make_layer(dev, seed):
    import torch
    from rocm_qlora.quantization import quantize_int4
    g = torch.Generator(device=dev).manual_seed(seed)
    layer = {}
    for name, K, N in LLAMA3_8B_PROJ:
        w = torch.randn(N, K, generator=g, device=dev) * 0.02
        packed, absmax = quantize_int4(w, BLOCK)
        del w
        a = (torch.rand(RANK, K, generator=g, device=dev) * 2 - 1) / math.sqrt(K)  # kaiming_uniform(a=sqrt 5)
        b = torch.randn(N, RANK, generator=g, device=dev) * 0.01
        layer[name] = (packed, absmax, a, b, N, K)
    return layer


def cpu_baseline(layer_cpu, xs_cpu, budget_s=20.0):
    """The oracle's CPU restatement of the reference path over whole decode
    steps, as many as fit in about budget_s (at least one)."""
    import torch
    from oracle import qlora_ref as R
    torch.set_num_threads(os.cpu_count() or 1)

    def step():
        for name, K, N in LLAMA3_8B_PROJ:
            packed, absmax, a, b, _, _ = layer_cpu[name]
            R.nf4_lora_linear(xs_cpu[K], packed, absmax, None, a, b, SCALING, N, BLOCK)

    t0 = time.perf_counter()
    step()  # warm-up, also sizes the sample
    first = time.perf_counter() - t0
    n = max(1, min(10, int(budget_s / max(first, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        step()
    dt = (time.perf_counter() - t0) / n
    return dt, n


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--m", type=int, default=1, help="decode tokens per step (activation rows)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path is built and measured on a single MI355X; "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    from rocm_qlora import ops
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    M = args.m

    layer_bytes = sum(N * K // 2 + (N * K // BLOCK) * 4 for _, K, N in LLAMA3_8B_PROJ)
    n_copies = max(2, math.ceil(520e6 / layer_bytes / 2) * 2)  # gate+up alone exceed 512 MB
    layers = [make_layer(dev, 1000 + c) for c in range(n_copies)]
    gx = torch.Generator(device=dev).manual_seed(7)
    xs = {K: torch.randn(M, K, generator=gx, device=dev).to(torch.bfloat16) for K in (4096, 14336)}

    def step(layer):
        out = []
        for name, K, N in LLAMA3_8B_PROJ:
            packed, absmax, a, b, _, _ = layer[name]
            out.append(ops.nf4_linear(xs[K], packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING))
        return out

    # warm every path (first launches set kernel attributes), then capture
    for layer in layers:
        step(layer)
    torch.cuda.synchronize()
    graphs = []
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for layer in layers:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step(layer)
            graphs.append(g)
    torch.cuda.synchronize()

    for i in range(args.warmup):
        graphs[i % n_copies].replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    t0.record(cur)
    for i in range(args.steps):
        graphs[i % n_copies].replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    step_bytes = sum(gemv_bytes(M, N, K) for _, K, N in LLAMA3_8B_PROJ)
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # roofline of the dominant kernel: plain GEMV launches at the gate/up shape
    K, N = 4096, 14336
    roof_w = [(layer[nm][0], layer[nm][1]) for layer in layers for nm in ("gate", "up")]
    x_roof = xs[K]

    def roof_pass():
        for packed, absmax in roof_w:
            ops.nf4_linear(x_roof, packed, absmax, N, BLOCK)

    roof_pass()
    torch.cuda.synchronize()
    rg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(rg, stream=stream):
            roof_pass()
    reps = 10
    rg.replay()
    torch.cuda.synchronize()
    t0.record(cur)
    for _ in range(reps):
        rg.replay()
    t1.record(cur)
    torch.cuda.synchronize()
    launches = reps * len(roof_w)
    us_launch = t0.elapsed_time(t1) * 1e3 / launches
    kb = kernel_bytes(M, N, K)
    achieved = kb / (us_launch * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu:
        layer_cpu = {nm: tuple(t.cpu() if torch.is_tensor(t) else t for t in v) for nm, v in layers[0].items()}
        xs_cpu = {k: v.cpu() for k, v in xs.items()}
        dt, n = cpu_baseline(layer_cpu, xs_cpu)
        cpu = {"value": round(step_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{n} decode step(s) of the same 7-projection layer (M={M}, LoRA r={RANK}) through "
                         f"the oracle's torch CPU restatement; {dt * 1e3:.1f} ms/step"}

    rec = {
        "metric": "NF4 dequant-GEMV GB/s + GEMM TFLOP/s (% roofline), Llama-3-8B proj shapes",
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
                   "tokens": M, "layer_copies": n_copies, "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "nf4_gemv_kernel", "shape": f"M={M} K={K} N={N}",
                     "bytes_per_launch": kb, "us_per_launch": round(us_launch, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
