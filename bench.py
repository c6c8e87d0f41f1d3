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
  roofline      the dominant kernel (the GEMV at the gate/up shape, no LoRA),
                timed with HIP events over back-to-back launches on the stream
                they run on; algorithmic bytes / average launch time vs 8 TB/s.
  gemm          the prefill/training shapes: the same seven projections at
                M = 2048 tokens with LoRA r = 64, alpha = 16, forward and dX
                backward, TFLOP/s and fraction of the 2.5 PFLOP/s bf16 MFMA peak.
  codec         NF4 + double quantization of an 11008x4096 bf16 weight (N(0,0.02)
                with 0.1 % outliers at +-8 sigma, blocks 64 / 256): quantize ->
                pack -> double-quantize the absmax, and double-dequantize ->
                bf16; algorithmic bytes / time vs 8 TB/s.
  byte_linears  INT8 (per-row absmax) and FP8 (e4m3fnuz, per-tensor scales)
                linears at the Llama-3-70B MLP shape 8192 -> 28672, M = 1
                (HBM: bytes / time, two weight copies rotating) and M = 512,
                4096 (TFLOP/s against the bf16 MFMA peak).
  cpu_baseline  the oracle's restatement of the reference's CPU path
                (dequantize_int4 -> .to(bf16) -> F.linear + LoRA) over a bounded
                sample of the same decode step on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m M] [--no-gemm] [--no-extra] [--no-cpu]
    python bench.py --summarize-profile DIR   # per-kernel, per-grid rocprofv3 kernel-trace table
    python bench.py --counters                # short eager run for rocprofv3 --pmc passes
    python bench.py --summarize-counters DIR [DIR ...]   # HBM bytes per launch from those passes
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

# (name, in_features K, out_features N)
LLAMA3_8B_PROJ = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
                  ("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096)]
RANK, ALPHA, BLOCK = 16, 32, 64
SCALING = ALPHA / RANK
GEMM_M, GEMM_RANK, GEMM_ALPHA = 2048, 64, 16

# HBM traffic of the roofline kernel per launch, measured with rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE and scaled by the same counters' reading for a copy
# kernel of known size (factors 0.5 for FETCH_SIZE, 1.0 for WRITE_SIZE on a
# 512 MiB device copy); keyed by (kernel, M, K, N).  None where not measured.
MEASURED_TRAFFIC = {("nf4_gemv_kernel", 1, 4096, 14336): 33331494}
COPY_BYTES = 512 << 20         # calibration copy: 512 MiB read + 512 MiB written


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


def cpu_baseline(layer_cpu, xs_cpu, budget_s=20.0):
    """The oracle's CPU restatement of the reference path over whole decode
    steps, as many as fit in about budget_s (at least one), on torch's
    default intra-op thread count."""
    from oracle import qlora_ref as R

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
    return (time.perf_counter() - t0) / n, n


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
    bf16, 0.1 % outliers at +-8 sigma), blocks 64 / 256, 10 graph replays
    each way.  Algorithmic bytes (each way): 2 numel (bf16 W) + numel / 2
    (packed) + numel / 64 (c2 codes) + 4 numel / 16384 (c2 scales)."""
    import torch
    from rocm_qlora.quantization import quantize_int4
    from rocm_qlora.quantization.double_quant import dq_quantize_absmax, dq_dequantize_to
    N, K = 11008, 4096
    numel = N * K
    g = torch.Generator(device=dev).manual_seed(5)
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    n_out = numel // 1000
    idx = torch.randperm(numel, generator=g, device=dev)[:n_out]
    sign = torch.randint(0, 2, (n_out,), generator=g, device=dev).float() * 2 - 1
    w.view(-1)[idx] = sign * 0.16
    w = w.to(torch.bfloat16)
    state = {}

    def encode():
        packed, c1 = quantize_int4(w, 64)
        c2, c2s = dq_quantize_absmax(c1, 256, True)
        state.update(packed=packed, c2=c2, c2s=c2s)

    encode()
    ge = _capture(encode, stream)
    packed, c2, c2s = state["packed"], state["c2"], state["c2s"]
    gd = _capture(lambda: dq_dequantize_to(packed, c2, c2s, 64, 256, True, torch.bfloat16, numel), stream)
    nbytes = 2 * numel + numel // 2 + numel // 64 + 4 * numel // 16384
    with _Range(f"rq-codec encode {N}x{K}"):
        ms_e = _time_graph(ge, 10)
    with _Range(f"rq-codec decode {N}x{K}"):
        ms_d = _time_graph(gd, 10)
    del ge, gd
    enc, dec = nbytes / ms_e / 1e6, nbytes / ms_d / 1e6
    return {"workload": f"NF4 + double quantization (blocks 64/256, fp8 c2) of a {N}x{K} bf16 weight with "
                        f"0.1% outliers at +-8 sigma",
            "bytes": nbytes, "encode_us": round(ms_e * 1e3, 2), "encode_gbs": round(enc, 1),
            "encode_frac": round(enc / HBM_PEAK_GBS, 4), "decode_us": round(ms_d * 1e3, 2),
            "decode_gbs": round(dec, 1), "decode_frac": round(dec / HBM_PEAK_GBS, 4)}


def bench_byte_linears(dev, stream):
    """INT8 per-row-absmax (bf16 MFMA) and FP8 (e4m3, fp8 MFMA) linears at 8192 -> 28672 with
    bf16 activations N(0,1), weights N(0,0.02); M = 1 rotates two weight
    copies (470 MB each kind, past the MALL), M = 512 and 4096 one copy."""
    import torch
    from rocm_qlora import ops
    from rocm_qlora.quantization import quantize_int8
    K, N = 8192, 28672
    g = torch.Generator(device=dev).manual_seed(9)
    int8_w, fp8_w = [], []
    for c in range(2):
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        int8_w.append(quantize_int8(w, per_channel=True))
        codes, scale = ops.fp8_quantize(w)
        fp8_w.append((ops.fp8_to_e4m3fn(codes), scale))  # as FP8LinearWrapper caches it
        del codes
        del w
    out = {}
    for M in (1, 512, 4096):
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        copies = 2 if M == 1 else 1
        for kind in ("int8", "fp8"):
            if kind == "int8":
                fn = lambda: [ops.int8_linear(x, q, s, N) for q, s in int8_w[:copies]]
            else:
                fn = lambda: [ops.fp8_linear(x, cw, sc) for cw, sc in fp8_w[:copies]]
            gr = _capture(fn, stream)
            with _Range(f"rq-{kind}-linear M={M} K={K} N={N}"):
                us = _time_graph(gr, 10) * 1e3 / copies
            del gr
            if M == 1:
                nb = N * K + 4 * N + 2 * M * K + 2 * M * N
                gbs = nb / us / 1e3
                out[f"{kind}_m{M}"] = {"us": round(us, 2), "gbs": round(gbs, 1),
                                        "frac": round(gbs / HBM_PEAK_GBS, 4), "bound": "hbm"}
            else:
                tf = 2 * M * N * K / us / 1e6
                peak, bound = (BF16_PEAK_TFLOPS, "bf16 mfma") if kind == "int8" else (FP8_PEAK_TFLOPS, "fp8 mfma")
                out[f"{kind}_m{M}"] = {"us": round(us, 2), "tflops": round(tf, 1),
                                        "frac": round(tf / peak, 4), "bound": bound}
        del x
    return {"workload": f"INT8 per-row and FP8 per-tensor linears, K={K} N={N}, bf16 activations", **out}


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


def run_counters(reps=4):
    """Eager launches for counter collection: one plain device copy of
    COPY_BYTES (calibration: its FETCH_SIZE / WRITE_SIZE readings against the
    bytes it must move), then the roofline GEMV (M=1, K=4096, N=14336, no
    LoRA) over the gate and up weights of six layer copies, `reps` rounds."""
    import torch
    from rocm_qlora import ops
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    src = torch.randint(0, 255, (COPY_BYTES,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    K, N = 4096, 14336
    weights = []
    for c in range(6):
        layer = make_layer(dev, 1000 + c)
        weights += [(layer[nm][0], layer[nm][1]) for nm in ("gate", "up")]
        del layer
    x = torch.randn(1, K, device=dev).to(torch.bfloat16)
    for _ in range(reps):
        for packed, absmax in weights:
            ops.nf4_linear(x, packed, absmax, N, BLOCK)
    torch.cuda.synchronize()
    print(f"counters: copy {COPY_BYTES} B, {reps * len(weights)} nf4_gemv_kernel launches M=1 K={K} N={N}",
          flush=True)


def summarize_counters(paths):
    """Per-kernel mean of each counter over the dispatches in rocprofv3 CSV
    counter files (`-f csv`), and the GEMV's HBM bytes per launch: FETCH_SIZE
    and WRITE_SIZE (KiB per dispatch) divided by what the same counter reads
    per byte for the calibration copy."""
    files = []
    for p in paths:
        files += glob.glob(os.path.join(p, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        sys.exit(f"no *counter_collection.csv under {paths}")
    per = {}   # (kernel, counter) -> {dispatch: value}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                key = (row["Kernel_Name"], row["Counter_Name"])
                d = per.setdefault(key, {})
                did = (f, row.get("Dispatch_Id", row.get("Correlation_Id")))
                d[did] = d.get(did, 0.0) + float(row["Counter_Value"])
    means = {}
    for (kname, cname), d in per.items():
        short = "copy" if "copy" in kname.lower() else ("nf4_gemv_kernel" if "nf4_gemv_kernel" in kname else None)
        vals = list(d.values())
        print(f"{_short(kname):<70} {cname:<12} n={len(vals):<4} mean={sum(vals) / len(vals):.1f}")
        if short:
            means.setdefault((short, cname), []).extend(vals)
    M, K, N = 1, 4096, 14336
    kb = kernel_bytes(M, N, K)
    out = {}
    for cname, expect in (("FETCH_SIZE", COPY_BYTES), ("WRITE_SIZE", COPY_BYTES)):
        c = means.get(("copy", cname))
        g = means.get(("nf4_gemv_kernel", cname))
        if not c or not g:
            continue
        factor = (max(c) * 1024.0) / expect
        gem = sum(g) / len(g) * 1024.0
        out[cname] = gem / factor
        print(f"{cname}: copy reads {max(c) * 1024.0 / 2**20:.1f} MiB for {expect / 2**20:.0f} MiB "
              f"(factor {factor:.4f}); nf4_gemv_kernel {gem / 1e6:.3f} MB raw -> {gem / factor / 1e6:.3f} MB")
    if len(out) == 2:
        t = out["FETCH_SIZE"] + out["WRITE_SIZE"]
        print(f"nf4_gemv_kernel M={M} K={K} N={N}: HBM traffic {t:.0f} B per launch "
              f"(algorithmic {kb} B, ratio {t / kb:.3f})")


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
    ap.add_argument("--counters", action="store_true", help="short eager run for rocprofv3 --pmc passes")
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
        run_counters()
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
    xs = {K: torch.randn(M, K, generator=gx, device=dev).to(torch.bfloat16) for K in (4096, 14336)}
    stream = torch.cuda.Stream()

    def step(layer):
        for name, K, N in LLAMA3_8B_PROJ:
            packed, absmax, a, b, _, _ = layer[name]
            ops.nf4_linear(xs[K], packed, absmax, N, BLOCK, lora_a=a, lora_b=b, scaling=SCALING)

    graphs = [_capture(lambda L=layer: step(L), stream) for layer in layers]
    for i in range(args.warmup):
        graphs[i % n_copies].replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    with _Range("rq-decode-step"):
        t0.record(cur)
        for i in range(args.steps):
            graphs[i % n_copies].replay()
        t1.record(cur)
        torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    step_bytes = sum(gemv_bytes(M, N, K) for _, K, N in LLAMA3_8B_PROJ)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    del graphs

    # roofline of the dominant kernel: plain GEMV launches at the gate/up shape
    K, N = 4096, 14336
    roof_w = [(layer[nm][0], layer[nm][1]) for layer in layers for nm in ("gate", "up")]
    x_roof = xs[K]

    def roof_pass():
        for packed, absmax in roof_w:
            ops.nf4_linear(x_roof, packed, absmax, N, BLOCK)

    rg = _capture(roof_pass, stream)
    reps = 10
    with _Range(f"rq-roofline nf4_gemv_kernel M={M} K={K} N={N}"):
        us_launch = _time_graph(rg, reps) * 1e3 / len(roof_w)
    kb = kernel_bytes(M, N, K)
    achieved = kb / (us_launch * 1e-6) / 1e9
    del rg
    print(f"bench: decode {ms_step * 1e3:.1f} us/step, {value:.0f} GB/s; gate/up GEMV {us_launch:.2f} us",
          file=sys.stderr, flush=True)

    gemm = None
    if not args.no_gemm:
        del layers
        torch.cuda.empty_cache()
        gemm = bench_gemm(dev, stream)
        print(f"bench: GEMM fwd {gemm['fwd_tflops']} TF/s, dX {gemm['dx_tflops']} TF/s", file=sys.stderr,
              flush=True)
        layer0 = make_layer(dev, 1000)
    else:
        layer0 = layers[0]

    codec = byte = None
    if not args.no_extra:
        codec = bench_codec(dev, stream)
        print(f"bench: codec encode {codec['encode_gbs']} GB/s, decode {codec['decode_gbs']} GB/s",
              file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        byte = bench_byte_linears(dev, stream)
        print("bench: byte linears " + ", ".join(f"{k} {v['us']} us" for k, v in byte.items()
                                                  if isinstance(v, dict)), file=sys.stderr, flush=True)
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        layer_cpu = {nm: tuple(t.cpu() if torch.is_tensor(t) else t for t in v) for nm, v in layer0.items()}
        xs_cpu = {k: v.cpu() for k, v in xs.items()}
        dt, n = cpu_baseline(layer_cpu, xs_cpu)
        cpu = {"value": round(step_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{n} decode step(s) of one 7-projection Llama-3-8B layer (M={M}, LoRA r={RANK}) "
                         f"through the oracle's torch CPU restatement of dequantize_int4 -> .to(bf16) -> "
                         f"F.linear + LoRA; {dt * 1e3:.1f} ms/step"}

    traffic = MEASURED_TRAFFIC.get(("nf4_gemv_kernel", M, K, N))
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
                   "tokens": M, "layer_copies": n_copies, "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "nf4_gemv_kernel", "shape": f"M={M} K={K} N={N}",
                     "bytes_per_launch": kb, "us_per_launch": round(us_launch, 3)},
        "gemm": gemm,
        "codec": codec,
        "byte_linears": byte,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
