"""Benchmark of the EXL3 quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload: Llama-3-8B-shaped decode stack at 4.0 bpw, 3INST
codebook, M = 1 fp16 activations ~ N(0, 1), random trellis words and +-1 suh / svh per layer;
32 distinct layers x 7 linears (q, k, v, o, gate, up, down) = 3.49 GB of packed weights,
far beyond the 256 MB Infinity Cache.  One step = one 32-layer sweep: 224 exl3_gemm calls
(the decode GEMV) replayed from one HIP graph, as the reference replays its decode step.

Prints one JSON line: value = packed-weight GB/s of the sweep, plus the roofline of the
dominant kernel (the K = 4 GEMV; per-launch HIP-event durations), per-shape figures and the
reference-style CPU path (host trellis reconstruct + Hadamard + ATen CPU matmul) timed on
this host's cores over a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "EXL3 GEMV GB/s (% HBM peak) at 4bpw M=1; prefill GEMM TFLOPS at M=2048"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def make_layers(torch, n_layers, K=4):
    from ampstein_amd.synth import LLAMA3_8B_SHAPES
    g = torch.Generator(device="cuda")
    layers = []
    for li in range(n_layers):
        row = []
        for si, (name, k, n) in enumerate(LLAMA3_8B_SHAPES):
            g.manual_seed(2000 + 7 * li + si)
            t = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16,
                              device="cuda", generator=g)
            s = (torch.randint(0, 2, (k,), device="cuda", generator=g) * 2 - 1).half()
            v = (torch.randint(0, 2, (n,), device="cuda", generator=g) * 2 - 1).half()
            row.append((name, k, n, t, s, v))
        layers.append(row)
    return layers


def cpu_baseline(seconds: float):
    """Reference CPU path on config 1 (4096 -> 4096, K = 4, 3INST): the oracle's host trellis
    reconstruct to fp16, Hadamard-128 on x (with suh) and on y (with svh), ATen CPU fp32
    matmul.  Repeated until `seconds` of work, on all host threads."""
    import numpy as np
    import torch
    from ampstein_amd import synth
    from oracle import oracle
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    L = synth.layer(4096, 4096, 4, 0, seed=1000)
    x = synth.activations(1, 4096, seed=1000)
    t_rec = t_had = t_mm = 0.0
    calls = 0
    t_end = time.perf_counter() + seconds
    while calls < 2 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        W = oracle.reconstruct(L.trellis, 4, cb=0, nthreads=threads)
        t1 = time.perf_counter()
        xh = oracle.had128(x, pre=L.suh)
        t2 = time.perf_counter()
        y = torch.from_numpy(xh.astype(np.float32)) @ torch.from_numpy(W.astype(np.float32))
        t3 = time.perf_counter()
        oracle.had128(y.numpy().astype(np.float16), post=L.svh)
        t4 = time.perf_counter()
        t_rec += t1 - t0
        t_had += (t2 - t1) + (t4 - t3)
        t_mm += t3 - t2
        calls += 1
    total = t_rec + t_had + t_mm
    us = total / calls * 1e6
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(L.packed_bytes / (us * 1e-6) / 1e9, 4), "unit": "GB/s", "cores": threads,
        "kind": "port",
        "sample": f"config 1 (4096x4096, K=4, 3INST, M=1) x {calls} calls: host reconstruct "
                  f"(oracle C, {threads} threads) + Hadamard-128 on x and y + ATen CPU fp32 matmul",
        "us_per_call": round(us, 1),
        "split_us": {"reconstruct": round(t_rec / calls * 1e6, 1), "hadamard": round(t_had / calls * 1e6, 1),
                     "matmul": round(t_mm / calls * 1e6, 1)},
        "nproc": os.cpu_count(), "torch_threads": torch.get_num_threads(), "cpu_model": cpu_model,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the EXL3 path runs on a single MI355X; see DESIGN.md for how it would shard)")
        return 2
    import torch
    from ampstein_amd import ops, _lib

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    ops.init(0)
    L = _lib.lib()
    layers = make_layers(torch, args.layers)
    x4096 = torch.randn((1, 4096), generator=torch.Generator(device="cuda").manual_seed(1),
                        device="cuda").half()
    x14336 = torch.randn((1, 14336), generator=torch.Generator(device="cuda").manual_seed(2),
                         device="cuda").half()
    outs = {n: torch.empty((1, n), dtype=torch.half, device="cuda") for n in (1024, 4096, 14336)}
    stream = torch.cuda.current_stream()

    calls = []
    for row in layers:
        for name, k, n, t, s, v in row:
            x = x14336 if k == 14336 else x4096
            calls.append((name, k, n, x, t, s, v, outs[n]))
    bytes_per_step = sum(c[4].numel() * 2 for c in calls)

    def launch(c, st):
        name, k, n, x, t, s, v, y = c
        rc = L.exl3_amd_gemm(x.data_ptr(), t.data_ptr(), y.data_ptr(), 0, s.data_ptr(), None,
                             v.data_ptr(), 1, k, n, 4.0, 0, 0, 0, st)
        if rc < 0:
            raise RuntimeError(L.exl3_amd_last_error().decode())

    # per-launch kernel durations (HIP events on the launch stream), one eager sweep x 3
    per_shape = {}
    evs = []
    for rep in range(3):
        for c in calls:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            launch(c, stream.cuda_stream)
            e1.record(stream)
            evs.append((c, e0, e1, rep))
    torch.cuda.synchronize()
    tot_ms = 0.0
    nmeas = 0
    for c, e0, e1, rep in evs:
        if rep == 0:
            continue   # first pass: cold code / first-touch
        ms = e0.elapsed_time(e1)
        d = per_shape.setdefault(c[0], {"k": c[1], "n": c[2], "bytes": c[4].numel() * 2, "ms": []})
        d["ms"].append(ms)
        tot_ms += ms
        nmeas += 1
    avg_launch_us = tot_ms / nmeas * 1e3
    avg_bytes = bytes_per_step / len(calls)

    # graph of the whole sweep
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        for c in calls:            # warm the captured path once outside the graph
            launch(c, cap.cuda_stream)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            for c in calls:
                launch(c, cap.cuda_stream)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    value = bytes_per_step / (ms_step * 1e-3) / 1e9

    shapes = {}
    for name, d in per_shape.items():
        us = sum(d["ms"]) / len(d["ms"]) * 1e3
        shapes[name] = {"k": d["k"], "n": d["n"], "us": round(us, 2),
                        "GB_s": round(d["bytes"] / (us * 1e-6) / 1e9, 1),
                        "frac_hbm": round(d["bytes"] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    achieved = avg_bytes / (avg_launch_us * 1e-6) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded random trellis words, +-1 suh/svh, N(0,1) fp16 x)",
        "config": {"workload": "llama3-8b-decode-sweep", "layers": args.layers, "bpw": 4,
                   "codebook": "3inst", "m": 1, "calls_per_step": len(calls),
                   "packed_bytes_per_step": bytes_per_step, "launch": "hip-graph replay"},
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel<K=4,3INST,M=1>",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "avg_launch_us": round(avg_launch_us, 3), "algorithmic_bytes_per_launch": round(avg_bytes)},
        "per_shape": shapes,
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
