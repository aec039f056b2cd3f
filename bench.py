"""Benchmark of the EXL3 quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-traffic]

Workload: Llama-3-8B-shaped decode stack at 4.0 bpw, 3INST
codebook, M = 1 fp16 activations ~ N(0, 1), random trellis words and +-1 suh / svh per layer;
32 distinct layers x 7 linears (q, k, v, o, gate, up, down) = 3.49 GB of packed weights, far
beyond the 256 MB Infinity Cache.  One step = one 32-layer sweep launched the way the
engine's decode step launches it (graphdec.uc:168-196): q/k/v as ONE sliced exl3_mgemm,
o as exl3_gemm, gate/up as ONE stacked exl3_mgemm, down as exl3_gemm -- 128 launches,
replayed from one HIP graph.

Prints one JSON line: value = packed-weight GB/s of the sweep; roofline of the dominant
kernel (the M = 1 GEMV as the stacked gate/up exl3_mgemm, half of the step's bytes: 32
back-to-back launches in a graph, HIP events on the replay stream, algorithmic bytes / average
launch time, inter-launch gaps included); traffic = HBM bytes per launch of that kernel from
rocprofv3 FETCH_SIZE and WRITE_SIZE passes (child processes, each scaled by the same counter
on a device copy of known size);
per-shape figures with one exl3_gemm per linear; the reference-style CPU path (host trellis
reconstruct + Hadamard + ATen CPU matmul) timed on this host's cores over a bounded sample.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "EXL3 GEMV GB/s (% HBM peak) at 4bpw M=1; prefill GEMM TFLOPS at M=2048"
COPY_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 traffic passes")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-prefill", action="store_true", help="skip the M = 2048 prefill GEMM line")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE expert GEMV line")
    ap.add_argument("--no-qwen", action="store_true", help="skip the configs[2] Qwen-27B-class line")
    ap.add_argument("--pmc-child", nargs="?", const="gateup", default=None,
                    help="profiled child for rocprofv3 --pmc: decode | gateup | prefill | dense | moe | moes | qwenm")
    ap.add_argument("--summarize-pmc", metavar="PMC_DIR", nargs="+",
                    help="print per-kernel averages and derived figures of rocprofv3 --pmc output "
                         "directories (one per counter pass) and exit")
    ap.add_argument("--decode-step", action="store_true",
                    help="only the captured decode step's variants (0.3 s apart, for a kernel trace)")
    ap.add_argument("--recon-rows", action="store_true",
                    help="print the route table by row count: GEMV groups, MFMA GEMM, recon route with and without its split k")
    ap.add_argument("--rates", action="store_true",
                    help="print the gfx950 issue-rate microbenchmarks (ampstein_amd/csrc/exl3_probe.hip) and exit")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="print per-kernel/grid duration stats of a rocprofv3 kernel trace and exit")
    ap.add_argument("--gap-ms", type=float, default=0.0,
                    help="with --summarize-trace: one table per phase, split at idle gaps longer than this")
    return ap.parse_args()


# ------------------------------------------------------------------ workload
def host_trellis(torch, k, n, K, seed):
    """Seeded host generation (one numpy PCG64 generator per tensor, the scheme of
    ampstein_amd/synth.py), then one copy to the device, so the CPU and GPU legs can see
    identical bytes.  Uniform uint16 trellis words, +-1 fp16 suh / svh."""
    import numpy as np
    rng = np.random.default_rng(seed)
    t = rng.integers(0, 65536, size=(k // 16, n // 16, int(16 * K)), dtype=np.uint16).view(np.int16)
    s = np.where(rng.integers(0, 2, k) > 0, 1.0, -1.0).astype(np.float16)
    v = np.where(rng.integers(0, 2, n) > 0, 1.0, -1.0).astype(np.float16)
    return torch.from_numpy(t).cuda(), torch.from_numpy(s).cuda(), torch.from_numpy(v).cuda()


def host_normal(torch, shape, seed):
    import numpy as np
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32).astype(np.float16)).cuda()


def make_stack(torch, n_layers, K=4):
    """Per layer: name -> bundles.Linear with host-generated random trellis words and signs
    (seed = 1000 * config + 7 * layer + linear)."""
    from ampstein_amd.synth import LLAMA3_8B_SHAPES
    from ampstein_amd.bundles import Linear
    layers = []
    for li in range(n_layers):
        row = {}
        for si, (name, k, n) in enumerate(LLAMA3_8B_SHAPES):
            t, s, v = host_trellis(torch, k, n, K, 2000 + 7 * li + si)
            row[name] = Linear(t, s, v, float(K))
        layers.append(row)
    return layers


class Sweep:
    """The decode-step launch sequence over all layers, bundled (engine schedule) or one
    exl3_gemm per linear.  Each entry: (label, launch(stream_ptr), packed bytes)."""

    def __init__(self, torch, layers, bundled):
        from ampstein_amd import bundles, _lib
        self.L = _lib.lib()
        dev = "cuda"
        self.x = host_normal(torch, (1, 1, 4096), 2001)
        self.x14 = host_normal(torch, (1, 1, 14336), 2002)
        self.outs = {nm: torch.empty((1, 1, n), dtype=torch.half, device=dev)
                     for nm, n in (("q", 4096), ("k", 1024), ("v", 1024), ("o", 4096), ("down", 4096))}
        self.gu = torch.empty((2, 1, 14336), dtype=torch.half, device=dev)
        self.entries = []
        for row in layers:
            if bundled:
                qkv = bundles.Sliced([row["q"], row["k"], row["v"]], [self.outs["q"], self.outs["k"], self.outs["v"]])
                gu = bundles.Multi([row["gate"], row["up"]], self.gu)
                nb = lambda *names: sum(row[n].trellis.numel() * 2 for n in names)
                self.entries.append(("qkv", self._bundle(qkv), nb("q", "k", "v")))
                self.entries.append(("o", self._gemm(row["o"], self.x, self.outs["o"]), nb("o")))
                self.entries.append(("gate_up", self._bundle(gu), nb("gate", "up")))
                self.entries.append(("down", self._gemm(row["down"], self.x14, self.outs["down"]), nb("down")))
            else:
                for nm in ("q", "k", "v", "o", "gate", "up", "down"):
                    xin = self.x14 if nm == "down" else self.x
                    out = self.gu[0] if nm in ("gate", "up") else self.outs[nm]
                    self.entries.append((nm, self._gemm(row[nm], xin, out), row[nm].trellis.numel() * 2))
        self.bytes = sum(e[2] for e in self.entries)

    def _gemm(self, lin, x, y):
        L = self.L
        k, n = lin.in_features, lin.out_features

        def launch(st):
            rc = L.exl3_amd_gemm(x.data_ptr(), lin.trellis.data_ptr(), y.data_ptr(), 0, lin.suh.data_ptr(), None,
                                 lin.svh.data_ptr(), 1, k, n, float(lin.K), 0, 0, 0, st)
            if rc < 0:
                raise RuntimeError(L.exl3_amd_last_error().decode())
        return launch

    def _bundle(self, b):
        def launch(st):
            b.run(self.x)    # enqueued on torch's current stream, which the caller sets
        return launch

    def run(self, torch, stream):
        with torch.cuda.stream(stream):
            st = stream.cuda_stream
            for _, fn, _ in self.entries:
                fn(st)


class Launches:
    """A launch sequence: entries of (label, launch(stream_ptr), packed bytes)."""

    def __init__(self, entries):
        self.entries = entries
        self.bytes = sum(e[2] for e in entries)

    def run(self, torch, stream):
        with torch.cuda.stream(stream):
            for _, fn, _ in self.entries:
                fn(stream.cuda_stream)


def event_times(torch, sweep, reps=3):
    """Per-launch HIP-event durations (ms) on the launch stream; the first pass is dropped."""
    stream = torch.cuda.Stream()
    recs = []
    with torch.cuda.stream(stream):
        for rep in range(reps):
            for label, fn, nbytes in sweep.entries:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                fn(stream.cuda_stream)
                e1.record(stream)
                recs.append((rep, label, nbytes, e0, e1))
    torch.cuda.synchronize()
    return [(label, nbytes, e0.elapsed_time(e1)) for rep, label, nbytes, e0, e1 in recs if rep > 0]


def dominant_region(torch, layers, reps=3, blocks=7):
    """The dominant launch of the sweep -- the stacked gate/up exl3_mgemm (58.7 MB, half the
    step's bytes) -- as its own timed region: one launch per layer (distinct weights), captured
    in a graph, HIP events around the replays on the replay stream.  Returns (avg us per launch
    of the median block, bytes per launch, launches timed)."""
    from ampstein_amd import bundles
    gu_out = torch.empty((2, 1, 14336), dtype=torch.half, device="cuda")
    x = host_normal(torch, (1, 1, 4096), 2003)
    bs = [bundles.Multi([row["gate"], row["up"]], gu_out) for row in layers]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for b in bs:
            b.run(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for b in bs:
            b.run(x)
    graph.replay()
    torch.cuda.synchronize()
    # `blocks` timed blocks of `reps` replays each; the median block (clock and thermal state
    # move a single short block by a few per cent)
    per = []
    with torch.cuda.stream(stream):
        for _ in range(blocks):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            per.append((e0, e1))
    torch.cuda.synchronize()
    n = reps * len(bs)
    us = sorted(e0.elapsed_time(e1) * 1e3 / n for e0, e1 in per)
    nbytes = layers[0]["gate"].trellis.numel() * 4
    return us[len(us) // 2], nbytes, n * blocks


def graph_time(torch, sweep, steps, warmup):
    stream = torch.cuda.Stream()
    sweep.run(torch, stream)                    # warm the path outside the graph
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _, fn, _ in sweep.entries:
            fn(stream.cuda_stream)
    torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, time.perf_counter() - t0


# ------------------------------------------------------------------ captured decode step
def decode_step_bench(torch, layers, steps=20, gap_s=0.0):
    """The linear part of the Llama-3-8B decode step with its neighbours (graphdec.uc:151-230:
    rms_norm_res, q/k/v sliced mgemm, o gemm, rms_norm_res, gate/up stacked mgemm, SwiGLU + down,
    final norm) captured into one graph over the same 32 layers; attention is outside the path
    (the q projection feeds o).  fused_swiglu: the down GEMV forms silu(gate) * up in its input
    load; fused_norm_swiglu: o and down also run the residual norm in their last column chunk;
    split_norm_swiglu: each norm divided between its neighbours (o / down add the residual and
    keep chunk sums of squares, q/k/v and gate/up normalise their input on load)."""
    from ampstein_amd.decode import DecodeStack, LayerWeights
    H = 4096
    ones = torch.ones(H, dtype=torch.half, device="cuda")
    lw = [LayerWeights(q=r["q"], k=r["k"], v=r["v"], o=r["o"], gate=r["gate"], up=r["up"], down=r["down"],
                       input_norm=ones, post_norm=ones) for r in layers]
    nbytes = sum(r[n].trellis.numel() * 2 for r in layers for n in ("q", "k", "v", "o", "gate", "up", "down"))
    x = host_normal(torch, (1, H), 2004)
    res = {}
    for name, fuse, fnorm, snorm, launches in (("split_norm_swiglu", True, False, True, 4),
                                               ("fused_norm_swiglu", True, True, False, 4),
                                               ("fused_swiglu", True, False, False, 6),
                                               ("separate_silu_mul", False, False, False, 7)):
        st = DecodeStack(lw, ones, fuse_swiglu=fuse, fuse_norm=fnorm, split_norm=snorm)
        st.capture()
        for _ in range(3):
            st(x)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            st.graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        res[name] = {"us_per_step": round(us, 1), "us_per_layer": round(us / len(layers), 2),
                     "launches_per_layer": launches, "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1)}
        del st
        if gap_s:
            time.sleep(gap_s)              # an idle gap: a kernel trace separates the variants by time
    return {"what": "32-layer decode step without attention: norms + linears + SwiGLU, one graph",
            "packed_bytes": nbytes, **res}


# ------------------------------------------------------------------ prefill GEMM
MFMA_F16_PEAK_TFLOPS = 2500.0


def timed(torch, fn, reps=5):
    fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def prefill_bench(torch):
    """M = 2048 fp16 x N(0,1) against 8192->28672 and 28672->8192 at 4 bpw (3INST).  Paths, all on
    this build's kernels: fused = the MFMA GEMM decoding the trellis in its loop (exl3_gemm, m > 8);
    recon = the reference's routing for rows >= 2048 (amp_torch.cpp:11149-11230): reconstruct_had_t
    then the dense MFMA GEMM (recon_mm); recon_rotated = its rows < 2048 branch (x rotated, W_hat
    reconstructed, recon_mm with the output rotation in its epilogue); both recon routes lay the
    GEMM's operands out in k slabs.  dense_gemm = recon_mm alone on a reconstructed W_hat^T and x,
    row-major; dense_gemm_slabs = the same operands in k slabs.  Beside them, labelled comparisons
    on the vendor library (torch.mm on hipBLASLt / rocBLAS, tuned): the same dense GEMM and the
    rotated recon route around it."""
    from ampstein_amd import ops
    M = 2048
    res = {}
    mine = ("fused", "recon", "recon_rotated", "dense_gemm", "dense_gemm_slabs")
    lib = ("library_dense_gemm", "library_recon_rotated")
    for si, (k, n) in enumerate(((8192, 28672), (28672, 8192))):
        t, s, v = host_trellis(torch, k, n, 4, 4000 + si)
        x = host_normal(torch, (M, k), 4010 + si)
        ah = torch.empty_like(x)
        C = torch.empty((M, n), dtype=torch.half, device="cuda")
        wt = torch.empty((n, k), dtype=torch.half, device="cuda")
        ops.reconstruct_t(wt, t, 4.0)
        xs, wts = ops.slabs_of(x), ops.slabs_of(wt)
        flops = 2.0 * M * k * n
        row = {}
        for name, fn in (("fused", lambda: ops.exl3_gemm(x, t, C, s, ah, v)),
                         ("recon", lambda: ops.exl3_gemm_recon(x, t, s, v, 4.0, fused_rows=2048)),
                         ("recon_rotated", lambda: ops.exl3_gemm_recon(x, t, s, v, 4.0, fused_rows=1 << 30)),
                         ("dense_gemm", lambda: ops.recon_mm(x, wt, C)),
                         ("dense_gemm_slabs", lambda: ops.recon_mm(xs, wts, C)),
                         ("library_dense_gemm", lambda: ops._library_mm(x, wt.t(), C)),
                         ("library_recon_rotated", lambda: ops.exl3_gemm_recon(x, t, s, v, 4.0, fused_rows=1 << 30,
                                                                             gemm="library"))):
            us = timed(torch, fn)
            row[name] = {"us": round(us, 1), "TFLOPS": round(flops / us / 1e6, 1),
                         "frac_mfma_peak": round(flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4)}
        res[f"{k}x{n}"] = row
        del t, s, v, x, ah, C, wt, xs, wts
        torch.cuda.empty_cache()
    tot = lambda name: sum(2.0 * M * int(sh.split("x")[0]) * int(sh.split("x")[1]) for sh in res) / \
        sum(res[sh][name]["us"] for sh in res) / 1e6
    best = {name: tot(name) for name in mine + lib}
    route = max(("fused", "recon", "recon_rotated"), key=lambda nm: best[nm])
    return {"metric": "prefill GEMM TFLOPS at M=2048 (configs[3], 4 bpw 3INST)", "m": M,
            "value": round(best[route], 1), "unit": "TFLOPS",
            "path": f"{route} (fastest of this build's hand-written routes; no vendor GEMM)",
            "peak": MFMA_F16_PEAK_TFLOPS, "frac": round(best[route] / MFMA_F16_PEAK_TFLOPS, 4),
            "paths_TFLOPS": {nm: round(best[nm], 1) for nm in mine},
            "dense_gemm_frac_mfma_peak": round(best["dense_gemm"] / MFMA_F16_PEAK_TFLOPS, 4),
            "dense_gemm_slabs_frac_mfma_peak": round(best["dense_gemm_slabs"] / MFMA_F16_PEAK_TFLOPS, 4),
            "comparison_library_TFLOPS": {nm: round(best[nm], 1) for nm in lib},
            "per_shape": res}


# ------------------------------------------------------------------ Qwen-27B-class shapes
QWEN_SHAPES = ((5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120))


def qwen_bench(torch, min_bytes=1 << 30):
    """the four Qwen-27B-class shapes as one layer, swept over enough distinct layers
    (>= 1 GB of packed weights, beyond the 256 MB MALL) in one graph, for K in {2, 3, 5, 8} x
    {3INST, MCG} x M in {1, 4, 8}, and the half rates K in {1.5, 2.5, 3.5} (MUL1, their only
    codebook) x M in {1, 8}.  The same random words serve every codebook.  GB/s = packed bytes
    of the sweep / graph time; per-shape us from HIP events around single launches."""
    from ampstein_amd import _lib
    from ampstein_amd.bundles import Linear
    res = {}
    plans = [(K, (0, 1), (1, 4, 8)) for K in (2, 3, 5, 8)] + [(K, (2,), (1, 8)) for K in (1.5, 2.5, 3.5)]
    for K, cbs, Ms in plans:
        per_layer = sum(int(k * n * K) // 8 for k, n in QWEN_SHAPES)
        n_layers = max(2, -(-min_bytes // per_layer))
        layers = [[Linear(*host_trellis(torch, k, n, K, 7000 + int(100 * K) + 4 * li + si), float(K))
                   for si, (k, n) in enumerate(QWEN_SHAPES)] for li in range(n_layers)]
        for cb in cbs:
            for M in Ms:
                xs = {k: host_normal(torch, (M, k), 7500 + k + M) for k in (5120, 17408)}
                ys = {n: torch.empty((M, n), dtype=torch.half, device="cuda") for n in (5120, 1024, 17408)}
                hads = {k: torch.empty((M, k), dtype=torch.half, device="cuda") for k in (5120, 17408)}
                L = _lib.lib()

                def launch(lin, st):
                    k, n = lin.in_features, lin.out_features
                    rc = L.exl3_amd_gemm(xs[k].data_ptr(), lin.trellis.data_ptr(), ys[n].data_ptr(), 0,
                                         lin.suh.data_ptr(), hads[k].data_ptr(), lin.svh.data_ptr(), M, k, n,
                                         float(K), cb == 1, cb == 2, 0, st)
                    if rc < 0:
                        raise RuntimeError(L.exl3_amd_last_error().decode())

                sw = Launches([(f"{lin.in_features}x{lin.out_features}", (lambda st, lin=lin: launch(lin, st)),
                                 lin.trellis.numel() * 2) for row in layers for lin in row])
                ms, _ = graph_time(torch, sw, 10, 2)
                ev = {}
                for label, nbytes, t_ms in event_times(torch, sw, reps=2):
                    ev.setdefault(label, []).append(t_ms)
                res[f"K{K}_{('3inst', 'mcg', 'mul1')[cb]}_M{M}"] = {
                    "sweep_GB_s": round(per_layer * n_layers / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm": round(per_layer * n_layers / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "per_shape_us": {lab: round(sum(v) / len(v) * 1e3, 2) for lab, v in ev.items()}}
                del xs, ys, hads
        del layers
        torch.cuda.empty_cache()
    return {"metric": "EXL3 GEMV GB/s on Qwen-27B-class shapes (configs[2])", "per_case": res}


# ------------------------------------------------------------------ MoE expert GEMV
def moe_bench(torch, reps=8, ms=(1, 8, 16), token_sorted=True, graph=True):
    """256 experts, gate/up 4096->2048, down 2048->4096, K per expert from {2,3,4} (seeded), mul1;
    router logits N(0,1), softmax top-8; M in {1, 8, 16}.  Algorithmic bytes = packed bytes of the
    distinct routed experts.  `reps` different routings rotate through one graph so the routed
    experts change between calls (the 256 MB MALL cannot hold them)."""
    import numpy as np
    from ampstein_amd import ops
    E, Hi, I, Ho, topk = 256, 4096, 2048, 4096, 8
    rng = np.random.default_rng(5000)
    Ks = rng.choice([2, 3, 4], E)
    mats = []
    for e in range(E):
        trio = []
        for pi, (k, n) in enumerate(((Hi, I), (Hi, I), (I, Ho))):
            trio.append(host_trellis(torch, k, n, int(Ks[e]), 6000 + 3 * e + pi))
        mats.append(trio)
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    tabs = [P([mats[e][pi][j].data_ptr() for e in range(E)]) for pi in range(3) for j in range(3)]
    bits = torch.tensor(Ks, dtype=torch.uint8, device="cuda")
    per_expert = {e: int(Ks[e]) * (2 * Hi * I + I * Ho) // 8 for e in range(E)}
    res = {}
    for M in ms:
        slots = M * topk
        routs = []
        for r in range(reps):
            logits = rng.standard_normal((M, E))
            p = np.exp(logits - logits.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            sel = np.argsort(-p, axis=1, kind="stable")[:, :topk]
            rw = np.take_along_axis(p, sel, 1).astype(np.float16)
            routs.append((torch.from_numpy(sel.astype(np.int64)).cuda(), torch.from_numpy(rw).cuda(),
                          sum(per_expert[int(e)] for e in set(sel.reshape(-1).tolist()))))
        x = host_normal(torch, (M, Hi), 5100 + M)
        z = lambda *sh, dt=torch.half: torch.zeros(sh, dtype=dt, device="cuda")
        had_g, had_u, act_out = z(slots, Hi), z(slots, Hi), z(slots, I)
        gu = z(slots, I, dt=torch.float)
        d_out = z(slots, Ho, dt=torch.float)
        ctr = torch.zeros(ops.moe_coop_ctr_len(slots, M, I, Ho), dtype=torch.int32, device="cuda")
        out = z(M, Ho, dt=torch.float)

        def call(sel, rw):
            ops.exl3_moe_coop(x, sel, rw, -1, -1, Hi, *tabs, None, None, None, 4.0, 4.0, 4.0, False, True, 0, 0.0,
                              True, had_g, had_u, gu, gu, act_out, d_out, ctr, out, None, None, bits, bits, bits)
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            for sel, rw, _ in routs:
                call(sel, rw)
        torch.cuda.synchronize()
        if not graph:
            continue
        cg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(cg, stream=stream):
            for sel, rw, _ in routs:
                call(sel, rw)
        cg.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(4):
            cg.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (4 * reps)
        nbytes = sum(r[2] for r in routs) / reps
        res[f"M{M}"] = {"us_per_call": round(us, 2), "routed_bytes": round(nbytes), "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    # token-sorted prefill MoE (exl3_moe) on the same experts: T tokens, pool = every assignment
    pre = {}
    conc = ops.exl3_moe_max_concurrency(torch.cuda.current_device())
    for T in ((512, 2048) if token_sorted else ()):
        logits = rng.standard_normal((T, E))
        sel = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
        p = np.exp(logits - logits.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        rw = np.take_along_axis(p, sel, 1).astype(np.float16)
        flat = sel.reshape(-1)
        order = np.argsort(flat, kind="stable")
        count = np.bincount(flat, minlength=E + 1).astype(np.int64)
        max_tok = -(-T * topk // conc)
        dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        cnt, tok, ws = dv(count), dv((order // topk).astype(np.int64)), dv(rw.reshape(-1)[order])
        x = host_normal(torch, (T, Hi), 5200 + T)
        out = torch.zeros((T, Ho), dtype=torch.float, device="cuda")
        tsg, tsu = (torch.empty((conc, max_tok, Hi), dtype=torch.half, device="cuda") for _ in range(2))
        tig, tiu = (torch.empty((conc, max_tok, I), dtype=torch.half, device="cuda") for _ in range(2))
        active = int((count[:E] > 0).sum())

        def call():
            ops.exl3_moe(x, out, cnt, tok, ws, tsg, tsu, tig, tiu, 0, 0.0, 0.0, 0.0, *tabs,
                         False, True, False, True, False, True, 0.0, active, None, None, 0, 1 << 30, 16,
                         bits, bits, bits)
        us = timed(torch, call, reps=5)
        flops = 2.0 * T * topk * (2 * Hi * I + I * Ho)
        nbytes = sum(per_expert[e] for e in range(E) if count[e] > 0)
        pre[f"T{T}"] = {"us_per_call": round(us, 1), "TFLOPS": round(flops / us / 1e6, 1),
                        "frac_mfma_peak": round(flops / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
                        "routed_bytes": nbytes, "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "active_experts": active, "max_rows_per_expert": int(count[:E].max())}
        del tsg, tsu, tig, tiu, out, x
        torch.cuda.empty_cache()
    return {"metric": "MoE mixed-K expert GEMV GB/s (configs[4]: 256 experts, K in {2,3,4}, mul1, top-8)",
            "launches_per_call": {"M1": 3, "M8": 5, "M16": 5}, "per_m": res,
            "prefill_token_sorted": {"op": "exl3_moe (token-sorted, grouped MFMA GEMM)", "per_T": pre}}


# ------------------------------------------------------------------ CPU baseline
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
    us = (t_rec + t_had + t_mm) / calls * 1e6
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


# ------------------------------------------------------------------ HBM traffic (rocprofv3)
GEMV_KERNEL = "gemv1_kernel"


def pmc_child(workload="decode"):
    """Profiled child (rocprofv3 --pmc runs): a device copy of known size (the calibration
    dispatch), then a short eager run of one workload:
      decode  -- two passes of the bundled decode sweep over 4 layers (qkv sliced mgemm, o gemm,
                 gate/up stacked mgemm, down gemm: four GEMV grids);
      gateup  -- the stacked gate/up mgemm alone, 2 x 4 launches (the traffic passes);
      prefill -- the MFMA GEMM at 2048 rows on 8192 -> 28672 and 28672 -> 8192;
      dense   -- the recon route's dense GEMM at 2048 rows, both shapes: on k-slab operands
                 (dense_gemm4_kernel<3, true>, the route's form), on row-major operands
                 (dense_gemm4_kernel<3, false>: the 64-bit-address DMA form, and the 8-wave
                 dense_gemm_kernel), and the vendor library's torch.mm on the row-major operands;
      moe     -- exl3_moe_coop, 256 experts, 16 tokens, twice;
      moes    -- the token-sorted exl3_moe on the same experts, T = 512 and 2048;
      qwenm   -- the row-batched matrix-core GEMV (gemvm_kernel) on the configs[2] shapes 5120 -> 17408
                 and 17408 -> 5120, K = 4 3INST, M = 4 and 8, twice each."""
    import torch
    from ampstein_amd import ops, bundles
    torch.cuda.set_device(0)
    ops.init(0)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    if workload in ("decode", "gateup"):
        layers = make_stack(torch, 4)
        if workload == "gateup":
            gu_out = torch.empty((2, 1, 14336), dtype=torch.half, device="cuda")
            x = host_normal(torch, (1, 1, 4096), 2005)
            for _ in range(2):
                for row in layers:
                    bundles.Multi([row["gate"], row["up"]], gu_out).run(x)
        else:
            sw = Sweep(torch, layers, bundled=True)
            stream = torch.cuda.Stream()
            for _ in range(2):
                sw.run(torch, stream)
    elif workload == "prefill":
        for si, (k, n) in enumerate(((8192, 28672), (28672, 8192))):
            t, s, v = host_trellis(torch, k, n, 4, 4000 + si)
            x = host_normal(torch, (2048, k), 4010 + si)
            C = torch.empty((2048, n), dtype=torch.half, device="cuda")
            wt = torch.empty((n, k), dtype=torch.half, device="cuda")
            for _ in range(2):
                ops.exl3_gemm(x, t, C, s, torch.empty_like(x), v)
            for _ in range(2):
                ops.exl3_gemm_recon(x, t, s, v, 4.0, fused_rows=1 << 30)
                ops.reconstruct_t(wt, t, 4.0)
                ops.recon_mm(x, wt, C)
            del t, s, v, x, C, wt
    elif workload == "dense":
        from ampstein_amd import _lib
        for k, n in ((28672, 8192), (8192, 28672)):
            x = host_normal(torch, (2048, k), 4020)
            wt = host_normal(torch, (n, k), 4021)
            C = torch.empty((2048, n), dtype=torch.half, device="cuda")
            xs, wts = ops.slabs_of(x), ops.slabs_of(wt)
            for _ in range(2):
                ops.recon_mm(xs, wts, C)              # the route's form: k slabs, buffer DMAs
            for var in (_lib.RECON_MM_GLOBAL_DMA, _lib.RECON_MM_8WAVES):
                with _lib.policy(_lib.POLICY_RECON_MM, var):
                    for _ in range(2):
                        ops.recon_mm(x, wt, C)        # row-major operands
            del xs, wts
            for _ in range(2):
                torch.mm(x, wt.t(), out=C)            # the vendor library's default solution
            del x, wt, C
    elif workload == "moe":
        moe_bench(torch, reps=1, ms=(16,), token_sorted=False, graph=False)
    elif workload == "moes":
        moe_bench(torch, reps=1, ms=(), token_sorted=True, graph=False)
    elif workload == "qwenm":
        for si, (k, n) in enumerate(((5120, 17408), (17408, 5120))):
            t, s, v = host_trellis(torch, k, n, 4, 5000 + si)
            for m in (4, 8):
                x = host_normal(torch, (m, k), 5010 + m)
                C = torch.empty((m, n), dtype=torch.half, device="cuda")
                for _ in range(2):
                    ops.exl3_gemm(x, t, C, s, torch.empty_like(x), v)
    torch.cuda.synchronize()
    return 0


# MI355X: 32 shader engines (SQ_BUSY_CYCLES is summed over them), 1024 SIMDs, and a wave64 VALU
# instruction holds its SIMD for 4 cycles
N_SE, N_SIMD, VALU_CYCLES = 32, 1024, 4


def summarize_pmc(outdirs):
    """Per (kernel, grid) average of every counter per dispatch over one or more rocprofv3 --pmc
    output directories (one per counter pass; this library's kernels and the calibration copy),
    then derived figures:
      cycles      SQ_BUSY_CYCLES / 32 (per shader engine: the dispatch's busy cycles)
      valu_busy   4 * SQ_INSTS_VALU / (1024 SIMDs * cycles)
      mfma_busy   SQ_VALU_MFMA_BUSY_CYCLES / (1024 * cycles)
      wait_share  SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (share of wave time waiting on a dependency)
      lds_conflict  SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS
      fetch/write MiB  FETCH_SIZE and WRITE_SIZE scaled by the copy calibration (the copy of
                  COPY_BYTES in the same run reads FETCH = COPY_BYTES / 2, WRITE = COPY_BYTES)."""
    acc = {}
    for outdir in outdirs:
        for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for r in csv.DictReader(f):
                    name = r["Kernel_Name"]
                    if not any(key in name for key in ("gemv", "gemm", "moe_", "moes_", "moeg", "reconstruct", "had128", "copy", "Copy", "Cijk")):
                        continue
                    key = (name.replace("(anonymous namespace)::", "").split("(")[0][:80], r.get("Grid_Size", ""))
                    d = acc.setdefault(key, {}).setdefault(r["Counter_Name"], {})
                    disp = (outdir, r.get("Dispatch_Id", r.get("Correlation_Id")))
                    d[disp] = d.get(disp, 0.0) + float(r["Counter_Value"])
    avg = {k: {c: sum(v.values()) / len(v) for c, v in ctrs.items()} for k, ctrs in acc.items()}
    ndisp = {k: max(len(v) for v in ctrs.values()) for k, ctrs in acc.items()}
    copies = [(int(g or 0), a) for (n, g), a in avg.items() if "copy" in n.lower()]
    cal = max(copies)[1] if copies else {}
    fscale = COPY_BYTES / (cal["FETCH_SIZE"] * 1024.0) if cal.get("FETCH_SIZE") else None
    wscale = COPY_BYTES / (cal["WRITE_SIZE"] * 1024.0) if cal.get("WRITE_SIZE") else None
    for (name, grid), a in sorted(avg.items()):
        if "copy" in name.lower() and a is not cal:
            continue
        print(f"{name}  grid {grid}  ({ndisp[(name, grid)]} dispatches)")
        for cname in sorted(a):
            print(f"    {cname:32s} avg {a[cname]:16.1f}")
        out = []
        cyc = a.get("SQ_BUSY_CYCLES", 0.0) / N_SE
        if cyc:
            out.append(f"cycles {cyc:.0f}")
            if "SQ_INSTS_VALU" in a:
                out.append(f"valu_busy {VALU_CYCLES * a['SQ_INSTS_VALU'] / (N_SIMD * cyc):.3f}")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in a:
                out.append(f"mfma_busy {a['SQ_VALU_MFMA_BUSY_CYCLES'] / (N_SIMD * cyc):.3f}")
        if a.get("SQ_WAVE_CYCLES"):
            out.append(f"wait_share {a.get('SQ_WAIT_INST_ANY', 0.0) / a['SQ_WAVE_CYCLES']:.3f}")
        if a.get("SQ_ACTIVE_INST_LDS"):
            out.append(f"lds_conflict {a.get('SQ_LDS_BANK_CONFLICT', 0.0) / a['SQ_ACTIVE_INST_LDS']:.3f}")
        if fscale and "FETCH_SIZE" in a:
            out.append(f"fetch_MiB {a['FETCH_SIZE'] * 1024.0 * fscale / 2**20:.2f}")
        if wscale and "WRITE_SIZE" in a:
            out.append(f"write_MiB {a['WRITE_SIZE'] * 1024.0 * wscale / 2**20:.2f}")
        if out:
            print("    derived: " + ", ".join(out))
    if fscale or wscale:
        print(f"copy calibration: FETCH_SIZE x {fscale}, WRITE_SIZE x {wscale} (copy of {COPY_BYTES} bytes)")
    return 0


def _counter_rows(outdir, counter):
    rows = []
    for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((r["Kernel_Name"], float(r["Counter_Value"])))
    return rows


def measure_traffic(gemv_alg_bytes_per_launch):
    """FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the GEMV launches, each scaled by the
    same counter's reading on a copy of COPY_BYTES.  Returns the traffic object or None."""
    prof = shutil.which("rocprofv3")
    if not prof:
        return None
    res = {}
    env = dict(os.environ, TMPDIR="/tmp")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        outdir = tempfile.mkdtemp(prefix=f"exl3_{counter}_", dir="/tmp")
        cmd = ["timeout", "-s", "KILL", "120", prof, "--pmc", counter, "--output-format", "csv", "-d", outdir,
               "--", sys.executable, os.path.abspath(__file__), "--pmc-child", "gateup"]
        p = subprocess.run(cmd, capture_output=True, text=True, env=env, cwd="/tmp")
        if p.returncode != 0:
            return {"error": f"rocprofv3 {counter} pass failed (rc {p.returncode})"}
        rows = _counter_rows(outdir, counter)
        copy = [v for name, v in rows if "copy" in name.lower()]
        gemv = [v for name, v in rows if GEMV_KERNEL in name]
        shutil.rmtree(outdir, ignore_errors=True)
        if not copy or not gemv:
            return {"error": f"{counter}: no copy or GEMV dispatches in the profile"}
        scale = COPY_BYTES / (max(copy) * 1024.0)
        res[counter] = (sum(gemv) / len(gemv) * 1024.0 * scale, scale, len(gemv))
    fetch, fscale, n = res["FETCH_SIZE"]
    write, wscale, _ = res["WRITE_SIZE"]
    return {"bytes_per_launch": round(fetch + write), "fetch_bytes": round(fetch), "write_bytes": round(write),
            "copy_scale": {"FETCH_SIZE": round(fscale, 4), "WRITE_SIZE": round(wscale, 4)},
            "dispatches": n, "algorithmic_bytes_per_launch": round(gemv_alg_bytes_per_launch),
            "ratio_to_algorithmic": round((fetch + write) / gemv_alg_bytes_per_launch, 4)}


# ------------------------------------------------------------------ main
def summarize_trace(path, gap_ms=0.0):
    """Per (kernel, grid) average durations of a rocprofv3 --kernel-trace csv (this library's
    kernels only): the figures the roofline's avg_launch_us is checked against.  gap_ms > 0:
    one table per phase, phases split where the GPU idles longer than gap_ms between kernels
    (bench.py --decode-step leaves such gaps between its variants)."""
    recs = []
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if not any(key in name for key in ("gemv", "reconstruct", "had128", "gemm", "moe_", "moes_", "moeg", "rms_norm",
                                               "silu_mul", "res_sq", "norm_sq", "Cijk")):
                continue
            grid = (r.get("Grid_Size_X") or r.get("Grid_Size"), r.get("Grid_Size_Y", "1"))
            recs.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), name, grid))
    recs.sort()
    phases, last_end = [[]], None
    for t0, t1, name, grid in recs:
        if gap_ms > 0 and last_end is not None and t0 - last_end > gap_ms * 1e6:
            phases.append([])
        phases[-1].append((t0, t1, name, grid))
        last_end = t1 if last_end is None else max(last_end, t1)
    for pi, ph in enumerate(phases):
        stats = {}
        for t0, t1, name, grid in ph:
            stats.setdefault((name, grid), []).append(t1 - t0)
        if gap_ms > 0:
            print(f"phase {pi}: {len(ph)} dispatches over {(ph[-1][1] - ph[0][0]) / 1e3:.0f} us")
        print(f"{'kernel':60s} {'grid (threads x, y)':>22s} {'calls':>6s} {'avg us':>9s} {'min us':>9s} {'max us':>9s}")
        for (name, grid), ds in sorted(stats.items(), key=lambda kv: -sum(kv[1])):
            print(f"{name[:60]:60s} {str(grid):>22s} {len(ds):6d} {sum(ds) / len(ds) / 1e3:9.2f} "
                  f"{min(ds) / 1e3:9.2f} {max(ds) / 1e3:9.2f}")
    return 0


RATE_OPS = ["v_bfe_u32", "v_mad_u64_u32", "v_bitop3_b32", "v_mad_u32_u16", "v_perm_b32", "v_alignbit_b32",
            "v_dot2_f32_f16", "v_pk_fma_f16", "v_add_u32", "v_mul_lo_u32"]


def recon_rows():
    """Prefill and medium-batch routes by row count (4 bpw 3INST unless noted, x N(0,1)): per shape
    and rows, us per call of exl3_gemm as 16-row GEMV groups (force_shape_idx 1, up to 192 rows),
    exl3_gemm on the MFMA GEMM (force 2: k split when its tiles fill at most half the CUs), the
    recon route's rotated branch (exl3_gemm_recon: x rotation, reconstruct, dense GEMM with its own
    split k) and the same route without the split (policy EXL3_AMD_RECON_MM_NO_SPLIT).  One JSON
    line per shape; null where a route is not timed."""
    import torch
    from ampstein_amd import ops, _lib
    torch.cuda.set_device(0)
    ops.init(0)
    shapes = ((4096, 4096, 4), (4096, 14336, 4), (14336, 4096, 4), (5120, 5120, 2), (17408, 5120, 4),
              (8192, 28672, 4), (28672, 8192, 4))
    for si, (k, n, K) in enumerate(shapes):
        t, s, v = host_trellis(torch, k, n, K, 7000 + si)
        row = {"shape": f"{k}x{n}", "K": K, "us": "gemv groups / mfma gemm / recon (split k) / recon (no split)"}
        for m in (16, 32, 64, 128, 192, 512, 2048):
            x = host_normal(torch, (m, k), 7100 + m)
            C = torch.empty((m, n), dtype=torch.half, device="cuda")
            ah = torch.empty_like(x)
            g = timed(torch, lambda: ops.exl3_gemm(x, t, C, s, ah, v, 1)) if m <= 192 else None
            f = timed(torch, lambda: ops.exl3_gemm(x, t, C, s, ah, v, 2))
            r = timed(torch, lambda: ops.exl3_gemm_recon(x, t, s, v, float(K), fused_rows=1 << 30))
            with _lib.policy(_lib.POLICY_RECON_MM, _lib.RECON_MM_NO_SPLIT):
                r0 = timed(torch, lambda: ops.exl3_gemm_recon(x, t, s, v, float(K), fused_rows=1 << 30))
            row[str(m)] = [None if g is None else round(g, 1), round(f, 1), round(r, 1), round(r0, 1)]
        print(json.dumps(row), flush=True)
        del t, s, v
        torch.cuda.empty_cache()
    # the recon route's two branches at prefill sizes (configs[3] shapes): the reference's fused W
    # (reconstruct_had, dense GEMM) and the rotated one (x rotated, reconstruct, GEMM, y rotated
    # in the epilogue); TFLOPS of the best of 3 timings of 5 calls each
    for si, (k, n) in enumerate(((8192, 28672), (28672, 8192))):
        t, s, v = host_trellis(torch, k, n, 4, 7300 + si)
        row = {"shape": f"{k}x{n}", "K": 4, "TFLOPS": "fused W / rotated"}
        for m in (2048, 4096, 8192):
            x = host_normal(torch, (m, k), 7400 + m)
            best = []
            for fr in (0, 1 << 30):
                best.append(min(timed(torch, lambda: ops.exl3_gemm_recon(x, t, s, v, 4.0, fused_rows=fr)) for _ in range(3)))
            row[str(m)] = [round(2.0 * m * k * n / (us * 1e-6) / 1e12, 1) for us in best]
            del x
            torch.cuda.empty_cache()
        print(json.dumps(row), flush=True)
        del t, s, v
    return 0


def rates():
    """Issue rates of single VALU instruction kinds (8 independent chains per lane, 4 waves per
    SIMD on every CU) and of random 16-bit LDS gathers from a 128 KiB table (one 1024-thread
    workgroup per CU), from ampstein_amd/lib/libexl3_probe.so.  Rates are wave64 instructions per
    SIMD per ns; `rel` divides by v_bfe_u32's rate (clock-independent)."""
    import ctypes
    import torch
    from ampstein_amd import build as B
    assert torch.cuda.is_available(), "bench.py --rates needs a GPU"
    torch.cuda.set_device(0)
    L = ctypes.CDLL(B.PROBE_LIB)
    L.exl3_probe_valu.restype = ctypes.c_float
    L.exl3_probe_valu.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    L.exl3_probe_lds_gather.restype = ctypes.c_float
    L.exl3_probe_lds_gather.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_lane = L.exl3_probe_chains()
    blocks, iters = 4 * cus, 4000                       # 4 workgroups of 4 waves per CU: 4 waves per SIMD
    out = torch.zeros(16 * blocks, dtype=torch.int32, device="cuda")
    simds = 4 * cus
    res = {"cus": cus, "waves_per_simd": 4, "valu": {}}
    for op, name in enumerate(RATE_OPS):
        best = None
        for _ in range(3):
            ms = L.exl3_probe_valu(op, out.data_ptr(), blocks, iters)
            assert ms > 0, f"probe {name} failed"
            best = ms if best is None else min(best, ms)
        insts = blocks * 4 * iters * per_lane              # wave instructions
        res["valu"][name] = {"ms": round(best, 3), "per_simd_per_ns": round(insts / simds / (best * 1e6), 4)}
    base = res["valu"]["v_bfe_u32"]["per_simd_per_ns"]
    for name in RATE_OPS:
        res["valu"][name]["rel"] = round(res["valu"][name]["per_simd_per_ns"] / base, 3)
    g_iters = 1000
    lds = {}
    for mode, name in ((0, "gather"), (1, "valu_only")):
        best = None
        for _ in range(3):
            ms = L.exl3_probe_lds_gather(out.data_ptr(), cus, g_iters, mode)
            assert ms > 0, "lds probe failed"
            best = ms if best is None else min(best, ms)
        gathers = cus * 16 * g_iters * per_lane            # wave-level ds_read_u16 instructions
        lds[name] = {"ms": round(best, 3), "wave_gathers_per_cu_per_ns": round(gathers / cus / (best * 1e6), 4),
                     "weights_per_s": round(gathers * 64 / (best * 1e-3) / 1e12, 3)}
    lds["note"] = "weights_per_s in T/s: 64 lanes x wave gathers; one 16-bit table entry per weight"
    res["lds_gather_128k"] = lds
    # read-only streaming at the decode GEMV's launch sizes, 24 launches over distinct buffers in
    # one graph (HIP events around the replays): contiguous per wave vs the GEMV's column order
    L.exl3_probe_stream.restype = ctypes.c_int
    L.exl3_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                    ctypes.c_void_p, ctypes.c_void_p]
    streams = {}
    for name, nbytes, row_bytes, wgs in (("q_4096x4096", 8 << 20, 32 << 10, 512),
                                         ("down_14336x4096", 28 << 20, 32 << 10, 448),
                                         ("gate_up_2x4096x14336", 56 << 20, 112 << 10, 896)):
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i) for i in range(24)]
        sink = torch.zeros(wgs * 4, dtype=torch.int32, device="cuda")
        row = {}
        for pattern in (0, 1):
            st = torch.cuda.Stream()
            def seq():
                for b in bufs:
                    rc = L.exl3_probe_stream(b.data_ptr(), nbytes, wgs, pattern, row_bytes, sink.data_ptr(), st.cuda_stream)
                    assert rc == 0, rc
            with torch.cuda.stream(st):
                seq()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=st):
                seq()
            gr.replay(); torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                gr.replay()
            e1.record(); torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (5 * len(bufs))
            row["contiguous" if pattern == 0 else "gemv_order"] = {"us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1)}
        row["workgroups"] = wgs
        streams[name] = row
        del bufs
        torch.cuda.empty_cache()
    res["stream_read"] = streams
    print(json.dumps(res))
    return 0


def main():
    args = parse()
    if args.rates:
        return rates()
    if args.recon_rows:
        return recon_rows()
    if args.decode_step:
        import torch
        from ampstein_amd import ops
        torch.cuda.set_device(0)
        ops.init(0)
        print(json.dumps(decode_step_bench(torch, make_stack(torch, args.layers), gap_s=0.3)), flush=True)
        return 0
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace, args.gap_ms)
    if args.summarize_pmc:
        return summarize_pmc(args.summarize_pmc)
    if args.pmc_child:
        return pmc_child(args.pmc_child)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the EXL3 path runs on a single MI355X; a multi-GPU split is design-only in this build)")
        return 2

    # the profiled child launches the stacked gate/up mgemm: 2 x 4096 x 14336 weights at 4 bits
    alg_per_launch = 2 * 4096 * 14336 / 2
    traffic = None if args.no_traffic else measure_traffic(alg_per_launch)

    import torch
    from ampstein_amd import ops
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    ops.init(0)
    layers = make_stack(torch, args.layers)
    bundled = Sweep(torch, layers, bundled=True)
    separate = Sweep(torch, layers, bundled=False)

    # launch durations (HIP events on the launch stream)
    ev_b = event_times(torch, bundled)
    ev_s = event_times(torch, separate)
    dom_us, dom_bytes, dom_n = dominant_region(torch, layers)
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9

    def per_label(ev):
        out = {}
        for label, nbytes, ms in ev:
            d = out.setdefault(label, [nbytes, []])
            d[1].append(ms)
        res = {}
        for label, (nbytes, mss) in out.items():
            us = sum(mss) / len(mss) * 1e3
            res[label] = {"bytes": nbytes, "us": round(us, 2), "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                          "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        return res

    ms_step, wall = graph_time(torch, bundled, args.steps, args.warmup)
    value = bundled.bytes / (ms_step * 1e-3) / 1e9
    ms_sep, _ = graph_time(torch, separate, max(5, args.steps // 5), 2)

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
        "config": {"workload": "llama3-8b-decode-sweep (configs[1])", "layers": args.layers, "bpw": 4,
                   "codebook": "3inst", "m": 1, "launches_per_step": len(bundled.entries),
                   "schedule": "qkv sliced mgemm, o gemm, gate/up stacked mgemm, down gemm",
                   "packed_bytes_per_step": bundled.bytes, "launch": "hip-graph replay"},
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm",
                     "kernel": "gemv1_kernel<4,0,8> as the stacked gate/up exl3_mgemm (2 x 4096x14336, grid 896x2 workgroups, 8 k-slices per wave)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes_per_launch"] if traffic and "bytes_per_launch" in traffic else None,
                     "avg_launch_us": round(dom_us, 3), "algorithmic_bytes_per_launch": dom_bytes,
                     "launches_timed": dom_n},
        "traffic_detail": traffic,
        "per_launch_bundled": per_label(ev_b),
        "per_shape": per_label(ev_s),
        "sweep_separate_gemm": {"ms_per_step": round(ms_sep, 4),
                                "GB_s": round(separate.bytes / (ms_sep * 1e-3) / 1e9, 1),
                                "launches_per_step": len(separate.entries)},
        "wall_s": round(wall, 3),
    }
    del bundled, separate
    out["decode_step"] = decode_step_bench(torch, layers)
    del layers
    torch.cuda.empty_cache()
    if not args.no_prefill:
        out["prefill"] = prefill_bench(torch)
    if not args.no_moe:
        out["moe"] = moe_bench(torch)
    if not args.no_qwen:
        out["qwen27b"] = qwen_bench(torch)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
