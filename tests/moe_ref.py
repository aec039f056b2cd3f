"""Test-side model of exl3_moe_coop (the reference's semantics, exl3_moe_coop_kernel.cuh): fp64
arithmetic on the oracle's bit-exact W_hat, with the kernel's fp16 rounding points (rotated gate
/ up input, rotated activation).  Also the host statement of the run table and a synthetic expert
set with its device pointer tables."""
import numpy as np
import scipy.special
from scipy.linalg import hadamard

from ampstein_amd import synth

H128 = hadamard(128).astype(np.float64) / np.sqrt(128.0)


def had(v):
    """Hadamard-128 over each 128-chunk of the last axis (orthonormal, natural order)."""
    sh = v.shape
    return (v.reshape(*sh[:-1], sh[-1] // 128, 128) @ H128).reshape(sh)


def f16(v):
    return np.asarray(v, np.float64).astype(np.float16).astype(np.float64)


def act_fn(act, gated, g, u, limit, gelu_erf=False):
    """act_gate of exl3_moe_coop_kernel.cuh:115-129 (GELU as its tanh form, or with gelu_erf the
    erf form of the reference's CPU forward, cpu/moe_mul1.cpp:2196-2201)."""
    if act == 3:
        if limit != 0.0:
            g = np.minimum(g, limit)
            u = np.clip(u, -limit, limit)
        return (u + 1.0) * (g / (1.0 + np.exp(-1.702 * g)))
    if not gated:
        x = np.maximum(0.0, u)
    elif act == 0:
        x = g / (1.0 + np.exp(-g))
    elif act == 1 and gelu_erf:
        x = 0.5 * g * (1.0 + scipy.special.erf(g / np.sqrt(2.0)))
    elif act == 1:
        x = 0.5 * g * (1.0 + np.tanh(0.797884560803 * (g + 0.044715 * g ** 3)))
    else:
        x = np.maximum(0.0, g) ** 2
    if limit != 0.0:
        u = np.clip(u, -limit, limit)
        x = np.minimum(x, limit)
    return x * u


def project(xp, W, suh, svh, bias, round16):
    """One expert projection: had(xp * suh) (rounded to fp16 when round16) @ W_hat, had, * svh,
    + bias."""
    hx = had(xp * suh)
    if round16:
        hx = f16(hx)
    y = had(hx @ W) * svh
    return y + bias if bias is not None else y


def expert_out(xp, W, sv, bias, act, gated, limit, round16=True, gelu_erf=False):
    """gate / up projections, activation, down projection of one expert for one row.
    W = (Wg, Wu, Wd) W_hat matrices, sv = ((suh, svh) per projection), bias per projection or
    None.  round16 applies the fp16 rounding points of the fused kernels (rotated inputs)."""
    uu = project(xp, W[1], *sv[1], bias[1], round16)
    gg = project(xp, W[0], *sv[0], bias[0], round16) if gated else uu
    return project(act_fn(act, gated, gg, uu, limit, gelu_erf), W[2], *sv[2], bias[2], round16)


class ExpertSet:
    """n experts: gate/up (Hi -> I) and down (I -> Ho) synthetic EXL3 matrices."""

    def __init__(self, torch, orc, n, Hi, I, Ho, Ks, cb, seed, bias=False):
        rng = np.random.default_rng(seed)
        self.n, self.Hi, self.I, self.Ho, self.cb = n, Hi, I, Ho, cb
        self.K = [float(k) if float(k) != int(k) else int(k) for k in Ks]     # b + 0.5: half rate (mul1)
        self.layers = []
        for e in range(n):
            g = synth.layer(Hi, I, self.K[e], cb, seed=seed * 1000 + 3 * e)
            u = synth.layer(Hi, I, self.K[e], cb, seed=seed * 1000 + 3 * e + 1)
            d = synth.layer(I, Ho, self.K[e], cb, seed=seed * 1000 + 3 * e + 2)
            self.layers.append((g, u, d))
        self.W = [tuple(orc.reconstruct(L.trellis, int(L.K), half=L.K != int(L.K), cb=cb).astype(np.float64)
                        for L in trio) for trio in self.layers]
        self.dev = [tuple(L.torch() for L in trio) for trio in self.layers]
        P = lambda v: torch.tensor(v, dtype=torch.long, device="cuda")
        self.tables = {}
        for pi, name in enumerate("gud"):
            self.tables[name + "_trellis"] = P([self.dev[e][pi][0].data_ptr() for e in range(n)])
            self.tables[name + "_suh"] = P([self.dev[e][pi][1].data_ptr() for e in range(n)])
            self.tables[name + "_svh"] = P([self.dev[e][pi][2].data_ptr() for e in range(n)])
        self.bits = {name: torch.tensor([int(k) for k in self.K], dtype=torch.uint8, device="cuda") for name in "gud"}
        self.bias_np = None
        if bias:
            self.bias_np = [tuple((rng.standard_normal(w) * 0.1).astype(np.float16) for w in (I, I, Ho)) for _ in range(n)]
            self.bias_dev = [tuple(torch.from_numpy(b).cuda() for b in trio) for trio in self.bias_np]
            for pi, name in enumerate("gud"):
                self.tables[name + "_bias"] = P([self.bias_dev[e][pi].data_ptr() for e in range(n)])

    def slot_out(self, x_row, e, act, gated, limit, use_bias=False):
        """One slot's down output (before the routing weight), fp64 with fp16 rounding points."""
        xp = np.zeros(self.Hi)
        xp[: x_row.shape[0]] = x_row
        sv = [(L.suh.astype(np.float64), L.svh.astype(np.float64)) for L in self.layers[e]]
        bias = [None] * 3
        if use_bias and self.bias_np is not None:
            bias = [b.astype(np.float64) for b in self.bias_np[e]]
        return expert_out(xp, self.W[e], sv, bias, act, gated, limit)


def active(sel, rw, mn, mx):
    ok = rw.astype(np.float32) != 0
    if mn >= 0:
        ok &= (sel >= mn) & (sel < mx)
    return ok


def reference(es, x, sel, rw, mn, mx, act, gated, limit, H_out, sh_out=None, sh_gate_w=None, use_bias=False):
    bsz, topk = sel.shape
    out = np.zeros((bsz, H_out))
    ok = active(sel, rw, mn, mx)
    for t in range(bsz):
        acc = np.zeros(es.Ho)
        for k in range(topk):
            if ok[t, k]:
                e = int(sel[t, k]) - (mn if mn >= 0 else 0)
                acc += float(rw[t, k]) * es.slot_out(x[t].astype(np.float64), e, act, gated, limit, use_bias)
        if sh_out is not None:
            gv = 1.0
            if sh_gate_w is not None:
                gv = 1.0 / (1.0 + np.exp(-float(x[t].astype(np.float64) @ sh_gate_w.astype(np.float64))))
            acc[: sh_out.shape[1]] += gv * sh_out[t]
        out[t] = acc[:H_out]
    return out


def host_runs(sel, rw, mn, mx, rows=8):
    """(n_runs, run_start[], order[]): active slots sorted by (local expert, slot), runs of at most
    `rows` slots of one expert."""
    ok = active(sel, rw, mn, mx).reshape(-1)
    loc = sel.reshape(-1) - (mn if mn >= 0 else 0)
    order = sorted([s for s in range(ok.size) if ok[s]], key=lambda s: (loc[s], s))
    starts, prev, cnt = [], None, 0
    for i, s in enumerate(order):
        if loc[s] != prev or cnt == rows:
            starts.append(i)
            prev, cnt = loc[s], 0
        cnt += 1
    return len(starts), starts + [len(order)], order


def routing(T, E, topk, seed, sentinel=0):
    """Top-k routing of T tokens over E experts (distinct experts per token); `sentinel`
    assignments get the id E (the reference's "less than top-k" bin)."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, E))
    sel = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    rw = np.take_along_axis(p, sel, axis=1).astype(np.float16)
    flat = sel.reshape(-1).astype(np.int64)
    if sentinel:
        flat[rng.choice(flat.size, sentinel, replace=False)] = E
    order = np.argsort(flat, kind="stable")
    token_sorted = (order // topk).astype(np.int64)
    weight_sorted = rw.reshape(-1)[order]
    count = np.bincount(flat, minlength=E + 1).astype(np.int64)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    start = np.concatenate([[0], np.cumsum(count)[:-1]]).astype(np.int64)
    return flat, order, inv, token_sorted, weight_sorted, count, start
