"""Test-side model of exl3_moe_coop (the reference's semantics, exl3_moe_coop_kernel.cuh): fp64
arithmetic on the oracle's bit-exact W_hat, with the kernel's fp16 rounding points (rotated gate
/ up input, rotated activation).  Also the host statement of the run table and a synthetic expert
set with its device pointer tables."""
import numpy as np
from scipy.linalg import hadamard

from ampstein_amd import synth

H128 = hadamard(128).astype(np.float64) / np.sqrt(128.0)


def had(v):
    """Hadamard-128 over each 128-chunk of the last axis (orthonormal, natural order)."""
    sh = v.shape
    return (v.reshape(*sh[:-1], sh[-1] // 128, 128) @ H128).reshape(sh)


def f16(v):
    return np.asarray(v, np.float64).astype(np.float16).astype(np.float64)


def act_fn(act, gated, g, u, limit):
    if act == 3:
        if limit != 0.0:
            g = np.minimum(g, limit)
            u = np.clip(u, -limit, limit)
        return (u + 1.0) * (g / (1.0 + np.exp(-1.702 * g)))
    if not gated:
        x = np.maximum(0.0, u)
    elif act == 0:
        x = g / (1.0 + np.exp(-g))
    elif act == 1:
        x = 0.5 * g * (1.0 + np.tanh(0.797884560803 * (g + 0.044715 * g ** 3)))
    else:
        x = np.maximum(0.0, g) ** 2
    if limit != 0.0:
        u = np.clip(u, -limit, limit)
        x = np.minimum(x, limit)
    return x * u


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
        (g, u, d), (Wg, Wu, Wd) = self.layers[e], self.W[e]
        xp = np.zeros(self.Hi)
        xp[: x_row.shape[0]] = x_row
        def proj(L, W, bias):
            hx = f16(had(xp * L.suh.astype(np.float64)))
            y = had(hx @ W) * L.svh.astype(np.float64)
            return y + (bias.astype(np.float64) if bias is not None else 0.0)
        bg, bu, bd = self.bias_np[e] if (use_bias and self.bias_np is not None) else (None, None, None)
        uu = proj(u, Wu, bu)
        gg = proj(g, Wg, bg) if gated else uu
        a = act_fn(act, gated, gg, uu, limit)
        ad = f16(had(a * d.suh.astype(np.float64)))
        v = had(ad @ Wd) * d.svh.astype(np.float64)
        return v + (bd.astype(np.float64) if bd is not None else 0.0)


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
