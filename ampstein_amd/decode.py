"""The linear part of a Llama-family decode step, captured into one HIP graph
(src/ucode/ampstein/graphdec.uc:151-230, step_ops).

Per layer, on persistent buffers and without host synchronisation:
    h, r = rms_norm_res(h, res, input_layernorm)         res = previous down output (zero first)
    q, k, v = sliced mgemm(r)                            one launch (models.sliced)
    o = exl3_gemm(attn)                                  attention itself is outside this path:
                                                         the q projection stands in for its output
    h, r = rms_norm_res(h, o, post_attention_layernorm)
    gate, up = stacked mgemm(r)                          one launch (models.multi)
    d = exl3_gemm(silu(gate) * up)                       one launch: the M = 1 GEMV forms the
                                                         SwiGLU product in its input load
and finally h, out = rms_norm_res(h, d_last, norm).  `fuse_swiglu=False` runs silu_mul and
exl3_gemm as two launches, as graphdec.uc does.  `fuse_norm=True` also folds each residual
norm into the GEMV before it (o_proj with the post-attention norm, down_proj with the next
layer's input norm or the final norm): the wave that completes the row's last column chunk
normalises the row, and 4 launches per layer remain.  `split_norm=True` divides each residual
norm between its neighbours instead: o_proj and down_proj add the residual in their chunk
epilogue and keep each chunk's sum of squares (exl3_gemm_res), and the next bundle (q/k/v,
gate/up) normalises its input while loading it (mgemm with norm_in); 4 launches per layer, no
serial pass, plus one launch at each end of the step (the first layer's sums, the final norm).
The split norm is the default (the fastest form measured); `split_norm=False` runs the
reference's own sequence of rms_norm_res calls.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch

from . import bundles, ops


@dataclass
class LayerWeights:
    q: bundles.Linear
    k: bundles.Linear
    v: bundles.Linear
    o: bundles.Linear
    gate: bundles.Linear
    up: bundles.Linear
    down: bundles.Linear
    input_norm: torch.Tensor          # (hidden) fp16
    post_norm: torch.Tensor           # (hidden) fp16


class DecodeStack:
    def __init__(self, layers: List[LayerWeights], final_norm: torch.Tensor, eps: float = 1e-5,
                 fuse_swiglu: bool = True, fuse_norm: bool = False, split_norm: bool = True):
        dev = final_norm.device
        L0 = layers[0]
        self.hidden = L0.q.in_features
        self.inter = L0.gate.out_features
        self.layers, self.final_norm, self.eps, self.fuse = layers, final_norm, eps, fuse_swiglu
        # fuse_norm asks for the other form of the same fusion (the norm in the GEMV's last chunk)
        self.fuse_norm, self.split_norm = fuse_norm, split_norm and not fuse_norm
        z = lambda *sh: torch.zeros(sh, dtype=torch.half, device=dev)
        H, I = self.hidden, self.inter
        self.x_in = z(1, H)
        self.h = z(1, H)
        self.r = z(1, H)
        self.out = z(1, H)
        self.zero = z(1, H)
        self.act = z(1, I)
        self.a_had_h = z(1, H)
        self.a_had_i = z(1, I)
        self.sq = torch.zeros((1, H // 128), dtype=torch.float, device=dev)
        self.qkv, self.gu, self.qbuf, self.oout, self.guout, self.dout = [], [], [], [], [], []
        for Lw in layers:
            qb, kb, vb = z(1, 1, Lw.q.out_features), z(1, 1, Lw.k.out_features), z(1, 1, Lw.v.out_features)
            gu = torch.zeros((2, 1, I), dtype=torch.half, device=dev)
            self.qbuf.append(qb)
            self.oout.append(z(1, H))
            self.guout.append(gu)
            self.dout.append(z(1, H))
            self.qkv.append(bundles.Sliced([Lw.q, Lw.k, Lw.v], [qb, kb, vb]))
            self.gu.append(bundles.Multi([Lw.gate, Lw.up], gu))
        self.graph = None

    def _linear(self, lin, x, y, a_had):
        ops.exl3_gemm(x, lin.trellis, y, lin.suh, a_had, lin.svh, 0, lin.mcg, lin.mul1)

    def step_ops(self) -> torch.Tensor:
        """One decode step over the current contents of x_in; returns the final normed row."""
        h, r, eps = self.h, self.r, self.eps
        h.copy_(self.x_in)
        nl = len(self.layers)
        if self.split_norm:
            sq = self.sq
            ops.res_sq(h, None, sq)
            for i, Lw in enumerate(self.layers):
                self.qkv[i].run(h.view(1, 1, -1), norm_in=(sq, Lw.input_norm, eps, r))
                o = Lw.o
                ops.exl3_gemm_res(self.qbuf[i].view(1, -1), o.trellis, self.oout[i], o.suh, o.svh, h, sq,
                                  o.mcg, o.mul1, A_had=self.a_had_h)
                self.gu[i].run(h.view(1, 1, -1), norm_in=(sq, Lw.post_norm, eps, r))
                dn = Lw.down
                g, u = self.guout[i][0], self.guout[i][1]
                if self.fuse:
                    ops.exl3_gemm_res(g, dn.trellis, self.dout[i], dn.suh, dn.svh, h, sq, dn.mcg, dn.mul1,
                                      up=u, act=self.act, A_had=self.a_had_i)
                else:
                    ops.silu_mul(g, u, out=self.act)
                    ops.exl3_gemm_res(self.act, dn.trellis, self.dout[i], dn.suh, dn.svh, h, sq, dn.mcg, dn.mul1,
                                      A_had=self.a_had_i)
            ops.norm_sq(h, sq, self.final_norm, eps, r=self.out)
            return self.out
        if self.fuse_norm:
            ops.rms_norm_res(h, self.zero, self.layers[0].input_norm, eps, y=h, n=r)
        for i, Lw in enumerate(self.layers):
            if self.fuse_norm:
                self.qkv[i].run(r.view(1, 1, -1))
                o = Lw.o
                ops.exl3_gemm_norm(self.qbuf[i].view(1, -1), o.trellis, self.oout[i], o.suh, o.svh, h, Lw.post_norm,
                                   r, eps, o.mcg, o.mul1, A_had=self.a_had_h)
                self.gu[i].run(r.view(1, 1, -1))
                dn = Lw.down
                last = i == nl - 1
                ops.exl3_gemm_norm(self.guout[i][0], dn.trellis, self.dout[i], dn.suh, dn.svh, h,
                                   self.final_norm if last else self.layers[i + 1].input_norm,
                                   self.out if last else r, eps, dn.mcg, dn.mul1,
                                   up=self.guout[i][1], act=self.act, A_had=self.a_had_i)
                continue
            res = self.zero if i == 0 else self.dout[i - 1]
            ops.rms_norm_res(h, res, Lw.input_norm, eps, y=h, n=r)
            self.qkv[i].run(r.view(1, 1, -1))
            self._linear(Lw.o, self.qbuf[i].view(1, -1), self.oout[i], self.a_had_h)
            ops.rms_norm_res(h, self.oout[i], Lw.post_norm, eps, y=h, n=r)
            self.gu[i].run(r.view(1, 1, -1))
            g, u = self.guout[i][0], self.guout[i][1]
            dn = Lw.down
            if self.fuse:
                ops.exl3_gemm_silu_mul(g, u, dn.trellis, self.dout[i], dn.suh, dn.svh, dn.mcg, dn.mul1,
                                       act=self.act, A_had=self.a_had_i)
            else:
                ops.silu_mul(g, u, out=self.act)
                self._linear(dn, self.act, self.dout[i], self.a_had_i)
        if not self.fuse_norm:
            ops.rms_norm_res(h, self.dout[-1], self.final_norm, eps, y=h, n=self.out)
        return self.out

    def capture(self) -> None:
        """Warm up eagerly on a side stream, then capture step_ops into one graph."""
        ops.init(self.h.device.index or 0)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step_ops()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self.step_ops()
        torch.cuda.synchronize()

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        self.x_in.copy_(x.view(1, -1))
        if self.graph is None:
            return self.step_ops()
        self.graph.replay()
        return self.out
