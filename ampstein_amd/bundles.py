"""Linear bundles of the decode step: several EXL3 linears sharing one input, run as ONE
exl3_mgemm launch -- the engine's models.multi / models.sliced (src/ucode/ampstein/models.uc:
338-430), which graphdec.uc:168-196 uses for q/k/v and gate/up.

A linear here is any object with .trellis (k/16, n/16, 16K) int16, .suh (k) fp16, .svh (n) fp16
CUDA tensors and .K, .mcg, .mul1, .in_features, .out_features.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ops


@dataclass
class Linear:
    trellis: torch.Tensor
    suh: torch.Tensor
    svh: torch.Tensor
    K: float = 4.0
    mcg: bool = False
    mul1: bool = False

    @property
    def in_features(self) -> int:
        return self.trellis.size(0) * 16

    @property
    def out_features(self) -> int:
        return self.trellis.size(1) * 16


def _check(linears):
    """Fused linears share K, codebook and in_features (models.uc:315-335)."""
    L0 = linears[0]
    for i, w in enumerate(linears[1:], 1):
        if (w.K, w.mul1, w.mcg, w.in_features) != (L0.K, L0.mul1, L0.mcg, L0.in_features):
            raise ValueError(f"bundle: fused linears must share K, in_features and codebook (matrix {i})")


def _ptrs(vals, device):
    return torch.tensor(vals, dtype=torch.long, device=device)


class Multi:
    """Equal-width bundle (gate/up): run(x) writes all outputs stacked into out (num, m, n)."""

    def __init__(self, linears, out: torch.Tensor):
        _check(linears)
        dev = out.device
        self.out = out
        self.B = _ptrs([w.trellis.data_ptr() for w in linears], dev)
        self.suh = _ptrs([w.suh.data_ptr() for w in linears], dev)
        self.svh = _ptrs([w.svh.data_ptr() for w in linears], dev)
        self.A_had = torch.zeros((len(linears), out.size(1), linears[0].in_features), dtype=torch.half, device=dev)
        self.K, self.mcg, self.mul1 = linears[0].K, linears[0].mcg, linears[0].mul1

    def run(self, x: torch.Tensor, norm_in=None) -> torch.Tensor:
        return ops.mgemm(x, self.B, self.out, self.suh, self.A_had, self.svh, self.K, self.mcg, self.mul1,
                         norm_in=norm_in)


class Sliced:
    """Unequal-width bundle (q/k/v): every linear cut into column slices of width gcd(widths);
    run(x) writes every slice in place into its output buffer (outs[i]: (1, m, n_i))."""

    def __init__(self, linears, outs):
        _check(linears)
        width = 0
        for w in linears:
            width = math.gcd(width, w.out_features)
        if width % 128 or width < 128:
            raise ValueError(f"sliced: unsuitable slice width {width}")
        dev = outs[0].device
        t_ptr, svh_ptr, c_ptr, stride, src = [], [], [], [], []
        for i, w in enumerate(linears):
            tw = w.trellis.size(2)
            for n0 in range(0, w.out_features, width):
                t_ptr.append(w.trellis.data_ptr() + (n0 // 16) * tw * 2)
                svh_ptr.append(w.svh.data_ptr() + n0 * 2)
                c_ptr.append(outs[i].data_ptr() + n0 * 2)
                stride.append(w.out_features)
                src.append(i)
        m = outs[0].size(-2)
        self.width = width
        self.slices = len(t_ptr)
        self.B = _ptrs(t_ptr, dev)
        self.svh = _ptrs(svh_ptr, dev)
        self.suh = _ptrs([w.suh.data_ptr() for w in linears], dev)
        i32 = lambda v: torch.tensor(v, dtype=torch.int32, device=dev)
        self.opts = {"size_n_list": i32([width] * len(t_ptr)), "c_ptrs": _ptrs(c_ptr, dev),
                     "n_stride_list": i32(stride), "had_src_list": i32(src), "num_had_src": len(linears)}
        self.carrier = torch.zeros((len(t_ptr), m, width), dtype=torch.half, device=dev)
        self.A_had = torch.zeros((len(linears), m, linears[0].in_features), dtype=torch.half, device=dev)
        self.K, self.mcg, self.mul1 = linears[0].K, linears[0].mcg, linears[0].mul1
        self.outs = outs

    def run(self, x: torch.Tensor, norm_in=None):
        ops.mgemm(x, self.B, self.carrier, self.suh, self.A_had, self.svh, self.K, self.mcg, self.mul1, self.opts,
                  norm_in=norm_in)
        return self.outs
