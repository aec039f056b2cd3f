"""LinearEXL3: an EXL3 linear layer read from a checkpoint, with the engine's routing between
the decode GEMV / GEMM and the reconstruct + dense GEMM path
(src/ucode/ampstein/models.uc:29-110).

Everything is derived from the trellis tensor, the format's own spec (docs/LESSONS.md L2):
    K            = trellis.shape[-1] / 16   (float divide: tile width 88 is K = 5.5)
    in_features  = trellis.shape[0] * 16
    out_features = trellis.shape[1] * 16
A `.mul1` marker tensor selects the mul1 codebook, a `.mcg` marker the mcg codebook; both at
once is an error, and a half-integer K without mul1 is rejected (models.uc:46-66).

forward(x): more than RECON_ROWS rows and at most RECON_MAX_N output features go through
exl3_gemm_recon; everything else through exl3_gemm into a fresh fp16 output; then + bias.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import bundles, ops
from .weights import Weights

RECON_ROWS = 144       # models.uc:35
RECON_MAX_N = 32768    # models.uc:36


class LinearError(ValueError):
    pass


class LinearEXL3:
    def __init__(self, ws: Weights, key: str, dev=None):
        shape = ws.info(key + ".trellis")["shape"]
        if len(shape) != 3:
            raise LinearError(f"LinearEXL3: {key}: trellis must be 3-D, got shape {shape}")
        rem = shape[2] % 16
        mul1 = ws.has(key + ".mul1")
        mcg = ws.has(key + ".mcg")
        if mul1 and mcg:
            raise LinearError(f"LinearEXL3: {key}: both .mul1 and .mcg marker tensors present")
        if rem != 0 and not mul1:
            raise LinearError(f"LinearEXL3: {key}: half-integer bitrate (tile width {shape[2]}) "
                              "requires mul1 support, not yet implemented")
        self.key = key
        self.dev = 0 if dev is None else dev
        self.trellis = ws.gpu(key + ".trellis", self.dev)
        self.suh = ws.gpu(key + ".suh", self.dev)
        self.svh = ws.gpu(key + ".svh", self.dev)
        self.bias = ws.gpu16(key + ".bias", self.dev) if ws.has(key + ".bias") else None
        self.K = shape[2] / 16.0
        self.mul1 = mul1
        self.mcg = mcg
        self.in_features = shape[0] * 16
        self.out_features = shape[1] * 16

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        m = x.size(0)
        if m > RECON_ROWS and self.out_features <= RECON_MAX_N:
            out = ops.exl3_gemm_recon(x.contiguous(), self.trellis, self.suh, self.svh, self.K,
                                      self.mul1, self.mcg)
        else:
            # exl3_gemm writes every element: no zero fill.  The binding hands the kernel a
            # scratch buffer of x's shape for the rotated input (amp_torch.cpp:11251-11294).
            out = torch.empty((m, self.out_features), dtype=torch.float16, device=x.device)
            ops.exl3_gemm(x, self.trellis, out, self.suh, torch.empty_like(x), self.svh, 0,
                          self.mcg, self.mul1)
        if self.bias is not None:
            out = out.add(self.bias)
        return out

    __call__ = forward


def linear(ws: Weights, key: str, dev=None) -> Optional[LinearEXL3]:
    """models.linear for the EXL3 weight class: a LinearEXL3 when `<key>.trellis` exists."""
    return LinearEXL3(ws, key, dev) if ws.has(key + ".trellis") else None


def multi(linears, out: torch.Tensor) -> bundles.Multi:
    """models.multi (models.uc:338-375): equal-shape bundle, one mgemm launch."""
    return bundles.Multi(linears, out)


def sliced(linears, outs) -> bundles.Sliced:
    """models.sliced (models.uc:377-430): unequal widths cut to gcd-width column slices."""
    return bundles.Sliced(linears, outs)
