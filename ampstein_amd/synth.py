"""Seeded synthetic EXL3 layers: uniform random trellis words, random +-1 fp16 sign vectors,
N(0, 1) fp16 activations.  One numpy PCG64 generator per (seed), so the CPU oracle and the
GPU see identical bytes.  Seed scheme for benchmark configurations: 1000 * config + index.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# Llama-3-8B decode-stack linears (in_features -> out_features)
LLAMA3_8B_SHAPES = [
    ("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
    ("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096),
]


@dataclass
class SynthLayer:
    trellis: np.ndarray      # uint16 (k/16, n/16, 16K [+8])
    suh: np.ndarray          # float16 (k)
    svh: np.ndarray          # float16 (n)
    k: int
    n: int
    K: float
    cb: int

    @property
    def bits(self) -> int:
        return int(self.K)

    @property
    def half(self) -> bool:
        return self.K != int(self.K)

    @property
    def packed_bytes(self) -> int:
        return self.trellis.nbytes

    def torch(self, device="cuda"):
        import torch
        t = torch.from_numpy(self.trellis.view(np.int16)).to(device)
        s = torch.from_numpy(self.suh).to(device)
        v = torch.from_numpy(self.svh).to(device)
        return t, s, v


def signs(rng: np.random.Generator, n: int) -> np.ndarray:
    return np.where(rng.integers(0, 2, n) > 0, 1.0, -1.0).astype(np.float16)


def layer(k: int, n: int, K: float = 4, cb: int = 0, seed: int = 0) -> SynthLayer:
    rng = np.random.default_rng(seed)
    bits = int(K)
    tu16 = 16 * bits + (8 if K != bits else 0)
    trellis = rng.integers(0, 65536, size=(k // 16, n // 16, tu16), dtype=np.uint16)
    return SynthLayer(trellis, signs(rng, k), signs(rng, n), k, n, K, cb)


def activations(m: int, k: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed + 7919)
    return rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
