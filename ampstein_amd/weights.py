"""Model weights over safetensors files, as the engine's weights.uc opens them
(src/ucode/ampstein/weights.uc:39-84, :134-270):

    single file:  <dir>/model.safetensors
    sharded HF:   <dir>/model.safetensors.index.json, whose "weight_map" routes every key
                  to a shard file (model-00001-of-00002.safetensors, ...)

Shards are opened lazily on first access to one of their keys and read through memory maps
(safetensors' own loader: nothing in the file is executed).  gpu() / gpu16() upload a tensor
on first touch and cache the device copy per (key, device), like ws.gpu / ws.gpu16.

The reader of the reference is a C module over mmap (src/torch/st.c); this one delegates the
file format to the safetensors package, which parses the same header (little-endian u64
length, JSON header with dtype / shape / data_offsets per key, then the raw bytes).
"""
from __future__ import annotations

import json
import os
from typing import Dict, List, Optional

import torch
from safetensors import safe_open

INDEX_NAME = "model.safetensors.index.json"
SINGLE_NAME = "model.safetensors"


class WeightsError(KeyError):
    """Unknown key or malformed index: the reference dies with the same messages."""


def _dev(dev) -> torch.device:
    if dev is None:
        return torch.device("cuda", 0)
    if isinstance(dev, int):
        return torch.device("cuda", dev)
    return torch.device(dev)


class Weights:
    """Key-addressed view of one model directory (weights.uc open())."""

    def __init__(self, model_dir: str, only_file: Optional[str] = None):
        self.dir = model_dir
        self._shards: Dict[str, object] = {}
        self._map: Optional[Dict[str, str]] = None
        self._single: Optional[str] = None
        self._gpu: Dict[tuple, torch.Tensor] = {}
        if only_file:
            self._single = only_file
        elif os.path.exists(os.path.join(model_dir, INDEX_NAME)):
            with open(os.path.join(model_dir, INDEX_NAME)) as f:
                idx = json.load(f)
            wm = idx.get("weight_map")
            if not wm:
                raise WeightsError(f"weights: {INDEX_NAME} has no weight_map")
            self._map = dict(wm)
        else:
            self._single = SINGLE_NAME
        if self._single is not None:
            self._keys = list(self._file(self._single).keys())

    # ---- file routing ------------------------------------------------------------------
    def _file(self, name: str):
        f = self._shards.get(name)
        if f is None:
            f = safe_open(os.path.join(self.dir, name), framework="pt", device="cpu")
            self._shards[name] = f
        return f

    def _shard_of(self, key: str) -> str:
        if self._map is not None:
            shard = self._map.get(key)
            if shard is None:
                raise WeightsError(f"weights: unknown key '{key}'")
            return shard
        if key not in self._keys:
            raise WeightsError(f"weights: unknown key '{key}'")
        return self._single

    # ---- the weights.uc interface --------------------------------------------------------
    def has(self, key: str) -> bool:
        return (key in self._map) if self._map is not None else (key in self._keys)

    def list(self) -> List[str]:
        return list(self._map) if self._map is not None else list(self._keys)

    def tensor(self, key: str) -> torch.Tensor:
        """CPU tensor (memory-mapped by the loader)."""
        return self._file(self._shard_of(key)).get_tensor(key)

    def fp16(self, key: str) -> torch.Tensor:
        return self.tensor(key).to(torch.float16)

    def info(self, key: str) -> dict:
        """{shape, dtype} without reading the tensor's bytes."""
        sl = self._file(self._shard_of(key)).get_slice(key)
        return {"shape": list(sl.get_shape()), "dtype": sl.get_dtype()}

    def gpu(self, key: str, dev=None) -> torch.Tensor:
        d = _dev(dev)
        ck = (key, str(d), None)
        t = self._gpu.get(ck)
        if t is None:
            t = self.tensor(key).to(d)
            self._gpu[ck] = t
        return t

    def gpu16(self, key: str, dev=None) -> torch.Tensor:
        """Device copy cast to fp16 on the device (the raw upload is cached too)."""
        d = _dev(dev)
        ck = (key, str(d), torch.float16)
        t = self._gpu.get(ck)
        if t is None:
            raw = self.gpu(key, dev)
            t = raw if raw.dtype == torch.float16 else raw.to(torch.float16)
            self._gpu[ck] = t
        return t

    def release(self, key: str, dev=None) -> None:
        self._gpu.pop((key, str(_dev(dev)), None), None)

    def drop(self, key: str, dev=None) -> None:
        d = str(_dev(dev))
        for ck in [c for c in self._gpu if c[0] == key and c[1] == d]:
            del self._gpu[ck]


def open_weights(model_dir: str, only_file: Optional[str] = None) -> Weights:
    """weights.uc open(model_dir, only_file)."""
    return Weights(model_dir, only_file)
