"""Checkpoint loader and LinearEXL3 (weights.uc, models.uc:29-110).

CPU: a synthetic EXL3 checkpoint written with safetensors, single-file and sharded (index
json), read back key by key; K / codebook / feature counts derived from the trellis shape and
the marker tensors, and the reference's rejections (both markers, half K without mul1,
unknown key).  GPU: forward() on both routes (decode GEMM at few rows, reconstruct + dense
GEMM above 144 rows), with and without bias, against the CPU oracle's fp64 linear.
"""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from ampstein_amd import synth
from ampstein_amd.weights import WeightsError, open_weights


def _layer_tensors(key, L, mul1=False, mcg=False, bias=None):
    d = {key + ".trellis": torch.from_numpy(L.trellis.view(np.int16).copy()),
         key + ".suh": torch.from_numpy(L.suh.copy()),
         key + ".svh": torch.from_numpy(L.svh.copy())}
    if mul1:
        d[key + ".mul1"] = torch.zeros(1, dtype=torch.int8)
    if mcg:
        d[key + ".mcg"] = torch.zeros(1, dtype=torch.int8)
    if bias is not None:
        d[key + ".bias"] = torch.from_numpy(bias.copy())
    return d


def _write_model(tmp, tensors, sharded):
    if not sharded:
        save_file(tensors, os.path.join(tmp, "model.safetensors"))
        return
    keys = sorted(tensors)
    half = len(keys) // 2
    wm = {}
    for i, part in enumerate((keys[:half], keys[half:])):
        name = f"model-0000{i + 1}-of-00002.safetensors"
        save_file({k: tensors[k] for k in part}, os.path.join(tmp, name))
        wm.update({k: name for k in part})
    with open(os.path.join(tmp, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)


@pytest.mark.parametrize("sharded", [False, True])
def test_weights_reader(tmp_path, sharded):
    La = synth.layer(256, 128, 4, 0, seed=1)
    Lb = synth.layer(128, 256, 2.5, 2, seed=2)
    t = {}
    t.update(_layer_tensors("a", La))
    t.update(_layer_tensors("b", Lb, mul1=True))
    _write_model(str(tmp_path), t, sharded)
    ws = open_weights(str(tmp_path))
    assert sorted(ws.list()) == sorted(t)
    assert ws.has("a.trellis") and not ws.has("a.mul1") and ws.has("b.mul1")
    assert ws.info("b.trellis") == {"shape": [8, 16, 40], "dtype": "I16"}
    assert np.array_equal(ws.tensor("a.trellis").numpy().view(np.uint16), La.trellis)
    assert np.array_equal(ws.fp16("b.suh").numpy(), Lb.suh)
    with pytest.raises(WeightsError):
        ws.tensor("c.trellis")


def test_weights_index_without_map(tmp_path):
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}}, f)
    with pytest.raises(WeightsError, match="no weight_map"):
        open_weights(str(tmp_path))


class _CpuWeights:
    """The loader with device uploads left on the host, for the CPU-side derivation checks."""

    def __init__(self, ws):
        self.ws = ws

    def __getattr__(self, name):
        return getattr(self.ws, name)

    def gpu(self, key, dev=None):
        return self.ws.tensor(key)

    def gpu16(self, key, dev=None):
        return self.ws.fp16(key)


@pytest.mark.parametrize("K,cb", [(2, 0), (4, 1), (3.5, 2), (8, 2), (1.5, 2)])
def test_linear_derivation(tmp_path, K, cb):
    from ampstein_amd.linear import LinearEXL3
    L = synth.layer(256, 384, K, cb, seed=3)
    _write_model(str(tmp_path), _layer_tensors("m.q", L, mul1=cb == 2, mcg=cb == 1), False)
    lin = LinearEXL3(_CpuWeights(open_weights(str(tmp_path))), "m.q")
    assert (lin.K, lin.mul1, lin.mcg) == (float(K), cb == 2, cb == 1)
    assert (lin.in_features, lin.out_features) == (256, 384)
    assert lin.bias is None


def test_linear_rejections(tmp_path):
    from ampstein_amd.linear import LinearEXL3, LinearError
    L = synth.layer(128, 128, 4, 0, seed=4)
    Lh = synth.layer(128, 128, 2.5, 2, seed=5)
    t = {}
    t.update(_layer_tensors("both", L, mul1=True, mcg=True))
    t.update(_layer_tensors("half", Lh))          # half-integer K without the .mul1 marker
    _write_model(str(tmp_path), t, False)
    ws = _CpuWeights(open_weights(str(tmp_path)))
    with pytest.raises(LinearError, match="both .mul1 and .mcg"):
        LinearEXL3(ws, "both")
    with pytest.raises(LinearError, match="tile width 40"):
        LinearEXL3(ws, "half")
    with pytest.raises(WeightsError):
        LinearEXL3(ws, "absent")


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 7, 64, 300])
@pytest.mark.parametrize("K,cb,with_bias", [(4, 0, False), (3, 1, True), (2.5, 2, True)])
def test_linear_forward(tmp_path, orc, rows, K, cb, with_bias):
    from ampstein_amd.linear import LinearEXL3
    k, n = 512, 384
    L = synth.layer(k, n, K, cb, seed=40 + rows)
    rng = np.random.default_rng(7)
    bias = rng.standard_normal(n).astype(np.float16) if with_bias else None
    _write_model(str(tmp_path), _layer_tensors("blk.o", L, mul1=cb == 2, mcg=cb == 1, bias=bias), True)
    lin = LinearEXL3(open_weights(str(tmp_path)), "blk.o", 0)
    x = synth.activations(rows, k, seed=rows)
    y = lin(torch.from_numpy(x).cuda()).float().cpu().numpy().astype(np.float64)
    ref = orc.linear(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb, y_fp32=True).astype(np.float64)
    if bias is not None:
        ref = ref + bias.astype(np.float64)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"linear forward rows={rows} K={K} cb={cb} bias={with_bias}: rel err {err:.2e}", flush=True)
    assert err < 2e-3
