"""CPU check of the token-sorted MoE's index structures (tests/moe_plan_model.py): for every
configuration of the GPU tests and a seeded sweep of random ones (multi-pass pools of any size,
experts straddling passes, count ranges, sentinel assignments, empty tokens, mixed and half
rates, gated and gateless), every read of workspace state or pool rows by the plan, gather,
grouped GEMM, activation and output kernels hits memory written earlier in the same pass, stale
position -> row entries are always rejected by the output kernel's guard, row tiles cover each
live pool row exactly once, and every in-range assignment reaches the output exactly once.
"""
import numpy as np
import pytest

from tests.moe_plan_model import rate_code, simulate
from tests.moe_ref import routing

# name, E, H, I, T, topk, Ks, act, max_tok, concurrency, lo, hi, sentinel (tests/test_gpu_moe_sorted.py)
GPU_CASES = [
    ("mcg-k3-silu-3pass", 8, 256, 384, 40, 2, [3] * 8, 0, 32, 1, 0, 1 << 30, 0),
    ("mul1-mixed-gelu", 8, 256, 256, 48, 3, [2, 3, 4, 2, 3, 4, 4, 2], 1, 64, 2, 0, 1 << 30, 3),
    ("mul1-k4-relu2-limit", 6, 384, 256, 30, 2, [4] * 6, 2, 64, 1, 0, 1 << 30, 0),
    ("mcg-k2-range", 8, 256, 256, 64, 2, [2] * 8, 0, 20, 2, 12, 18, 0),
    ("mul1-k5-many-rows", 2, 256, 256, 300, 2, [5, 5], 0, 320, 2, 0, 1 << 30, 0),
    ("mul1-k1.5-silu", 8, 256, 256, 48, 2, [1.5] * 8, 0, 64, 2, 0, 1 << 30, 0),
    ("mul1-k2.5-gelu", 8, 256, 384, 48, 3, [2.5] * 8, 1, 64, 2, 0, 1 << 30, 2),
    ("mul1-k3.5-many-rows", 2, 256, 256, 300, 2, [3.5, 3.5], 0, 320, 2, 0, 1 << 30, 0),
]


def check(E, H, I, T, topk, Ks, act, max_tok, conc, lo, hi, sentinel, seed, tile_rows=None, tok_mode=True):
    flat, order, inv, token_sorted, weight_sorted, count, start = routing(T, E, topk, seed=seed, sentinel=sentinel)
    codes = [rate_code(k) for k in Ks]
    Kcodes = [codes, codes, codes]
    contrib, lay = simulate(count, token_sorted, T, E, H, I, max_tok, conc, lo, hi, Kcodes, gated=act != 2,
                            tile_rows=tile_rows, tok_mode=tok_mode)
    # every assignment of an in-range expert contributes once; the rest (sentinel, out of range) never
    exp = np.zeros(len(token_sorted), np.int64)
    for e in range(E):
        c = int(count[e])
        if 0 < c <= max_tok and lo <= c <= hi:
            exp[int(start[e]):int(start[e]) + c] = 1
    assert np.array_equal(contrib, exp)
    return lay


@pytest.mark.parametrize("case", GPU_CASES, ids=[c[0] for c in GPU_CASES])
@pytest.mark.parametrize("tok_mode", [True, False], ids=["token-major", "atomic"])
def test_gpu_case_index_walk(case, tok_mode):
    name, E, H, I, T, topk, Ks, act, max_tok, conc, lo, hi, sentinel = case
    check(E, H, I, T, topk, Ks, act, max_tok, conc, lo, hi, sentinel, seed=len(name), tok_mode=tok_mode)


@pytest.mark.parametrize("tile_rows", [32, 64, 96, 128])
def test_tile_sizes_index_walk(tile_rows):
    check(4, 256, 256, 160, 2, [2, 3, 4, 2], 0, 256, 1, 0, 1 << 30, 0, seed=18, tile_rows=tile_rows)
    check(4, 256, 384, 160, 2, [2.5] * 4, 1, 256, 1, 0, 1 << 30, 0, seed=17, tile_rows=tile_rows)


def test_edges_index_walk():
    """One token; a count range that excludes every expert; a 5- and a 13-row pool (experts
    straddle pass boundaries, the last pass partly empty)."""
    check(4, 128, 256, 1, 2, [2, 3, 4, 2], 0, 8, 1, 0, 1 << 30, 0, seed=2)
    check(4, 128, 256, 12, 2, [2, 3, 4, 2], 0, 5, 1, 100, 200, 0, seed=4)
    check(4, 128, 256, 12, 2, [2, 3, 4, 2], 1, 13, 1, 0, 1 << 30, 0, seed=4)
    check(4, 128, 256, 12, 2, [2, 3, 4, 2], 1, 5, 1, 0, 1 << 30, 0, seed=4)


def test_random_index_walks():
    rng = np.random.default_rng(2024)
    for it in range(120):
        E = int(rng.integers(1, 40))
        topk = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.integers(1, 200))
        Ks = [float(rng.choice([1.5, 2, 2.5, 3, 3.5, 4, 5, 8])) for _ in range(E)]
        max_tok = int(rng.integers(1, 2 * T * topk // max(E, 1) + 3))
        conc = int(rng.integers(1, 4))
        lo = int(rng.integers(0, 3))
        hi = int(rng.integers(lo, 2 * max_tok + 2))
        sentinel = int(rng.integers(0, min(5, T * topk) + 1))
        act = int(rng.integers(0, 3))
        tile_rows = int(rng.choice([0, 32, 64, 96, 128]))
        check(E, 128 * int(rng.integers(1, 4)), 128 * int(rng.integers(1, 4)), T, topk, Ks, act, max_tok, conc,
              lo, hi, sentinel, seed=it, tile_rows=tile_rows or None, tok_mode=bool(rng.integers(0, 2)))
