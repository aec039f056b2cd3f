"""Token-sorted MoE (exl3_moe, exl3_moe.cu:137-418) and its fixed-order reduction
(exl3_moe_gather, exl3_moe.cu:420-531) through the C ABI.

The model restates exl3_moe_kernel.cuh:78-313 in fp64 on the oracle's bit-exact W_hat, with the
kernel's fp16 rounding points: rotated gate / up inputs, gate / up GEMM outputs, the rotated
activation (had_hf_r_128_guad_inner), the down GEMM output; the last rotation, routing weight and
svh stay fp32 (had_hf_r_128_d_inner).  Bar: max |y - ref| / max |ref| < 2e-3.  The gather is
checked bit for bit on exactly representable values.
"""
import numpy as np
import pytest
import torch

from ampstein_amd import _lib
from tests.moe_ref import ExpertSet, act_fn, f16, had, routing

pytestmark = pytest.mark.gpu


def model_row(es, x_row, e, act, limit):
    """One assignment's down output before the routing weight (fp64, fused-kernel rounding)."""
    (g, u, d), (Wg, Wu, Wd) = es.layers[e], es.W[e]
    gated = act != 2
    xr = x_row.astype(np.float64)
    hu = f16(had(xr * u.suh.astype(np.float64)))
    uu = f16(f16(had(f16(hu @ Wu))) * u.svh.astype(np.float64))
    if gated:
        hg = f16(had(xr * g.suh.astype(np.float64)))
        gg = f16(f16(had(f16(hg @ Wg))) * g.svh.astype(np.float64))
    else:
        gg = np.zeros_like(uu)
    if act == 0:
        ga = f16(gg / (1.0 + np.exp(-gg)))
    elif act == 1:
        ga = f16(0.5 * gg * (1.0 + np.tanh(0.797884560803 * (gg + 0.044715 * gg ** 3))))
    elif act == 2:
        ga = np.maximum(uu, 0.0)
    else:
        ga = gg
    if limit != 0.0:
        L = float(np.float16(limit))
        uu = np.clip(uu, -L, L)
        ga = np.minimum(ga, L)
    a = f16(f16(ga * uu) * d.suh.astype(np.float64))
    ad = f16(had(a))
    D = f16(ad @ Wd)
    return had(D) * d.svh.astype(np.float64)


def model(es, x, flat, token_sorted, weight_sorted, count, start, max_tok, lo, hi, act, limit):
    T, H = x.shape
    out = np.zeros((T, H))
    slot_rows = {}
    for e in range(es.n):
        c = int(count[e])
        if not (0 < c <= max_tok and lo <= c <= hi):
            continue
        for j in range(c):
            pos = int(start[e]) + j
            t = int(token_sorted[pos])
            y = model_row(es, x[t], e, act, limit) * float(weight_sorted[pos])
            out[t] += y
            slot_rows[(e, j)] = y
    return out, slot_rows


def run_moe(es, x, rt, max_tok, concurrency, lo, hi, act, limit, Ks, scratch_mode=False, m_tile=16, poison=False):
    flat, order, inv, token_sorted, weight_sorted, count, start = rt
    from ampstein_amd import ops
    T, H = x.shape
    I = es.I
    dev = "cuda"
    xs = torch.from_numpy(x).to(dev)
    out = torch.zeros((T, H), dtype=torch.float, device=dev)
    ts = [torch.zeros((concurrency, max_tok, H), dtype=torch.half, device=dev) for _ in range(2)]
    ti = [torch.zeros((concurrency, max_tok, I), dtype=torch.half, device=dev) for _ in range(2)]
    tb = es.tables
    mcg, mul1 = es.cb == 1, es.cb == 2
    bits = (None, None, None)
    Kg = Ku = Kd = 0.0
    if len(set(Ks)) > 1:
        bits = (es.bits["g"], es.bits["u"], es.bits["d"])
    else:
        Kg = Ku = Kd = float(Ks[0])
    elig = [e for e in range(es.n) if 0 < count[e] <= max_tok and lo <= count[e] <= hi]
    scratch = fused_base = None
    if scratch_mode:
        fb = np.zeros(es.n, np.int64)
        acc = 0
        for e in range(es.n):
            fb[e] = acc
            if e in elig:
                acc += int(count[e])
        scratch = torch.full((max(acc, 1), H), float("nan"), dtype=torch.float, device=dev)
        fused_base = torch.from_numpy(fb).to(dev)
    if poison:       # every workspace int -1, every fp32 NaN: any read of state this call did not write shows
        _lib.check(_lib.lib().exl3_amd_debug_fill_workspace(torch.cuda.current_device(), 0xFF))
    ops.exl3_moe(xs, out, torch.from_numpy(count).to(dev), torch.from_numpy(token_sorted).to(dev),
                 torch.from_numpy(weight_sorted).to(dev), ts[0], ts[1], ti[0], ti[1], act, Kg, Ku, Kd,
                 tb["g_trellis"], tb["g_suh"], tb["g_svh"], tb["u_trellis"], tb["u_suh"], tb["u_svh"],
                 tb["d_trellis"], tb["d_suh"], tb["d_svh"], mcg, mul1, mcg, mul1, mcg, mul1,
                 limit, len(elig), scratch, fused_base, lo, hi, m_tile, *bits)
    torch.cuda.synchronize()
    return out, scratch, fused_base, elig


CASES = [
    # name, E, H, I, T, topk, cb, Ks, act, limit, max_tok, concurrency, lo, hi, sentinel
    ("mcg-k3-silu-3pass", 8, 256, 384, 40, 2, 1, [3] * 8, 0, 0.0, 32, 1, 0, 1 << 30, 0),
    ("mul1-mixed-gelu", 8, 256, 256, 48, 3, 2, [2, 3, 4, 2, 3, 4, 4, 2], 1, 0.0, 64, 2, 0, 1 << 30, 3),
    ("mul1-k4-relu2-limit", 6, 384, 256, 30, 2, 2, [4] * 6, 2, 4.0, 64, 1, 0, 1 << 30, 0),
    ("mcg-k2-range", 8, 256, 256, 64, 2, 1, [2] * 8, 0, 6.0, 20, 2, 12, 18, 0),
    ("mul1-k5-many-rows", 2, 256, 256, 300, 2, 2, [5, 5], 0, 0.0, 320, 2, 0, 1 << 30, 0),
    # half rates (mul1): the MFMA tiles' 1.5 / 2.5 / 3.5 decode, 64- and 256-row tiles
    ("mul1-k1.5-silu", 8, 256, 256, 48, 2, 2, [1.5] * 8, 0, 0.0, 64, 2, 0, 1 << 30, 0),
    ("mul1-k2.5-gelu", 8, 256, 384, 48, 3, 2, [2.5] * 8, 1, 0.0, 64, 2, 0, 1 << 30, 2),
    ("mul1-k3.5-many-rows", 2, 256, 256, 300, 2, 2, [3.5, 3.5], 0, 0.0, 320, 2, 0, 1 << 30, 0),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_exl3_moe(orc, case, poison=False):
    name, E, H, I, T, topk, cb, Ks, act, limit, max_tok, conc, lo, hi, sentinel = case
    print(f"exl3_moe case {name}", flush=True)
    es = ExpertSet(torch, orc, E, H, I, H, Ks, cb, seed=CASES.index(case) + 31)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, H)).astype(np.float16)
    rt = routing(T, E, topk, seed=len(name), sentinel=sentinel)
    flat, order, inv, token_sorted, weight_sorted, count, start = rt
    out, _, _, elig = run_moe(es, x, rt, max_tok, conc, lo, hi, act, limit, Ks, poison=poison)
    ref, _ = model(es, x, flat, token_sorted, weight_sorted, count, start, max_tok, lo, hi, act, limit)
    y = out.cpu().numpy().astype(np.float64)
    assert np.isfinite(y).all(), "non-finite output"
    assert len(elig) > 0
    touched = np.abs(ref).sum(axis=1) > 0
    assert np.all(y[~touched] == 0.0), "rows without an in-range expert must stay untouched"
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"  experts in range {len(elig)}/{E}, rel err {err:.2e}", flush=True)
    assert err < 2e-3


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_exl3_moe_poisoned_workspace(orc, case):
    """The same cases with the library workspace filled with 0xff bytes before the call (plan
    ints -1, chunk sums NaN): the call reads only state it wrote, so the results are unchanged."""
    test_exl3_moe(orc, case, poison=True)


READBACK_CASES = [CASES[0], CASES[5], CASES[1]]


@pytest.mark.parametrize("case", READBACK_CASES, ids=[c[0] for c in READBACK_CASES])
def test_exl3_moe_plan_readback(orc, case):
    """The plan the GPU built for the call's last pass (row map, row tiles, per (matrix, rate)
    tile lists and counts, per-token position lists, position -> row map) read back from the
    workspace and compared with the host model (tests/moe_plan_model.py): identical, except that
    the order within a tile list is the order of LDS atomics and is compared as a set."""
    from tests import moe_plan_model as pm
    name, E, H, I, T, topk, cb, Ks, act, limit, max_tok, conc, lo, hi, sentinel = case
    es = ExpertSet(torch, orc, E, H, I, H, Ks, cb, seed=CASES.index(case) + 31)
    x = np.random.default_rng(5).standard_normal((T, H)).astype(np.float16)
    rt = routing(T, E, topk, seed=len(name), sentinel=sentinel)
    flat, order, inv, token_sorted, weight_sorted, count, start = rt
    run_moe(es, x, rt, max_tok, conc, lo, hi, act, limit, Ks, poison=True)
    num_assign = len(token_sorted)
    pool = min(conc * max_tok, num_assign)
    tr = pm.tile_rows_for(num_assign, E)
    lay = pm.Layout(E, T, num_assign, H, I, pool, tr, True)
    codes = [pm.rate_code(k) for k in Ks]
    w0 = ((num_assign - 1) // pool) * pool                     # the last pass
    info, tiles, lists, invd, total = pm.plan(count, E, num_assign, max_tok, lo, hi, pool, tr, w0, [codes] * 3)
    dev = torch.cuda.current_device()

    def ints(off, n):
        buf = np.empty(max(n, 1), np.int32)
        _lib.check(_lib.lib().exl3_amd_debug_read_workspace(dev, 4 * off, 4 * n, buf.ctypes.data))
        return buf[:n]

    assert np.array_equal(ints(lay.rowinfo, 3 * pool).reshape(pool, 3), info.astype(np.int32))
    assert np.array_equal(ints(lay.rt, 3 * len(tiles)).reshape(-1, 3), np.array(tiles, np.int32).reshape(-1, 3))
    counts = ints(lay.counts, 3 * pm.MOES_RATES).reshape(3, pm.MOES_RATES)
    for m in range(3):
        for s_ in range(pm.MOES_RATES):
            assert counts[m, s_] == len(lists[m][s_]), (m, s_)
            got = ints(lay.lists + (m * pm.MOES_RATES + s_) * lay.rt_cap, int(counts[m, s_]))
            assert sorted(got.tolist()) == sorted(lists[m][s_]), (m, s_)
    tstart, tpos = pm.tokens(token_sorted, T)
    assert np.array_equal(ints(lay.tok_start, T + 1), tstart)
    assert np.array_equal(ints(lay.tok_pos, len(tpos)), tpos)
    inv_row = ints(lay.inv_row, num_assign)
    for pos_, r in invd.items():
        assert inv_row[pos_] == r, pos_


@pytest.mark.parametrize("case", CASES[:3], ids=[c[0] for c in CASES[:3]])
def test_exl3_moe_atomic_output(orc, kernel_policy, case):
    """The atomic output kernel (used when the per-token lists do not fit one workgroup's LDS),
    forced: the same cases, the same bar."""
    kernel_policy(_lib.POLICY_MOE_OUTPUT, _lib.MOE_OUTPUT_ATOMIC)
    test_exl3_moe(orc, case)


TILE_CASES = [
    # ~80 rows per expert: 32- and 64-row tiles split every expert, 96 and 128 hold most whole
    ("mul1-mixed-80rows", 4, 256, 256, 160, 2, 2, [2, 3, 4, 2], 0, 0.0, 256, 1, 0, 1 << 30, 0),
    ("mul1-k2.5-80rows", 4, 256, 384, 160, 2, 2, [2.5] * 4, 1, 0.0, 256, 1, 0, 1 << 30, 0),
]


@pytest.mark.parametrize("tile_rows", [32, 64, 96, 128])
@pytest.mark.parametrize("case", TILE_CASES, ids=[c[0] for c in TILE_CASES])
def test_exl3_moe_tile_rows(orc, kernel_policy, case, tile_rows):
    """Every row-tile size of the grouped GEMM (16-row groups R = 2, 4, 6, 8) against the model."""
    kernel_policy(_lib.POLICY_MOE_TILE_ROWS, tile_rows)
    name, E, H, I, T, topk, cb, Ks, act, limit, max_tok, conc, lo, hi, sentinel = case
    es = ExpertSet(torch, orc, E, H, I, H, Ks, cb, seed=TILE_CASES.index(case) + 71)
    x = np.random.default_rng(7).standard_normal((T, H)).astype(np.float16)
    rt = routing(T, E, topk, seed=len(name) + 1, sentinel=sentinel)
    flat, order, inv, token_sorted, weight_sorted, count, start = rt
    out, _, _, elig = run_moe(es, x, rt, max_tok, conc, lo, hi, act, limit, Ks)
    ref, _ = model(es, x, flat, token_sorted, weight_sorted, count, start, max_tok, lo, hi, act, limit)
    y = out.cpu().numpy().astype(np.float64)
    assert count.max() > 64, "the case must put more than 64 rows on some expert"
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"  {name} tile {tile_rows}: max rows {count.max()}, rel err {err:.2e}", flush=True)
    assert err < 2e-3


def test_exl3_moe_slots_and_gather(orc):
    """Deterministic mode: slot outputs against the model per (expert, row); then the fixed-order
    gather sums them into the token rows; two runs are bit-identical."""
    from ampstein_amd import ops
    E, H, I, T, topk = 8, 256, 256, 40, 2
    Ks = [3, 4, 2, 3, 4, 2, 3, 4]
    es = ExpertSet(torch, orc, E, H, I, H, Ks, 2, seed=77)
    x = np.random.default_rng(9).standard_normal((T, H)).astype(np.float16)
    rt = routing(T, E, topk, seed=11, sentinel=2)
    flat, order, inv, token_sorted, weight_sorted, count, start = rt
    max_tok, lo, hi = 64, 0, 1 << 30
    ref, slot_rows = model(es, x, flat, token_sorted, weight_sorted, count, start, max_tok, lo, hi, 0, 0.0)
    outs = []
    for rep in range(2):
        out, scratch, fused_base, elig = run_moe(es, x, rt, max_tok, 1, lo, hi, 0, 0.0, Ks, scratch_mode=True)
        assert float(out.abs().max()) == 0.0, "slot mode leaves output_state alone"
        sc = scratch.cpu().numpy().astype(np.float64)
        fb = fused_base.cpu().numpy()
        worst = 0.0
        for (e, j), y in slot_rows.items():
            worst = max(worst, np.abs(sc[fb[e] + j] - y).max())
        scale = max(np.abs(v).max() for v in slot_rows.values())
        assert worst / scale < 2e-3, worst / scale
        kind = np.array([1 if e in elig else 0 for e in range(E)], np.int64)
        dev = "cuda"
        T_ = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
        ops.exl3_moe_gather(out, scratch, T_(flat), T_(inv), T_(start), fused_base, T_(kind), T_(weight_sorted))
        torch.cuda.synchronize()
        y = out.cpu().numpy().astype(np.float64)
        err = np.abs(y - ref).max() / np.abs(ref).max()
        assert err < 2e-3, err
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_exl3_moe_gather_exact():
    """Slot resolution, kinds, sentinel experts and k order, on values where every product and
    sum is exact: the result must match bit for bit."""
    from ampstein_amd import ops
    rng = np.random.default_rng(3)
    T, topk, E, H = 37, 4, 6, 200
    flat = rng.integers(0, E + 1, size=T * topk).astype(np.int64)      # E = sentinel, skipped
    order = np.argsort(flat, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    count = np.bincount(flat, minlength=E + 1)
    start = np.concatenate([[0], np.cumsum(count)[:-1]]).astype(np.int64)
    kind = np.array([1, 2, 0, 2, 1, 2], np.int64)
    slot_base = np.zeros(E, np.int64)
    acc = 0
    for e in range(E):
        slot_base[e] = acc
        acc += int(count[e])
    scratch = rng.integers(-64, 64, size=(acc, H)).astype(np.float32)
    weight_sorted = (rng.integers(-8, 8, size=T * topk) / 4.0).astype(np.float16)
    out0 = rng.integers(-16, 16, size=(T, H)).astype(np.float32)
    exp = out0.astype(np.float64).copy()
    for t in range(T):
        s = 0.0
        for k in range(topk):
            a = t * topk + k
            e = flat[a]
            if e >= E or kind[e] == 0:
                continue
            pos = inv[a]
            wt = float(weight_sorted[pos]) if kind[e] == 2 else 1.0
            s += scratch[slot_base[e] + pos - start[e]].astype(np.float64) * wt
        exp[t] += s
    dev = "cuda"
    T_ = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
    out = T_(out0)
    ops.exl3_moe_gather(out, T_(scratch), T_(flat), T_(inv), T_(start), T_(slot_base), T_(kind), T_(weight_sorted))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), exp.astype(np.float32))


def test_exl3_moe_edges(orc):
    """No expert in range leaves the output alone; one token; a pool of 5 rows so that experts
    straddle pass boundaries (rows of one expert in two passes)."""
    E, H, I = 4, 128, 256
    es = ExpertSet(torch, orc, E, H, I, H, [2, 3, 4, 2], 2, seed=90)
    x1 = np.random.default_rng(1).standard_normal((1, H)).astype(np.float16)
    rt1 = routing(1, E, 2, seed=2)
    Ks = [2, 3, 4, 2]
    out, _, _, elig = run_moe(es, x1, rt1, 8, 1, 0, 1 << 30, 0, 0.0, Ks)
    ref, _ = model(es, x1, rt1[0], rt1[3], rt1[4], rt1[5], rt1[6], 8, 0, 1 << 30, 0, 0.0)
    assert np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max() < 2e-3
    x = np.random.default_rng(3).standard_normal((12, H)).astype(np.float16)
    rt = routing(12, E, 2, seed=4)
    out, _, _, elig = run_moe(es, x, rt, 5, 1, 100, 200, 0, 0.0, Ks)       # count range excludes all
    assert elig == [] or float(out.abs().max()) == 0.0
    # max_tok 13 holds every expert (24 assignments over 4 experts), pool = 13 rows -> 2 passes
    out, _, _, elig = run_moe(es, x, rt, 13, 1, 0, 1 << 30, 1, 0.0, Ks)
    ref, _ = model(es, x, rt[0], rt[3], rt[4], rt[5], rt[6], 13, 0, 1 << 30, 1, 0.0)
    assert len(elig) == E
    assert np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max() < 2e-3
