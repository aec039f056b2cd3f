"""CPU check of the XCD-local split-k hand-off's workgroup mapping and of its per-launch guard.

The mapping functions are the kernels' own (exl3_kernels.h gemv_block_coords, moe_chunk_coords,
gemv1b_block, gemv1b_pair_span), called on the host through exl3_amd_debug_handoff_map.  For every
grid the planner can produce, the workgroups that count at one hand-off counter must have the
same linear workgroup id modulo the XCD count (round-robin dispatch then puts them on one XCD),
the arrivals per counter must equal the total its last-arrival test uses, and every (counter,
split) must be covered exactly once.

The guard (exl3_xcd.cuh): the counter is 64-bit and every arrival also adds its XCC id + 1 and
its square; the last arrival raises the alarm unless n * S2 == S1^2 (all ids equal).  Replayed
here over the same groups under several dispatch policies: round-robin from any starting XCD never
raises it; any policy that splits a group over two XCDs raises it, whatever the arrival order.
"""
import numpy as np
import pytest

from ampstein_amd import _lib

pytestmark = pytest.mark.filterwarnings("ignore")


def gemv_groups(X, chunks, splits, bszm=1):
    """counter (j, chunk) -> linear ids of the workgroups that arrive at it (grid = splits*chunks x bszm)."""
    gx = splits * chunks
    groups = {}
    seen = set()
    for j in range(bszm):
        for b in range(gx):
            chunk, slot = _lib.handoff_map(0, X, splits, 0, 0, b)[:2]
            assert 0 <= chunk < chunks and 0 <= slot < splits
            assert (j, chunk, slot) not in seen
            seen.add((j, chunk, slot))
            groups.setdefault((j, chunk), []).append(j * gx + b)
    assert len(seen) == bszm * chunks * splits
    return groups


def moe_groups(X, chunks, rest):
    groups, seen = {}, set()
    for b in range(chunks * rest):
        chunk, r = _lib.handoff_map(1, X, chunks, 0, 0, b)[:2]
        assert 0 <= chunk < chunks and 0 <= r < rest
        assert (chunk, r) not in seen
        seen.add((chunk, r))
        groups.setdefault(chunk, []).append(b)
    return groups


def gemv1b_groups(X, pairs, KS, R):
    """pair -> linear ids of the workgroups that arrive at its counter (only pairs whose span has
    two or more workgroups use a counter)."""
    per_x = pairs // X
    G = X * ((per_x * KS + 4 * R - 1) // (4 * R)) + X     # one extra row of workgroups: all past the end
    cover = {}
    for b in range(G):
        v, pa, pb, straddle = _lib.handoff_map(2, X, pairs, KS, R, b)
        x, lb = b % X, b // X
        T0 = lb * 4 * R
        if not v:
            assert T0 >= per_x * KS
            continue
        # slices of residue x's list this workgroup streams, and the pairs they belong to
        sl = range(T0, min(T0 + 4 * R, per_x * KS))
        touched = sorted({x + X * (t // KS) for t in sl})
        assert touched[0] == pa and touched[-1] == pb and len(touched) <= 2
        assert bool(straddle) == (len(touched) == 2)
        assert pa % X == x and pb % X == x
        for p in touched:
            cover.setdefault(p, []).append(b)
    assert sorted(cover) == list(range(pairs))
    groups = {}
    for p, bs in cover.items():
        q = p // X
        first, count = _lib.handoff_map(3, X, 0, KS, R, q)[:2]
        assert sorted(b // X for b in bs) == list(range(first, first + count)), (p, bs, first, count)
        if count > 1:
            groups[p] = bs
    return groups


GEMV_CASES = [(8, 8, 1), (8, 16, 2), (8, 56, 8), (8, 224, 3), (8, 112, 13), (4, 12, 5), (8, 8, 64)]


@pytest.mark.parametrize("X,chunks,splits", GEMV_CASES)
@pytest.mark.parametrize("bszm", [1, 3])
def test_gemv_groups_share_residue(X, chunks, splits, bszm):
    for (j, chunk), lins in gemv_groups(X, chunks, splits, bszm).items():
        assert len(lins) == splits
        assert {lin % X for lin in lins} == {chunk % X}


def test_gemv_mapping_without_xcd_is_a_bijection():
    gemv_groups(0, 24, 5)


@pytest.mark.parametrize("X,chunks,rest", [(8, 8, 1), (8, 16, 6), (8, 112, 4), (4, 8, 9)])
def test_moe_groups_share_residue(X, chunks, rest):
    for chunk, bs in moe_groups(X, chunks, rest).items():
        assert len(bs) == rest
        assert {b % X for b in bs} == {chunk % X}


# plans plan_balanced can produce: each residue's list of pairs // X * KS slices is a whole number
# of workgroups' 4 R slices, and 4 R <= KS
@pytest.mark.parametrize("X,pairs,KS,R", [(8, 56, 256, 8), (8, 224, 448, 7), (8, 16, 112, 7), (8, 8, 256, 16),
                                          (8, 8, 64, 16), (4, 12, 96, 4), (8, 112, 512, 14)])
def test_gemv1b_groups_share_residue(X, pairs, KS, R):
    for p, bs in gemv1b_groups(X, pairs, KS, R).items():
        assert {b % X for b in bs} == {p % X}


def guard_alarms(groups, xcc_of, rng):
    """Replay the guard: each group's arrivals in a random order add 1 + (v << 16) + (v^2 << 32)
    (v = XCC + 1) to a 64-bit counter; the arrival that makes the count whole raises the alarm
    when n * S2 != S1^2.  Returns whether the alarm was raised."""
    alarm = False
    for lins in groups.values():
        ctr = 0
        for i in rng.permutation(len(lins)):
            v = xcc_of(lins[i]) + 1
            ctr += 1 | (v << 16) | ((v * v) << 32)
            assert ctr < 1 << 64
            n, s1, s2 = ctr & 0xFFFF, (ctr >> 16) & 0xFFFF, ctr >> 32
            if n == len(lins) and n * s2 != s1 * s1:
                alarm = True
    return alarm


def test_counter_fields_hold_the_largest_group():
    """3000 arrivals (the library's cap) of the largest id the check can see (XCC 15, + 1 by the
    test hook): no field overflows into the next."""
    n, v = 3000, 17
    assert n < 1 << 16 and n * v < 1 << 16 and n * v * v < 1 << 32


def mixed(groups, xcc_of):
    return any(len({xcc_of(b) for b in lins}) > 1 for lins in groups.values())


@pytest.mark.parametrize("kind", ["gemv", "moe", "gemv1b"])
def test_guard_flags_exactly_the_mixed_launches(kind):
    X = 8
    rng = np.random.default_rng(7)
    if kind == "gemv":
        groups = gemv_groups(X, 56, 8, bszm=2)
    elif kind == "moe":
        groups = moe_groups(X, 16, 6)
    else:
        groups = gemv1b_groups(X, 56, 256, 8)
    G = 1 + max(max(v) for v in groups.values())
    policies = {f"round-robin from {b0}": (lambda b, b0=b0: (b0 + b) % X) for b0 in range(X)}
    policies["blocked"] = lambda b: min(b * X // G, X - 1)
    policies["round-robin of pairs"] = lambda b: (b // 2) % X
    policies["round-robin over 7"] = lambda b: b % 7
    table = rng.integers(0, X, G)
    policies["random"] = lambda b: int(table[b])
    for name, f in policies.items():
        for trial in range(3):
            assert guard_alarms(groups, f, rng) == mixed(groups, f), name
        if name.startswith("round-robin from"):
            assert not mixed(groups, f)
        elif name in ("blocked", "random"):
            assert mixed(groups, f), name


def test_fake_block_hook_lands_in_a_shared_group():
    """The GPU test's hook (policy EXL3_AMD_POLICY_XCD_FAKE = X + 1: workgroup X reports
    XCC id + 1) hits a counter that workgroup 0 also arrives at, for the split GEMV grid it uses."""
    X = 8
    groups = gemv_groups(X, 32, 4)
    assert any(0 in lins and X in lins for lins in groups.values())
    f = lambda b: (b + (1 if b == X else 0)) % X
    assert guard_alarms(groups, f, np.random.default_rng(0))


def test_handoff_map_rejects():
    with pytest.raises(_lib.Exl3Error):
        _lib.handoff_map(9, 8, 1, 1, 1, 0)
    with pytest.raises(_lib.Exl3Error):
        _lib.handoff_map(1, 8, 12, 0, 0, 0)         # chunks not a multiple of the XCD count
    with pytest.raises(_lib.Exl3Error):
        _lib.handoff_map(0, 8, 0, 0, 0, 0)
    with pytest.raises(_lib.Exl3Error):
        _lib.handoff_map(2, 8, 16, 112, 5, 0)       # 224 slices per residue: not whole workgroups of 20
