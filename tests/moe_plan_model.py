"""Host model of the token-sorted MoE's index structures (exl3_amd_moe, ampstein_amd/csrc/
exl3_moe_sorted.hip and the moeg_kernel walk in exl3_gemm.hip), with a shadow-memory check of
every workspace and pool-buffer read.

What the kernels compute per call and per pass of `pool` rows (exl3_moe.cu:137-418 semantics):
  tokens    tok_start[T + 1], tok_pos[total]: each token's sorted positions, ascending;
  plan      rowinfo[3 * pool] = (sorted position or -1, expert, row within the expert),
            rt[3 * tiles] = (expert, first pool row, rows), lists[3 * RATES][rt_cap] of tile ids
            per (matrix, rate slot), counts[3 * RATES], inv_row[position] = pool row;
then gather (pool rows -> ts_g / ts_u, chunk sums ps_g / ps_u), the grouped GEMMs over the tile
lists, the activation (ti_* -> ti_g, ps_d), the down GEMM (-> ts_g) and the token-major output.

`simulate` replays those index walks in the kernels' own order over shadow buffers that record,
per element, the pass that last wrote it (-1: never in this call), and asserts that every read
of workspace state or pool rows hits an element written earlier in the same pass -- except the
reads that the kernels guard (inv_row of a position outside the pass, which the output kernel
validates through rowinfo), for which it asserts that the guard rejects every stale value.
"""
from __future__ import annotations

import numpy as np

MOES_RATES = 11
PLAN_EMAX = 4096
WS_BYTES = 64 << 20


def rate_slot(K: int) -> int:
    """moes_rate_slot (exl3_kernels.h): rate code -> list slot, -1 when no instance exists."""
    if 1 <= K <= 8:
        return K - 1
    if 17 <= K <= 19:
        return K - 9
    return -1


def rate_code(K: float) -> int:
    k2 = int(2 * K)
    return 16 + k2 // 2 if k2 % 2 else k2 // 2


def tile_rows_for(num_assign: int, E: int, reg_gemm: bool = True, forced: int = 0) -> int:
    """The tile height rule of exl3_amd_moe (exl3_capi.cpp)."""
    mean = num_assign // max(E, 1)
    want = mean * 3 // 2
    if reg_gemm:
        tr = 32 if want <= 32 else (64 if want <= 64 else (96 if want <= 96 else 128))
        if forced in (32, 64, 96, 128):
            tr = forced
    else:
        tr = 64 if mean <= 40 else (128 if mean <= 96 else 256)
        if forced in (64, 128, 256):
            tr = forced
    return tr


class Layout:
    """Workspace regions of exl3_amd_moe in int32 units (offsets from the workspace base)."""

    def __init__(self, E, bsz, num_assign, H, I, pool, tile_rows, tok_mode):
        self.pool, self.tile_rows = pool, tile_rows
        self.rt_cap = pool // tile_rows + min(E, pool) + 1
        self.rowinfo = 0
        self.rt = 3 * pool
        self.lists = self.rt + 3 * self.rt_cap
        self.counts = self.lists + 3 * MOES_RATES * self.rt_cap
        self.ps_g = self.counts + 3 * MOES_RATES
        self.ps_u = self.ps_g + pool * (H // 128)
        self.ps_d = self.ps_u + pool * (H // 128)
        end = self.ps_d + pool * (I // 128)
        self.tok_mode = tok_mode
        if tok_mode:
            self.tok_start = end
            self.tok_pos = self.tok_start + bsz + 1
            self.inv_row = self.tok_pos + num_assign
            end = self.inv_row + num_assign
        self.end = end
        assert end * 4 <= WS_BYTES, "the call must fit the library workspace"


def tokens(token_sorted: np.ndarray, T: int):
    """moes_tokens_kernel: per-token ascending lists of sorted positions."""
    lists = [[] for _ in range(T)]
    for p, tk in enumerate(token_sorted):
        if 0 <= tk < T:
            lists[int(tk)].append(p)
    start = np.zeros(T + 1, np.int64)
    pos = []
    for t in range(T):
        start[t] = len(pos)
        pos.extend(sorted(lists[t]))
    start[T] = len(pos)
    return start.astype(np.int32), np.array(pos, np.int32)


def plan(count, E, num_assign, max_tok, lo, hi, pool, tile_rows, w0, Kcodes):
    """moes_plan_kernel for the pass starting at eligible row w0.  Kcodes[m][e]: rate code of
    matrix m (gate, up, down) of expert e.  Returns (rowinfo, tiles, lists, inv_row dict)."""
    c = np.clip(np.asarray(count[:E], np.int64), 0, 0x3FFFFFFF)
    ok = (c > 0) & (c <= max_tok) & (c >= lo) & (c <= hi)
    cst = np.where(ok, c, 0)
    start = np.concatenate([[0], np.cumsum(c)[:-1]])
    cst_start = np.concatenate([[0], np.cumsum(cst)[:-1]])
    total = int(cst.sum())
    w1 = w0 + pool
    tiles, lists = [], [[[] for _ in range(MOES_RATES)] for _ in range(3)]
    for e in range(E):
        a, b = max(int(cst_start[e]), w0), min(int(cst_start[e] + cst[e]), w1)
        n = max(0, b - a)
        j = 0
        while j * tile_rows < n:
            tid = len(tiles)
            tiles.append((e, a - w0 + tile_rows * j, min(tile_rows, n - tile_rows * j)))
            for m in range(3):
                s = rate_slot(int(Kcodes[m][e]))
                if s >= 0:
                    lists[m][s].append(tid)
            j += 1
    rowinfo = np.full((pool, 3), -1, np.int64)
    inv = {}
    for r in range(pool):
        cc = w0 + r
        info, e, jj = -1, 0, 0
        if cc < total:
            e = int(np.searchsorted(cst_start, cc, side="right") - 1)   # last e with start <= cc
            jj = cc - int(cst_start[e])
            info = int(start[e]) + jj
            if info >= num_assign:
                info = -1
        rowinfo[r] = (info, e, jj)
        if info >= 0:
            inv[info] = r
    return rowinfo, tiles, lists, inv, total


class Shadow:
    """Per-element pass stamps of one buffer: -1 = not written in this call."""

    def __init__(self, shape, name):
        self.w = np.full(shape, -1, np.int64)
        self.name = name

    def write(self, idx, p):
        self.w[idx] = p

    def read(self, idx, p, what):
        v = self.w[idx]
        assert np.all(v == p), f"{what}: read of {self.name}{idx} not written in pass {p} (stamps {np.unique(v)})"


def simulate(count, token_sorted, T, E, H, I, max_tok, conc, lo, hi, Kcodes, gated=True, tile_rows=None,
             tok_mode=True):
    """Replay one exl3_amd_moe call's index walks; assert that every read hits memory written in
    the same pass (or is rejected by its guard).  Returns per-token contributions per pass."""
    num_assign = len(token_sorted)
    pool = min(conc * max_tok, num_assign)
    tr = tile_rows or tile_rows_for(num_assign, E)
    lay = Layout(E, T, num_assign, H, I, pool, tr, tok_mode)
    hc, ic = H // 128, I // 128
    rowinfo = Shadow((pool, 3), "rowinfo")
    rt_sh = Shadow((lay.rt_cap, 3), "rt")
    lists_sh = Shadow((3, MOES_RATES, lay.rt_cap), "lists")
    counts_sh = Shadow((3, MOES_RATES), "counts")
    ps = {m: Shadow((pool, hc if m != "d" else ic), "ps_" + m) for m in "gud"}
    ts_g, ts_u = Shadow((pool, hc), "ts_g"), Shadow((pool, hc), "ts_u")       # per 128-chunk
    ti_g, ti_u = Shadow((pool, ic), "ti_g"), Shadow((pool, ic), "ti_u")
    inv_sh = Shadow(num_assign, "inv_row")
    contributions = np.zeros(num_assign, np.int64)
    start, pos_list = tokens(token_sorted, T)
    for p, w0 in enumerate(range(0, num_assign, pool)):
        info, tiles, lists, inv, total = plan(count, E, num_assign, max_tok, lo, hi, pool, tr, w0, Kcodes)
        assert len(tiles) <= lay.rt_cap, "row tiles exceed rt_cap"
        rowinfo.write(slice(None), p)
        for t in range(len(tiles)):
            rt_sh.write(t, p)
        for m in range(3):
            for s in range(MOES_RATES):
                assert len(lists[m][s]) <= lay.rt_cap
                for i in range(len(lists[m][s])):
                    lists_sh.write((m, s, i), p)
        counts_sh.write(slice(None), p)
        for pos, r in inv.items():
            inv_sh.write(pos, p)
        # tiles partition exactly the rows that carry a position
        cover = np.zeros(pool, np.int64)
        for e, r0, M in tiles:
            assert 0 < M <= tr and 0 <= r0 and r0 + M <= pool
            cover[r0:r0 + M] += 1
            assert np.all(info[r0:r0 + M, 1] == e), "a tile's rows belong to its expert"
        assert np.array_equal(cover, (info[:, 0] >= 0).astype(np.int64)), "tiles cover each live row once"
        # gather: every pool row reads its rowinfo; live rows stage gate / up rows and chunk sums
        for r in range(pool):
            rowinfo.read((r, 0), p, "gather")
            if info[r, 0] < 0:
                continue
            rowinfo.read((r, 1), p, "gather")
            assert 0 <= info[r, 0] < num_assign
            if gated:
                ts_g.write(r, p)
                ps["g"].write(r, p)
            ts_u.write(r, p)
            ps["u"].write(r, p)

        def gemm(phase):
            mats = ([0] if gated else []) + [1] if phase == 0 else [2]
            for s in range(MOES_RATES):
                for mi, m in enumerate(mats):
                    counts_sh.read((m, s), p, "moeg count")
                    for li in range(len(lists[m][s])):
                        lists_sh.read((m, s, li), p, "moeg list")
                        tid = lists[m][s][li]
                        rt_sh.read(tid, p, "moeg tile")
                        e, r0, M = tiles[tid]
                        rows = slice(r0, r0 + M)             # X rows clamp to M - 1: inside the tile
                        src = {0: (ts_g, ps["g"]), 1: (ts_u, ps["u"]), 2: (ti_g, ps["d"])}[m]
                        src[0].read(rows, p, f"moeg A rows (matrix {m})")
                        src[1].read(rows, p, f"moeg mul1 row sums (matrix {m})")
                        dst = {0: ti_g, 1: ti_u, 2: ts_g}[m]
                        dst.write(rows, p)

        gemm(0)
        # activation: live rows read up (and gate) outputs, write the down input in place
        for r in range(pool):
            rowinfo.read((r, 0), p, "act")
            if info[r, 0] < 0:
                continue
            ti_u.read(r, p, "act up")
            if gated:
                ti_g.read(r, p, "act gate")
            ti_g.write(r, p)
            ps["d"].write(r, p)
        gemm(1)
        # token-major output: each token's positions; rows of this pass through inv_row
        if tok_mode:
            for tok in range(T):
                for pi in range(int(start[tok]), int(start[tok + 1])):
                    pos = int(pos_list[pi])
                    if inv_sh.w[pos] == p:
                        r = inv[pos]
                    else:
                        # stale (earlier call or pass): any r; the guard must reject every one
                        for r_any in range(pool):
                            assert info[r_any, 0] != pos, "a stale inv_row entry passes the rowinfo guard"
                        continue
                    assert 0 <= r < pool and info[r, 0] == pos
                    rowinfo.read((r, 0), p, "out")
                    rowinfo.read((r, 1), p, "out")
                    ts_g.read(r, p, "out down row")
                    contributions[pos] += 1
        else:
            for r in range(pool):
                rowinfo.read((r, 0), p, "out")
                if info[r, 0] >= 0:
                    ts_g.read(r, p, "out down row")
                    contributions[int(info[r, 0])] += 1
    return contributions, lay
