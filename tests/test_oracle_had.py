"""Pins the oracle's reconstruct_had rounding sequence (oracle/exl3_oracle.c, had_block_h16,
restating vendor/exl3/exllamav3_ext/quant/reconstruct.cu:290-357) with inputs whose results have
closed forms.

The transform is fed through exl3o_had_transform, the same per-block code that
exl3o_reconstruct_had runs after its trellis decode (the decode is pinned in test_oracle.py).

- Family A: W_hat a sum of up to three signed Walsh outer products with power-of-two weights.
  Every intermediate of the reference's sequence is exactly representable, and fp16 rs = 181/2048
  squared rounds to exactly 1/128 at the second multiply.  So any correct implementation must
  return diag(suh) H W_hat H diag(svh) / 128 bit for bit.  This pins indices, signs, the
  orientation of suh (rows) and svh (columns), and the 4-point + lane stage structure.
- Families B-E: a few arbitrary fp16 entries placed so that exactly one step of the sequence
  rounds.  The expected value is written from the reference's expressions at that step with
  numpy's binary16 conversion (correct rounding from float64, where every sum of two fp16 values
  is exact):
    B: the column 4-point stage in fp16: s0 = a0+a1, d0 = a0-a1, s1, d1, then (s0+s1)*rs ...
    C: the order of the column lane stages (partner lane xor 1, 2, 4, 8, 16);
    D: the row 4-point stage in fp32, rounded to fp16 once, then * rs in fp16;
    E: the order of the row lane stages.
  A dropped rounding, an fp32 column stage, fp16 row sums, reversed stage order or a transposed
  operand each fail one of them.
- Family F: on random trellis data the gain <W, ref> / <ref, ref> is 128 rs^2 = 32761/32768
  (rs rounded to fp16 in both passes), and the error obeys the first-order bound of the
  sequence's 15 roundings.
"""
import numpy as np
import pytest
import scipy.linalg

H = scipy.linalg.hadamard(128).astype(np.float64)
H4 = scipy.linalg.hadamard(4).astype(np.float64)
H32 = scipy.linalg.hadamard(32).astype(np.float64)
RS = float(np.float16(0.08838834764831845))          # __float2half2_rn(r_scale) = 181/2048
U = 2.0 ** -11                                       # fp16 unit roundoff


def h(x):
    """Round float64 to binary16 (RNE) and back."""
    return float(np.float64(x).astype(np.float16))


def signs(rng, n, mags=(0.5, 1.0, 2.0)):
    return (rng.choice([-1.0, 1.0], n) * rng.choice(mags, n)).astype(np.float16)


def rand_h(rng, lo=-4, hi=4):
    """fp16 values with random signs, 11-bit significands and exponents in [lo, hi]."""
    while True:
        v = h(rng.choice([-1.0, 1.0]) * rng.uniform(1.0, 2.0) * 2.0 ** int(rng.integers(lo, hi + 1)))
        if v != 0.0:
            return v


def run(orc, W_hat, suh, svh):
    return orc.had_transform(W_hat.astype(np.float16), suh, svh).astype(np.float64)


def test_constants():
    assert RS == 181 / 2048
    assert h(h(h(4.0 * RS) * 32 * 4 * RS)) == 4.0          # (128 RS)(4 RS) rounds to exactly 4
    assert np.array_equal(H, np.kron(H32, H4))               # H[a, b] = H32[a/4, b/4] H4[a%4, b%4]


# ---------------------------------------------------------------- family A: exact

@pytest.mark.parametrize("seed", range(6))
def test_walsh_sums_exact(orc, seed):
    rng = np.random.default_rng(100 + seed)
    kb, nb = 2, 3
    W_hat = np.zeros((128 * kb, 128 * nb))
    for bk in range(kb):
        for bn in range(nb):
            e = int(rng.integers(-6, 2))
            blk = np.zeros((128, 128))
            for _ in range(int(rng.integers(1, 4))):
                i, j = rng.integers(0, 128, 2)
                blk += rng.choice([-1.0, 1.0]) * 2.0 ** e * np.outer(H[:, i], H[j, :])
            W_hat[bk * 128:(bk + 1) * 128, bn * 128:(bn + 1) * 128] = blk
    assert np.array_equal(W_hat.astype(np.float16).astype(np.float64), W_hat)
    suh, svh = signs(rng, 128 * kb), signs(rng, 128 * nb)
    Hb = lambda b: np.kron(np.eye(b), H)
    want = suh.astype(np.float64)[:, None] * (Hb(kb) @ W_hat @ Hb(nb) / 128.0) * svh.astype(np.float64)
    got = run(orc, W_hat, suh, svh)
    assert np.array_equal(got, want)
    assert np.count_nonzero(want) <= 3 * kb * nb


# ---------------------------------------------------------------- families B-E: one rounding step

def place(rng):
    return rng.choice([-1.0, 1.0], 128).astype(np.float16), rng.choice([-1.0, 1.0], 128).astype(np.float16)


@pytest.mark.parametrize("seed", range(20))
def test_column_four_point_stage(orc, seed):
    """Rows 4g..4g+3 of column j hold a0..a3 (all else 0): only the fp16 4-point stage and its
    * rs round; every later step is exact or a single rounding with a closed form."""
    rng = np.random.default_rng(200 + seed)
    g, j = int(rng.integers(0, 32)), int(rng.integers(0, 128))
    a = [rand_h(rng) for _ in range(4)]
    W_hat = np.zeros((128, 128))
    W_hat[4 * g:4 * g + 4, j] = a
    suh, svh = place(rng)
    s0, d0, s1, d1 = h(a[0] + a[1]), h(a[0] - a[1]), h(a[2] + a[3]), h(a[2] - a[3])
    c = [h(h(s0 + s1) * RS), h(h(d0 + d1) * RS), h(h(s0 - s1) * RS), h(h(d0 - d1) * RS)]
    want = np.zeros((128, 128))
    for R in range(128):
        x = H32[g, R // 4] * c[R % 4]                     # lane stages: one group, exact
        y = h(x * RS)                                     # row pass: one entry per row
        want[R] = float(suh[R]) * y * H[j] * svh.astype(np.float64)
    got = run(orc, W_hat, suh, svh)
    assert np.array_equal(got, want)


def three_groups(rng):
    """Three lane groups G0, G0 ^ 2^p, G0 ^ 2^q (p < q): G0 and G1 meet at stage p, then G2 at q."""
    p, q = sorted(rng.choice(5, 2, replace=False))
    G0 = int(rng.integers(0, 32))
    return [G0, G0 ^ (1 << int(p)), G0 ^ (1 << int(q))]


@pytest.mark.parametrize("seed", range(20))
def test_column_lane_stage_order(orc, seed):
    rng = np.random.default_rng(300 + seed)
    G, r0, j = three_groups(rng), int(rng.integers(0, 4)), int(rng.integers(0, 128))
    a = [rand_h(rng) for _ in range(3)]
    W_hat = np.zeros((128, 128))
    for m in range(3):
        W_hat[4 * G[m] + r0, j] = a[m]
    suh, svh = place(rng)
    u = [h(a[m] * RS) for m in range(3)]
    want = np.zeros((128, 128))
    for R in range(128):
        t = R // 4
        col = H4[r0, R % 4] * h(h(H32[G[0], t] * u[0] + H32[G[1], t] * u[1]) + H32[G[2], t] * u[2])
        want[R] = float(suh[R]) * h(col * RS) * H[j] * svh.astype(np.float64)
    got = run(orc, W_hat, suh, svh)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(20))
def test_row_four_point_stage_fp32(orc, seed):
    """Row i, columns 4g..4g+3 hold b0..b3: the column pass is exact up to one * rs per entry; the
    row pass sums the four in fp32 (exact here), rounds once to fp16, then * rs in fp16."""
    rng = np.random.default_rng(400 + seed)
    g, i = int(rng.integers(0, 32)), int(rng.integers(0, 128))
    b = [rand_h(rng) for _ in range(4)]
    W_hat = np.zeros((128, 128))
    W_hat[i, 4 * g:4 * g + 4] = b
    suh, svh = place(rng)
    y = [h(b[c] * RS) for c in range(4)]
    z = [h(h(sum(H4[c, r] * y[c] for c in range(4))) * RS) for r in range(4)]
    want = np.zeros((128, 128))
    for R in range(128):
        for C in range(128):
            want[R, C] = float(suh[R]) * H[i, R] * H32[g, C // 4] * z[C % 4] * float(svh[C])
    got = run(orc, W_hat, suh, svh)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(20))
def test_row_lane_stage_order(orc, seed):
    rng = np.random.default_rng(500 + seed)
    G, c0, i = three_groups(rng), int(rng.integers(0, 4)), int(rng.integers(0, 128))
    b = [rand_h(rng) for _ in range(3)]
    W_hat = np.zeros((128, 128))
    for m in range(3):
        W_hat[i, 4 * G[m] + c0] = b[m]
    suh, svh = place(rng)
    y = [h(h(b[m] * RS) * RS) for m in range(3)]
    want = np.zeros((128, 128))
    for C in range(128):
        t = C // 4
        v = H4[c0, C % 4] * h(h(H32[G[0], t] * y[0] + H32[G[1], t] * y[1]) + H32[G[2], t] * y[2])
        want[:, C] = suh.astype(np.float64) * H[i, :] * v * float(svh[C])
    got = run(orc, W_hat, suh, svh)
    assert np.array_equal(got, want)


def test_families_discriminate():
    """The closed forms separate the plausible alternatives on inputs drawn like the tests': an
    fp16-summed row stage and the reversed lane order each change some expected value."""
    rng = np.random.default_rng(700)
    diff_row, diff_order = 0, 0
    for _ in range(20):
        y = [h(rand_h(rng) * RS) for _ in range(4)]
        s0, d0, s1, d1 = h(y[0] + y[1]), h(y[0] - y[1]), h(y[2] + y[3]), h(y[2] - y[3])
        for r, f16_sum in enumerate([s0 + s1, d0 + d1, s0 - s1, d0 - d1]):
            diff_row += h(sum(H4[c, r] * y[c] for c in range(4))) != h(f16_sum)
        G = three_groups(rng)
        u = [h(rand_h(rng) * RS) for _ in range(3)]
        for t in range(32):
            s = [H32[G[m], t] * u[m] for m in range(3)]
            diff_order += h(h(s[0] + s[1]) + s[2]) != h(h(s[0] + s[2]) + s[1])
    assert diff_row > 0 and diff_order > 0


# ---------------------------------------------------------------- family F: statistics

@pytest.mark.parametrize("cb", [0, 1, 2])
def test_gain_and_bound_random(orc, cb):
    rng = np.random.default_rng(600 + cb)
    trellis = rng.integers(0, 65536, (16, 16, 64), dtype=np.uint16)    # 256 x 256, K = 4
    suh = np.where(rng.integers(0, 2, 256) > 0, 1.0, -1.0).astype(np.float16)
    svh = np.where(rng.integers(0, 2, 256) > 0, 1.0, -1.0).astype(np.float16)
    W_hat = orc.reconstruct(trellis, 4, cb=cb)
    W = orc.reconstruct_had(trellis, suh, svh, 4, cb=cb).astype(np.float64)
    # composition: reconstruct_had is the transform of the decoded W_hat
    assert np.array_equal(W, orc.had_transform(W_hat, suh, svh).astype(np.float64))
    Hb = np.kron(np.eye(2), H)
    ref = suh.astype(np.float64)[:, None] * (Hb @ W_hat.astype(np.float64) @ Hb / 128.0) * svh.astype(np.float64)
    gain = float(np.sum(W * ref) / np.sum(ref * ref))
    # fp16 rs in both passes: 128 rs^2 = 32761/32768 (1 - 2.1e-4); an fp32 rs in either pass
    # moves the gain by 1.1e-4, rounding noise moves it by ~1e-5
    assert abs(gain - 32761 / 32768) < 3e-5, gain
    # first order: 15 fp16 roundings on the path of each element (column: 2 adds, * rs, 5 lane
    # stages; row: round, * rs, 5 lane stages), each orthogonal-stage error <= u of the stage's
    # norm, plus the systematic rs offset
    frob = np.linalg.norm(W - ref) / np.linalg.norm(ref)
    assert frob <= 15 * U + (1 - 32761 / 32768), frob
    assert frob > 0.1 * U                                # the sequence does round
