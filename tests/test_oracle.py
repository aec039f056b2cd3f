"""Pins the CPU oracle (oracle/exl3_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible restatement mistake fails it:
reference-produced vectors (tests/golden, from the reference's own
cpu/moe_mul1.cpp), known answers, independent implementations of the
binary16 rounding (numpy) and of the bit windows (a bit string), and the
mathematics of the Hadamard transform.
"""
import ctypes
from fractions import Fraction

import numpy as np
import pytest
import scipy.linalg

H128 = scipy.linalg.hadamard(128).astype(np.float64)  # Sylvester, natural order


def f16(bits):
    return np.array(bits, dtype=np.uint16).view(np.float16)


# ---------------------------------------------------------------- binary16 arithmetic

def test_half_add_mul_match_numpy(orc):
    rng = np.random.default_rng(1)
    a = rng.integers(0, 0x7c00, 20000, dtype=np.uint16) | (rng.integers(0, 2, 20000, dtype=np.uint16) << 15)
    b = rng.integers(0, 0x7c00, 20000, dtype=np.uint16) | (rng.integers(0, 2, 20000, dtype=np.uint16) << 15)
    fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
    # sums and products of two halves are exact in float64: numpy's cast is one RNE rounding
    add_ref = (fa + fb).astype(np.float16).view(np.uint16)
    mul_ref = (fa * fb).astype(np.float16).view(np.uint16)
    L = orc.lib()
    add = np.array([L.exl3o_hadd(int(x), int(y)) for x, y in zip(a, b)], np.uint16)
    mul = np.array([L.exl3o_hmul(int(x), int(y)) for x, y in zip(a, b)], np.uint16)
    # +0 / -0 of exact zero sums: compare as values
    assert np.array_equal(add.view(np.float16).astype(np.float64), add_ref.view(np.float16).astype(np.float64))
    nz = mul_ref.view(np.float16) != 0
    assert np.array_equal(mul[nz], mul_ref[nz])


def test_half_from_float_matches_numpy(orc):
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([65504.0, 65519.99, 65520.0, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001, 3 * 2 ** -26], np.float32),
    ]).astype(np.float32)
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([orc.lib().exl3o_h_from_f32(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


def test_half_fma_single_rounding(orc):
    L = orc.lib()
    rng = np.random.default_rng(3)
    checked = 0
    for _ in range(4000):
        a, b, c = (int(v) for v in rng.integers(0, 0x7bff, 3))
        a |= int(rng.integers(0, 2)) << 15
        c |= int(rng.integers(0, 2)) << 15
        fa, fb, fc = (Fraction(float(f16(v))) for v in (a, b, c))
        exact = fa * fb + fc
        as_double = float(exact)
        if Fraction(as_double) != exact or exact == 0:
            continue  # numpy's cast would be a second rounding: skip
        assert L.exl3o_hfma(a, b, c) == int(np.float16(as_double).view(np.uint16))
        checked += 1
    assert checked > 3000


# ---------------------------------------------------------------- codebooks

KNOWN = {  # values computed from quant/codebook.cuh by exact arithmetic
    (0, 0): 0x3A25, (0, 1): 0xBB5B, (0, 0xFFFF): 0xB110, (0, 0x1234): 0xC066,
    (1, 0): 0x3F60, (1, 1): 0x304E,
    (2, 0): 0xC2E8, (2, 1): 0x3921,
}


@pytest.mark.parametrize("cb_state", sorted(KNOWN))
def test_codebook_known_answers(orc, cb_state):
    cb, s = cb_state
    assert orc.decode(s, cb) == KNOWN[cb_state]


@pytest.mark.parametrize("cb,std", [(0, 1.2437), (1, 1.2441), (2, 1.0003)])
def test_codebook_distribution(orc, cb, std):
    v = orc.decode_all(cb).view(np.float16).astype(np.float64)
    assert abs(v.std() - std) < 1e-3
    assert abs(v.mean()) < 0.01
    if cb == 0:
        assert abs(v.min() + 3.957) < 2e-3 and abs(v.max() - 3.973) < 2e-3


def test_codebook_3inst_mcg_independent(orc):
    s = np.arange(65536, dtype=np.uint64)
    for cb, (mul, add) in {0: (89226354, 64248484), 1: (0xCBAC1FED, 0)}.items():
        x = (s * mul + add) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = (x & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
        hi = (x >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
        ref = (lo + hi).astype(np.float16).view(np.uint16)
        assert np.array_equal(orc.decode_all(cb), ref)


def test_codebook_mul1_vs_reference_cpu(orc, golden):
    # moe_mul1.cpp computes (bytesum - 510) * k_inv in fp32; the GPU value is one fp16 fma.
    ours = orc.decode_all(2).view(np.float16).astype(np.float64)
    ref = golden["mul1_f32"].astype(np.float64)
    # the two differ only by the fp16 rounding of the bias constant (half an ulp of 10.4)
    # and of the result: a wrong multiplier or byte sum would be off by O(1)
    assert np.all(np.abs(ours - ref) <= 2.0 ** -8 + np.abs(ours) * 2.0 ** -11)
    # exact value of the fma: bytesum-affine, checked with rationals on every distinct sum
    k_inv, bias = Fraction(float(f16(0x1EEE))), Fraction(float(f16(0xC931)))
    for s in range(1024, 2045):
        exact = float(Fraction(s) * k_inv + bias)
        assert orc.lib().exl3o_hfma(int(np.float16(s).view(np.uint16)), 0x1EEE, 0xC931) == \
            int(np.float16(exact).view(np.uint16))


# ---------------------------------------------------------------- windows / tile layout

def bitstring_state(tile_u16, bits, half, t):
    """Independent statement: the tile is one MSB-first bit ring over its uint32 words
    (word i = u16[2i] | u16[2i+1] << 16); position t's state is the 16 bits that end
    after the first e(t) stream bits, e(t) = sum of the widths of positions 0..t."""
    words = [int(tile_u16[2 * i]) | (int(tile_u16[2 * i + 1]) << 16) for i in range(len(tile_u16) // 2)]
    stream = "".join(format(w, "032b") for w in words)
    if half:
        widths = [bits if p % 2 == 0 else bits + 1 for p in range(256)]
    else:
        widths = [bits] * 256
    e = sum(widths[: t + 1])
    ring = stream * 3
    start = e - 16 + len(stream)
    return int(ring[start:start + 16], 2)


@pytest.mark.parametrize("bits,half", [(b, False) for b in range(1, 9)] + [(b, True) for b in (1, 2, 3)])
def test_state_vs_bitstring(orc, bits, half):
    rng = np.random.default_rng(100 + bits + 10 * half)
    tile = rng.integers(0, 65536, 16 * bits + (8 if half else 0), dtype=np.uint16)
    for t in range(256):
        assert orc.state(tile, bits, half, t) == bitstring_state(tile, bits, half, t), t


@pytest.mark.parametrize("bits", range(1, 9))
def test_state_vs_reference_cpu(orc, golden, bits):
    tiles, states = golden[f"state_tiles_K{bits}"], golden[f"state_K{bits}"]
    for i in range(tiles.shape[0]):
        got = [orc.state(tiles[i], bits, False, t) for t in range(256)]
        assert np.array_equal(np.array(got, np.uint16), states[i])


def test_half25_window_ends_vs_reference_cpu(orc, golden):
    # the oracle's half-K windows must end where the reference's 2.5 bpw ring says
    ends = golden["window_end_half25"]
    rng = np.random.default_rng(7)
    tile = rng.integers(0, 65536, 40, dtype=np.uint16)
    words = [int(tile[2 * i]) | (int(tile[2 * i + 1]) << 16) for i in range(20)]
    ring = "".join(format(w, "032b") for w in words) * 3
    for t in range(256):
        e = int(ends[t])
        assert orc.state(tile, 2, True, t) == int(ring[e - 16:e], 2)


def test_tile_perm_vs_reference_cpu(orc, golden):
    assert np.array_equal(orc.tile_perm(), golden["tc_perm"])
    assert sorted(orc.tile_perm().tolist()) == list(range(256))


def test_reconstruct_zero_trellis(orc):
    for cb in range(3):
        W = orc.reconstruct(np.zeros((2, 3, 64), np.uint16), 4, cb=cb)
        assert np.all(W.view(np.uint16) == orc.decode(0, cb))


@pytest.mark.parametrize("bits,half", [(2, False), (3, False), (4, False), (5, False), (2, True)])
def test_reconstruct_single_bit(orc, bits, half):
    """Flipping one stream bit changes exactly the weights whose windows cover it."""
    tu = 16 * bits + (8 if half else 0)
    rng = np.random.default_rng(11)
    trellis = rng.integers(0, 65536, (2, 2, tu), dtype=np.uint16)
    cb = 2 if half else 1
    base = orc.reconstruct(trellis, bits, half, cb)
    perm = orc.tile_perm()
    nbits = tu * 16
    widths = [bits if (not half or p % 2 == 0) else bits + 1 for p in range(256)]
    ends = np.cumsum(widths)
    for bit in rng.integers(0, nbits, 6):
        word, pos = divmod(int(bit), 32)          # MSB-first position inside the word
        u16i = 2 * word + (0 if pos >= 16 else 1)
        mask = 1 << ((31 - pos) & 15)
        t2 = trellis.copy()
        t2[1, 0, u16i] ^= mask
        W = orc.reconstruct(t2, bits, half, cb)
        diff = np.argwhere(W.view(np.uint16) != base.view(np.uint16))
        # positions whose 16-bit window [e-16, e) (mod ring) contains this bit
        cover = {p for p in range(256) if (int(bit) - (ends[p] - 16)) % nbits < 16}
        changed = {(r % 16) * 16 + c % 16 for r, c in diff}
        assert all(16 <= r < 32 and c < 16 for r, c in diff)
        assert changed <= {int(perm[p]) for p in cover}
        assert len(changed) >= len(cover) - 2   # a flip rarely maps to the same value


def test_reconstruct_slice_matches_full(orc):
    rng = np.random.default_rng(5)
    trellis = rng.integers(0, 65536, (4, 24, 48), dtype=np.uint16)
    full = orc.reconstruct(trellis, 3, cb=1)
    part = orc.reconstruct(trellis, 3, cb=1, n=128, n_offset=128)
    assert np.array_equal(full[:, 128:256].view(np.uint16), part.view(np.uint16))


# ---------------------------------------------------------------- Hadamard

def test_fwht_vs_reference_cpu_bit_exact(orc, golden):
    for i in range(golden["had_in"].shape[0]):
        assert np.array_equal(orc.fwht128_f32(golden["had_in"][i]).view(np.uint32),
                              golden["had_out"][i].view(np.uint32))


def test_had128_math(orc):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    y = orc.had128(x)
    ref = (x.reshape(3, 2, 128).astype(np.float64) @ H128 / np.sqrt(128)).reshape(3, 256)
    assert np.max(np.abs(y - ref)) < 1e-5
    z = orc.had128(y)                                     # H is an involution
    assert np.max(np.abs(z - x)) < 1e-5
    e = np.zeros((1, 128), np.float32)
    e[0, 5] = 1.0
    assert np.allclose(orc.had128(e)[0], H128[5] / np.sqrt(128), atol=1e-7)


def test_had128_half_scales(orc):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 384)).astype(np.float16)
    s = np.where(rng.integers(0, 2, 384) > 0, 1.0, -1.0).astype(np.float16)
    pre = orc.had128(x, pre=s)
    ref = ((x.astype(np.float64) * s).reshape(4, 3, 128) @ H128 / np.sqrt(128)).reshape(4, 384)
    assert np.max(np.abs(pre.astype(np.float64) - ref)) <= np.max(np.abs(ref)) * 2 ** -10
    post = orc.had128(x, post=s)
    ref2 = (x.astype(np.float64).reshape(4, 3, 128) @ H128 / np.sqrt(128)).reshape(4, 384) * s
    assert np.max(np.abs(post.astype(np.float64) - ref2)) <= np.max(np.abs(ref2)) * 2 ** -10
    # fp32 butterfly then one rounding: each output is the RNE half of the fp32 value
    f = orc.had128(x.astype(np.float32))
    assert np.array_equal(orc.had128(x).view(np.uint16), f.astype(np.float16).view(np.uint16))


def test_reconstruct_had_vs_f64(orc):
    rng = np.random.default_rng(12)
    trellis = rng.integers(0, 65536, (16, 16, 64), dtype=np.uint16)   # 256 x 256, K = 4
    suh = np.where(rng.integers(0, 2, 256) > 0, 1.0, -1.0).astype(np.float16)
    svh = np.where(rng.integers(0, 2, 256) > 0, 1.0, -1.0).astype(np.float16)
    W_hat = orc.reconstruct(trellis, 4).astype(np.float64)
    Hb = np.kron(np.eye(2), H128) / np.sqrt(128)
    ref = np.diag(suh.astype(np.float64)) @ Hb @ W_hat @ Hb @ np.diag(svh.astype(np.float64))
    W = orc.reconstruct_had(trellis, suh, svh, 4).astype(np.float64)
    err = np.abs(W - ref).max() / np.abs(ref).max()
    assert err < 4e-3, err
    assert np.abs(W - ref).mean() / np.abs(ref).mean() < 1e-3


# ---------------------------------------------------------------- reference linear

@pytest.mark.parametrize("y_fp32", [False, True])
def test_linear_vs_numpy_f64(orc, y_fp32):
    rng = np.random.default_rng(13)
    m, k, n, bits, cb = 3, 256, 384, 3, 1
    trellis = rng.integers(0, 65536, (k // 16, n // 16, 16 * bits), dtype=np.uint16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    suh = np.where(rng.integers(0, 2, k) > 0, 1.0, -1.0).astype(np.float16)
    svh = np.where(rng.integers(0, 2, n) > 0, 1.0, -1.0).astype(np.float16)
    W_hat = orc.reconstruct(trellis, bits, cb=cb).astype(np.float64)
    Hk = np.kron(np.eye(k // 128), H128) / np.sqrt(128)
    Hn = np.kron(np.eye(n // 128), H128) / np.sqrt(128)
    ref = ((x.astype(np.float64) * suh) @ Hk @ W_hat @ Hn) * svh.astype(np.float64)
    y = orc.linear(x, trellis, suh, svh, bits, cb=cb, y_fp32=y_fp32).astype(np.float64)
    y64 = orc.linear_f64(x, trellis, suh, svh, bits, cb=cb)
    scale = np.abs(ref).max()
    assert np.abs(y64 - ref).max() / scale < 2e-3        # A_had rounding only
    assert np.abs(y - ref).max() / scale < 2e-3
    # no rotations: plain product with the rotated-basis weights
    y0 = orc.linear(x, trellis, None, None, bits, cb=cb, y_fp32=True).astype(np.float64)
    assert np.abs(y0 - x.astype(np.float64) @ W_hat).max() < 1e-4 * np.abs(y0).max()
