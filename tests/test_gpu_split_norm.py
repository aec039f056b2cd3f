"""The decode step's residual norm split between its neighbours (rms_norm_res, amp_kernels.cu:279-365).

Producer half: h = fp16(h + c) and per-128-column sums of float(h)^2 (res_sq on its own,
exl3_gemm_res in the GEMV's chunk epilogue).  Consumer half: r = fp16(fp16(h * scale) * w),
scale = 1 / sqrt(sum / n + eps) (norm_sq on its own, exl3_mgemm with norm_in in the M = 1
stream GEMV's input load).

Bars: h bit-identical to fp16(h + c); the chunk sums within fp32 rounding of the fp64 sums; r
within one fp16 ulp of the fp64 statement (the fp32 sum of squares runs in another order); the
fused and standalone forms of each half bit-identical (C, h, sq and the mgemm outputs), on every
GEMV epilogue the planner can pick (direct store, XCD hand-off, matrix-core GEMV; the finish
kernel's in test_gpu_xcd_guard.py, which owns the hook that turns the hand-off off);
the captured decode step bit-identical across graph replays and within 5e-3 of the oracle model.
"""
import numpy as np
import pytest
import torch

from ampstein_amd import _lib, bundles, ops, synth
from tests.test_gpu_decode import _model, _stack, norm_model, ulp_diff

pytestmark = pytest.mark.gpu


def _h(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(t):
    return t.cpu().numpy().view(np.uint16 if t.dtype == torch.half else np.uint32)


@pytest.mark.parametrize("rows,n", [(1, 128), (1, 4096), (3, 5120), (2, 14336), (1, 32768)])
def test_res_sq_norm_sq_vs_model(rows, n):
    rng = np.random.default_rng(rows * 7 + n)
    h = (rng.standard_normal((rows, n)) * 3).astype(np.float16)
    c = (rng.standard_normal((rows, n)) * 2).astype(np.float16)
    w = (rng.standard_normal(n) * 0.5 + 1).astype(np.float16)
    hd, cd, wd = _h(h), _h(c), _h(w)
    sq = torch.empty((rows, n // 128), dtype=torch.float, device="cuda")
    ops.res_sq(hd, cd, sq)
    ye, ne = norm_model(h, c, w, 1e-5)
    assert np.array_equal(_bits(hd), ye.view(np.uint16))
    yy = ye.astype(np.float64).reshape(rows, n // 128, 128)
    ref_sq = (yy * yy).sum(-1)
    got_sq = sq.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got_sq - ref_sq) <= 1e-5 * ref_sq + 1e-30)
    r = ops.norm_sq(hd, sq, wd, 1e-5)
    assert ulp_diff(r.cpu().numpy(), ne).max() <= 1


def test_res_sq_without_residual_keeps_h():
    """c None: h keeps its bits exactly (negative zeros included); the sums are h's."""
    rng = np.random.default_rng(5)
    h = rng.standard_normal((2, 1024)).astype(np.float16)
    h[0, :7] = np.float16(-0.0)
    hd = _h(h)
    sq = torch.empty((2, 8), dtype=torch.float, device="cuda")
    ops.res_sq(hd, None, sq)
    assert np.array_equal(_bits(hd), h.view(np.uint16))
    hh = h.astype(np.float64).reshape(2, 8, 128)
    assert np.allclose(sq.cpu().numpy(), (hh * hh).sum(-1), rtol=1e-5)


def test_split_norm_rejects():
    h = torch.zeros((1, 200), dtype=torch.half, device="cuda")
    with pytest.raises(_lib.Exl3Error):
        _lib.check(_lib.lib().exl3_amd_res_sq(h.data_ptr(), None, h.data_ptr(), 1, 200, None))
    big = torch.zeros((1, 32768 + 128), dtype=torch.half, device="cuda")
    sq = torch.zeros(257, dtype=torch.float, device="cuda")
    with pytest.raises(_lib.Exl3Error):
        _lib.check(_lib.lib().exl3_amd_norm_sq(big.data_ptr(), sq.data_ptr(), big.data_ptr(), big.data_ptr(),
                                               1, 32768 + 128, 1e-5, None))


# GEMV epilogues, as (policy, value for k) settings: the default plan (XCD hand-off, or a direct
# store with one split), a forced single split, the matrix-core GEMV for single rows (block epilogue).
PLANS = {
    "default": [],
    "one-split": [(_lib.POLICY_GEMV_SLICES, lambda k: k // 16)],
    "mfma-rows": [(_lib.POLICY_GEMV_ROWS, lambda k: _lib.GEMV_ROWS_MFMA_ALL)],
}


def _gemm_res_case(k, n, swiglu, m, seed):
    L = synth.layer(k, n, 4, 0, seed=seed)
    L.svh = (L.svh.astype(np.float32) / 16).astype(np.float16)
    t, s, v = L.torch("cuda")
    rng = np.random.default_rng(seed + 1)
    a = _h(rng.standard_normal((m, k)).astype(np.float16))
    up = _h(rng.standard_normal((m, k)).astype(np.float16)) if swiglu else None
    h0 = _h((rng.standard_normal((m, n)) * 4).astype(np.float16))
    return t, s, v, a, up, h0


def _check_gemm_res(t, s, v, a, up, h0, m, n, reps=2):
    for rep in range(reps):               # a second call behaves the same (counters re-armed)
        C1 = torch.full((m, n), float("nan"), dtype=torch.half, device="cuda")
        h1 = h0.clone()
        sq1 = torch.full((m, n // 128), float("nan"), dtype=torch.float, device="cuda")
        ops.exl3_gemm_res(a, t, C1, s, v, h1, sq1, up=up)
        C2 = torch.empty_like(C1)
        if up is not None:
            ops.exl3_gemm_silu_mul(a, up, t, C2, s, v)
        else:
            ops.exl3_gemm(a, t, C2, s, torch.empty_like(a), v)
        h2 = h0.clone()
        sq2 = torch.empty_like(sq1)
        ops.res_sq(h2, C2, sq2)
        torch.cuda.synchronize()
        assert torch.equal(C1, C2), f"C differs (call {rep})"
        assert torch.equal(h1, h2), f"h differs (call {rep})"
        assert np.array_equal(_bits(sq1), _bits(sq2)), f"chunk sums differ (call {rep})"


@pytest.mark.parametrize("plan", list(PLANS))
@pytest.mark.parametrize("k,n", [(4096, 4096), (1024, 5120), (512, 640), (14336, 4096)])
@pytest.mark.parametrize("swiglu", [False, True])
def test_gemm_res_matches_two_calls(kernel_policy, plan, k, n, swiglu):
    for key, val in PLANS[plan]:
        kernel_policy(key, val(k))
    print(f"[split norm] gemm_res {plan} k={k} n={n} swiglu={swiglu}", flush=True)
    _check_gemm_res(*_gemm_res_case(k, n, swiglu, 1, k + n), 1, n)


@pytest.mark.parametrize("m", [3, 12])
def test_gemm_res_many_rows(m):
    """More rows: the linear, then res_sq (two launches); same results as the two calls."""
    _check_gemm_res(*_gemm_res_case(1024, 512, False, m, 31 + m), m, 512)


def _linears(k, widths, seed):
    out = []
    for i, n in enumerate(widths):
        L = synth.layer(k, n, 4, 0, seed=seed + i)
        t, s, v = L.torch("cuda")
        out.append(bundles.Linear(t, s, v, 4.0, False, False))
    return out


@pytest.mark.parametrize("plan", ["default", "mfma-rows"])
@pytest.mark.parametrize("k", [512, 4096, 14336])
@pytest.mark.parametrize("m", [1, 3])
def test_mgemm_norm_in_matches_two_calls(kernel_policy, plan, k, m):
    """Stacked (gate/up) and sliced (q/k/v) bundles with norm_in: bit-identical to norm_sq then
    the plain bundle on r."""
    for key, val in PLANS[plan]:
        kernel_policy(key, val(k))
    rng = np.random.default_rng(k + m)
    h = _h((rng.standard_normal((1, m, k)) * 3).astype(np.float16))
    w = _h((rng.standard_normal(k) * 0.3 + 1).astype(np.float16))
    sq = torch.empty((m, k // 128), dtype=torch.float, device="cuda")
    ops.res_sq(h.view(m, k), None, sq)
    r_ref = ops.norm_sq(h.view(m, k), sq, w, 1e-5)
    print(f"[split norm] mgemm_norm_in {plan} k={k} m={m}", flush=True)
    # stacked
    lin = _linears(k, [1024, 1024], 500 + k)
    out1 = torch.zeros((2, m, 1024), dtype=torch.half, device="cuda")
    out2 = torch.zeros_like(out1)
    b1, b2 = bundles.Multi(lin, out1), bundles.Multi(lin, out2)
    r = torch.empty((m, k), dtype=torch.half, device="cuda")
    for rep in range(2):
        b1.run(h, norm_in=(sq, w, 1e-5, r))
        b2.run(r_ref.view(1, m, k))
        torch.cuda.synchronize()
        assert torch.equal(out1, out2), f"stacked differs (call {rep})"
    # sliced
    lin = _linears(k, [1024, 256, 256], 600 + k)
    o1 = [torch.zeros((1, m, n), dtype=torch.half, device="cuda") for n in (1024, 256, 256)]
    o2 = [torch.zeros_like(o) for o in o1]
    s1, s2 = bundles.Sliced(lin, o1), bundles.Sliced(lin, o2)
    s1.run(h, norm_in=(sq, w, 1e-5, r))
    s2.run(r_ref.view(1, m, k))
    torch.cuda.synchronize()
    for a, b in zip(o1, o2):
        assert torch.equal(a, b), "sliced differs"


def test_decode_stack_split_norm(orc):
    H, Q, KV, I = 512, 512, 128, 1024
    st, host, wf = _stack(H, Q, KV, I, 2)
    st.split_norm = True
    st_u, _, _ = _stack(H, Q, KV, I, 2, fuse=False)
    st_u.split_norm = True
    ref_stack, _, _ = _stack(H, Q, KV, I, 2)
    rng = np.random.default_rng(17)
    xs = [rng.standard_normal(H).astype(np.float16) for _ in range(2)]
    eager = [st(_h(x)).clone() for x in xs]
    separate = [ref_stack(_h(x)).clone() for x in xs]
    for x, e in zip(xs, eager):
        assert torch.equal(st_u(_h(x)), e), "split norm: fused and unfused SwiGLU differ"
    st.capture()
    for rep in range(2):
        for x, e in zip(xs, eager):
            y = st(_h(x))
            torch.cuda.synchronize()
            assert torch.equal(y, e), f"graph replay {rep} differs from the eager step"
            _ = torch.randn(1000, device="cuda").sum()        # eager work between replays
    for x, e, sep in zip(xs, eager, separate):
        ref = _model(host, wf, x, 4, 0).astype(np.float64)
        got = e.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        d = np.abs(got - sep.cpu().numpy().astype(np.float64)).max() / np.abs(ref).max()
        print(f"decode stack (split norm) rel err {err:.2e}, vs separate norms {d:.2e}", flush=True)
        assert err < 5e-3


@pytest.mark.parametrize("K,cb", [(2, 1), (3, 0), (2.5, 2), (5, 2), (8, 0)])
def test_split_norm_codebooks(K, cb):
    """Both halves on other bitrates and codebooks (the norm input form and the residual
    epilogue are instances of every rate): producer bit-identical to exl3_gemm + res_sq,
    consumer bit-identical to norm_sq + the plain bundle."""
    k, n = 4096, 1024
    L = synth.layer(k, n, K, cb, seed=int(10 * K) + cb)
    L.svh = (L.svh.astype(np.float32) / 16).astype(np.float16)
    t, s, v = L.torch("cuda")
    mcg, mul1 = cb == 1, cb == 2
    rng = np.random.default_rng(int(10 * K) + 7 * cb)
    a = _h(rng.standard_normal((1, k)).astype(np.float16))
    h0 = _h((rng.standard_normal((1, n)) * 4).astype(np.float16))
    # producer
    C1, h1 = torch.empty((1, n), dtype=torch.half, device="cuda"), h0.clone()
    sq1 = torch.empty((1, n // 128), dtype=torch.float, device="cuda")
    ops.exl3_gemm_res(a, t, C1, s, v, h1, sq1, mcg, mul1)
    C2, h2 = torch.empty_like(C1), h0.clone()
    sq2 = torch.empty_like(sq1)
    ops.exl3_gemm(a, t, C2, s, torch.empty_like(a), v, 0, mcg, mul1)
    ops.res_sq(h2, C2, sq2)
    torch.cuda.synchronize()
    assert torch.equal(C1, C2) and torch.equal(h1, h2)
    assert np.array_equal(_bits(sq1), _bits(sq2))
    # consumer: a stacked pair of this rate's matrices reading the residual row h (k wide)
    lin = []
    for i in range(2):
        Li = synth.layer(k, 512, K, cb, seed=900 + int(10 * K) + i)
        ti, si, vi = Li.torch("cuda")
        lin.append(bundles.Linear(ti, si, vi, float(K), mcg, mul1))
    hk = _h((rng.standard_normal((1, 1, k)) * 3).astype(np.float16))
    w = _h((rng.standard_normal(k) * 0.3 + 1).astype(np.float16))
    sqk = torch.empty((1, k // 128), dtype=torch.float, device="cuda")
    ops.res_sq(hk.view(1, k), None, sqk)
    r_ref = ops.norm_sq(hk.view(1, k), sqk, w, 1e-5)
    o1 = torch.zeros((2, 1, 512), dtype=torch.half, device="cuda")
    o2 = torch.zeros_like(o1)
    bundles.Multi(lin, o1).run(hk, norm_in=(sqk, w, 1e-5, torch.empty((1, k), dtype=torch.half, device="cuda")))
    bundles.Multi(lin, o2).run(r_ref.view(1, 1, k))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
