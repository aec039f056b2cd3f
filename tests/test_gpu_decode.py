"""Decode-step neighbours and the captured decode step (graphdec.uc:151-230).

rms_norm_res (amp_kernels.cu:279-365): y = fp16(x + r) bit for bit; n within one fp16 ulp of the
fp64 statement (the fp32 sum of squares runs in another order than the reference's warp tree).
silu_mul (amp_kernels.cu:235-251): within one fp16 ulp of fp64 silu(g) * u rounded once.
exl3_gemm_silu_mul: bit-identical to silu_mul followed by exl3_gemm (fused at one row, two calls
above).  DecodeStack: graph replays bit-identical to the eager step (with eager work between
replays), fused and unfused SwiGLU bit-identical, and the step within 5e-3 of a CPU model built
from the oracle's linears.
"""
import numpy as np
import pytest
import torch

from ampstein_amd import bundles, ops, synth

pytestmark = pytest.mark.gpu


def f16(v):
    return np.asarray(v, np.float64).astype(np.float16)


def ulp_diff(a, b):
    ia = a.view(np.int16).astype(np.int32)
    ib = b.view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


def norm_model(x, r, w, eps):
    y = f16(x.astype(np.float64) + r.astype(np.float64))
    yy = y.astype(np.float64)
    scale = 1.0 / np.sqrt((yy * yy).mean(axis=-1, keepdims=True) + eps)
    n = f16(f16(yy * scale).astype(np.float64) * w.astype(np.float64))
    return y, n


@pytest.mark.parametrize("rows,dim", [(1, 4096), (3, 5120), (2, 1028), (1, 64)])
def test_rms_norm_res(rows, dim):
    rng = np.random.default_rng(dim + rows)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float16)
    r = (rng.standard_normal((rows, dim)) * 2).astype(np.float16)
    w = (rng.standard_normal(dim) * 0.5 + 1).astype(np.float16)
    xs, rs, ws = (torch.from_numpy(a).cuda() for a in (x, r, w))
    y, n = ops.rms_norm_res(xs, rs, ws, 1e-5)
    ye, ne = norm_model(x, r, w, 1e-5)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), ye.view(np.uint16))
    assert ulp_diff(n.cpu().numpy(), ne).max() <= 1
    # in place: y aliases x
    ops.rms_norm_res(xs, rs, ws, 1e-5, y=xs, n=n)
    assert np.array_equal(xs.cpu().numpy().view(np.uint16), ye.view(np.uint16))


def test_silu_mul():
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(40000) * 4).astype(np.float16)
    u = (rng.standard_normal(40000) * 2).astype(np.float16)
    out = ops.silu_mul(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()).cpu().numpy()
    gg = g.astype(np.float64)
    ref = f16(gg / (1.0 + np.exp(-gg)) * u.astype(np.float64))
    assert ulp_diff(out, ref).max() <= 1


@pytest.mark.parametrize("m", [1, 3, 12])
@pytest.mark.parametrize("K,cb", [(4, 0), (3, 1), (2, 2), (2.5, 2)])
def test_gemm_silu_mul_matches_two_calls(m, K, cb):
    k, n = 1024, 512
    L = synth.layer(k, n, K, cb, seed=int(10 * K) + cb)
    t, s, v = L.torch("cuda")
    rng = np.random.default_rng(m)
    g = torch.from_numpy((rng.standard_normal((m, k)) * 2).astype(np.float16)).cuda()
    u = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).cuda()
    C1 = torch.empty((m, n), dtype=torch.half, device="cuda")
    C2 = torch.empty_like(C1)
    tag = ops.exl3_gemm_silu_mul(g, u, t, C1, s, v, cb == 1, cb == 2)
    a = ops.silu_mul(g, u)
    tag2 = ops.exl3_gemm(a, t, C2, s, torch.empty_like(a), v, 0, cb == 1, cb == 2)
    assert tag == tag2
    assert np.array_equal(C1.cpu().numpy().view(np.uint16), C2.cpu().numpy().view(np.uint16))


def _stack(H, Q, KV, I, n_layers, K=4, cb=0, fuse=True):
    seed = [100]

    def lin(k, n):
        seed[0] += 1
        L = synth.layer(k, n, K, cb, seed=seed[0])
        # checkpoints carry the output scale in svh: 1/16 (exact in fp16) keeps the stack in range
        L.svh = (L.svh.astype(np.float32) / 16).astype(np.float16)
        t, s, v = L.torch("cuda")
        return bundles.Linear(t, s, v, float(K), cb == 1, cb == 2), L

    from ampstein_amd.decode import DecodeStack, LayerWeights
    rng = np.random.default_rng(9)
    layers, host = [], []
    for _ in range(n_layers):
        parts = {name: lin(k, n) for name, (k, n) in
                 dict(q=(H, Q), k=(H, KV), v=(H, KV), o=(Q, H), gate=(H, I), up=(H, I), down=(I, H)).items()}
        wi = (rng.standard_normal(H) * 0.2 + 1).astype(np.float16)
        wp = (rng.standard_normal(H) * 0.2 + 1).astype(np.float16)
        layers.append(LayerWeights(**{k2: p[0] for k2, p in parts.items()},
                                   input_norm=torch.from_numpy(wi).cuda(), post_norm=torch.from_numpy(wp).cuda()))
        host.append(({k2: p[1] for k2, p in parts.items()}, wi, wp))
    wf = (rng.standard_normal(H) * 0.2 + 1).astype(np.float16)
    return DecodeStack(layers, torch.from_numpy(wf).cuda(), fuse_swiglu=fuse, split_norm=False), host, wf


def _model(host, wf, x, K, cb, eps=1e-5):
    from oracle import oracle as orc

    def lin(L, v):
        return orc.linear(v.reshape(1, -1), L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)

    h = x.reshape(1, -1).astype(np.float16)
    res = np.zeros_like(h)
    for parts, wi, wp in host:
        h, r = norm_model(h, res, wi, eps)
        q = lin(parts["q"], r)
        o = lin(parts["o"], q)
        h, r = norm_model(h, o, wp, eps)
        g, u = lin(parts["gate"], r), lin(parts["up"], r)
        gg = g.astype(np.float64)
        a = f16(gg / (1.0 + np.exp(-gg)) * u.astype(np.float64))
        res = lin(parts["down"], a)
    return norm_model(h, res, wf, eps)[1]


def test_decode_stack_graph_and_model(orc):
    H, Q, KV, I = 512, 512, 128, 1024
    st, host, wf = _stack(H, Q, KV, I, 2)
    st_u, _, _ = _stack(H, Q, KV, I, 2, fuse=False)
    rng = np.random.default_rng(3)
    xs = [rng.standard_normal(H).astype(np.float16) for _ in range(3)]
    eager = [st(torch.from_numpy(x).cuda()).clone() for x in xs]
    unfused = [st_u(torch.from_numpy(x).cuda()).clone() for x in xs]
    for a, b in zip(eager, unfused):
        assert torch.equal(a, b), "fused and unfused SwiGLU differ"
    st.capture()
    for rep in range(2):
        for x, e in zip(xs, eager):
            y = st(torch.from_numpy(x).cuda())
            torch.cuda.synchronize()
            assert torch.equal(y, e), f"graph replay {rep} differs from the eager step"
            _ = torch.randn(1000, device="cuda").sum()        # eager work between replays
    for x, e in zip(xs, eager):
        ref = _model(host, wf, x, 4, 0).astype(np.float64)
        got = e.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"decode stack rel err {err:.2e}", flush=True)
        assert err < 5e-3


@pytest.mark.parametrize("k,n", [(4096, 4096), (1024, 5120), (512, 640), (14336, 1024)])
@pytest.mark.parametrize("swiglu", [False, True])
def test_gemm_norm_matches_two_calls(k, n, swiglu):
    """Fused residual norm in the GEMV's last chunk: C and the updated residual bit-identical to
    exl3_gemm + rms_norm_res, the normed row within one fp16 ulp (the sum of squares is
    reduced in another order)."""
    L = synth.layer(k, n, 4, 0, seed=k + n)
    L.svh = (L.svh.astype(np.float32) / 16).astype(np.float16)
    t, s, v = L.torch("cuda")
    rng = np.random.default_rng(n)
    a = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float16)).cuda()
    up = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float16)).cuda() if swiglu else None
    h0 = torch.from_numpy((rng.standard_normal((1, n)) * 4).astype(np.float16)).cuda()
    w = torch.from_numpy((rng.standard_normal(n) * 0.2 + 1).astype(np.float16)).cuda()
    C1, r1, h1 = torch.empty((1, n), dtype=torch.half, device="cuda"), torch.empty((1, n), dtype=torch.half, device="cuda"), h0.clone()
    for rep in range(2):                  # the row counter must re-arm: a second call behaves the same
        h1.copy_(h0)
        ops.exl3_gemm_norm(a, t, C1, s, v, h1, w, r1, 1e-5, up=up)
        torch.cuda.synchronize()
        C2 = torch.empty_like(C1)
        if swiglu:
            ops.exl3_gemm_silu_mul(a, up, t, C2, s, v)
        else:
            ops.exl3_gemm(a, t, C2, s, torch.empty_like(a), v)
        h2, r2 = ops.rms_norm_res(h0, C2, w, 1e-5)
        assert torch.equal(C1, C2)
        assert torch.equal(h1, h2)
        assert ulp_diff(r1.cpu().numpy(), r2.cpu().numpy()).max() <= 1


def test_decode_stack_fused_norm(orc):
    H, Q, KV, I = 512, 512, 128, 1024
    st, host, wf = _stack(H, Q, KV, I, 2)
    st.fuse_norm = True
    rng = np.random.default_rng(13)
    xs = [rng.standard_normal(H).astype(np.float16) for _ in range(2)]
    eager = [st(torch.from_numpy(x).cuda()).clone() for x in xs]
    st.capture()
    for rep in range(2):
        for x, e in zip(xs, eager):
            y = st(torch.from_numpy(x).cuda())
            torch.cuda.synchronize()
            assert torch.equal(y, e), f"graph replay {rep} differs from the eager step"
    for x, e in zip(xs, eager):
        ref = _model(host, wf, x, 4, 0).astype(np.float64)
        got = e.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"decode stack (fused norm) rel err {err:.2e}", flush=True)
        assert err < 5e-3
