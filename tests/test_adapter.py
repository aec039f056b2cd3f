"""The at::Tensor adapter (ampstein_amd/adapter/exl3_amd_adapter.cpp): the operators ampstein's
bindings call, with amp_torch.cpp's C++ signatures, over the C ABI.

CPU: the module loads, exposes the operators, and raises c10::Error (RuntimeError) on bad
arguments before any launch, as the vendored TORCH_CHECKs do (tests/bindings_errors.uc of the
reference requires every binding to raise on bad arguments).
GPU: each operator against the CPU oracle on seeded inputs, to the bars of the direct tests
(bit-exact reconstruct, < 2e-3 relative for the GEMV / GEMM / MoE outputs).
"""
import numpy as np
import pytest
import torch

from ampstein_amd import synth, torch_adapter

TOL = 2e-3
OPS = ("exl3_gemm", "exl3_mgemm", "exl3_moe_coop", "had_r_128", "reconstruct", "reconstruct_had_slice",
       "exl3_moe", "exl3_moe_gather", "exl3_moe_max_concurrency", "rms_norm_res", "silu_mul")


@pytest.fixture(scope="module")
def ad():
    return torch_adapter.load()


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def test_adapter_exports_operators(ad):
    for name in OPS:
        assert callable(getattr(ad, name)), name


def test_adapter_rejects_bad_arguments(ad):
    h = lambda *s: torch.zeros(s, dtype=torch.half)
    B = torch.zeros((8, 8, 64), dtype=torch.int16)
    with pytest.raises(RuntimeError, match="A is incorrect datatype"):
        ad.exl3_gemm(torch.zeros((1, 128)), B, h(1, 128), None, None, None, 0, False, False, 0)
    with pytest.raises(RuntimeError, match="A and B shapes"):
        ad.exl3_gemm(h(1, 64), B, h(1, 128), None, None, None, 0, False, False, 0)
    with pytest.raises(RuntimeError, match="both mcg and mul1"):
        ad.exl3_gemm(h(1, 128), B, h(1, 128), None, None, None, 0, True, True, 0)
    with pytest.raises(RuntimeError, match="half-integer"):
        ad.exl3_gemm(h(1, 128), torch.zeros((8, 8, 40), dtype=torch.int16), h(1, 128), None, None, None,
                     0, False, False, 0)
    with pytest.raises(RuntimeError, match="must be a GPU tensor"):
        ad.exl3_gemm(h(1, 128), B, h(1, 128), None, None, None, 0, False, False, 0)
    with pytest.raises(RuntimeError, match="unpacked is incorrect datatype"):
        ad.reconstruct(torch.zeros((128, 128)), B, 4.0, False, False)
    with pytest.raises(RuntimeError, match="divisible by 128"):
        ad.had_r_128(h(2, 100), h(2, 100), None, None, 1.0)
    with pytest.raises(RuntimeError, match="unsupported datatype"):
        ad.had_r_128(torch.zeros((2, 128), dtype=torch.int32), torch.zeros((2, 128), dtype=torch.int32),
                     None, None, 1.0)
    L = torch.zeros(2, dtype=torch.long)
    with pytest.raises(RuntimeError, match="A must have 3 dimensions"):
        ad.exl3_mgemm(h(1, 128), L, h(2, 1, 128), L, h(0), L, None, None, 4.0, -1, 0, 0, -1, -1, 0, 1,
                      None, None, None, None, 0)
    x, sel, rw = h(1, 256), torch.zeros((1, 4), dtype=torch.long), h(1, 3)
    with pytest.raises(RuntimeError, match="sel/rw must be"):
        ad.exl3_moe_coop(x, sel, rw, -1, -1, 256, *([L] * 9), None, None, None, 4.0, 4.0, 4.0, False, False,
                         0, 0.0, True, h(4, 256), h(4, 256), h(4, 256), h(4, 256), h(4, 256),
                         torch.zeros((4, 256)), torch.zeros(64, dtype=torch.int32), torch.zeros((1, 256)),
                         None, None, None, None, None)


def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ampstein_amd import ops
    ops.init(0)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 5, 32])
@pytest.mark.parametrize("K,cb", [(4, 0), (3, 1), (2, 2)])
def test_adapter_exl3_gemm(ad, orc, m, K, cb):
    """GEMV (m <= 8, tag 90), and m = 32 (A_had written) through the adapter: the library routes
    this small shape to 16-row GEMV groups (tag 90); force_shape_idx 2 takes the MFMA GEMM."""
    gpu()
    L = synth.layer(512, 384, K, cb, seed=300 + 10 * K + cb)
    t, s, v = L.torch("cuda:0")
    x = synth.activations(m, 512, seed=m)
    A = torch.from_numpy(x).cuda()
    A_had = torch.empty_like(A)
    C = torch.empty((m, 384), dtype=torch.half, device="cuda")
    tag = ad.exl3_gemm(A, t, C, s, A_had, v, 0 if m <= 8 else 2, cb == 1, cb == 2, 0)
    torch.cuda.synchronize()
    assert tag == (90 if m <= 8 else 91)
    ref = orc.linear(x, L.trellis, L.suh, L.svh, K, cb=cb)
    assert rel_err(C.cpu().numpy(), ref) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("K,cb", [(4, 0), (2, 1), (5, 2)])
def test_adapter_reconstruct_bit_exact(ad, orc, K, cb):
    gpu()
    L = synth.layer(256, 512, K, cb, seed=400 + K)
    t, s, v = L.torch("cuda:0")
    W = torch.empty((256, 512), dtype=torch.half, device="cuda")
    ad.reconstruct(W, t, float(K), cb == 1, cb == 2)
    Wh = torch.empty((256, 256), dtype=torch.half, device="cuda")
    ad.reconstruct_had_slice(Wh, t, s, v, float(K), cb == 1, cb == 2, 128)
    torch.cuda.synchronize()
    assert np.array_equal(W.cpu().numpy().view(np.uint16), orc.reconstruct(L.trellis, K, cb=cb).view(np.uint16))
    ref_had = orc.reconstruct_had(L.trellis, L.suh, L.svh, K, cb=cb, n=256, n_offset=128)
    assert np.array_equal(Wh.cpu().numpy().view(np.uint16), ref_had.view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("fp32", [False, True])
def test_adapter_had_r_128(ad, orc, fp32):
    gpu()
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 384)).astype(np.float32 if fp32 else np.float16)
    pre = synth.signs(rng, 384)
    xi = torch.from_numpy(x).cuda()
    y = torch.empty_like(xi)
    ad.had_r_128(xi, y, torch.from_numpy(pre).cuda(), None, 1.0)
    ad.had_r_128(xi, xi, None, None, 1.0)      # in place
    torch.cuda.synchronize()
    ref = orc.had128(x.astype(np.float32) if fp32 else x, pre=pre)
    assert rel_err(y.cpu().numpy(), ref) < 1e-3
    assert rel_err(xi.cpu().numpy(), orc.had128(x.astype(np.float32) if fp32 else x)) < 1e-3


@pytest.mark.gpu
def test_adapter_exl3_mgemm_stacked(ad, orc):
    gpu()
    layers = [synth.layer(512, 1024, 4, 0, seed=500 + i) for i in range(2)]
    dev = [L.torch("cuda:0") for L in layers]
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    B, suh, svh = P([d[0].data_ptr() for d in dev]), P([d[1].data_ptr() for d in dev]), P([d[2].data_ptr() for d in dev])
    x = synth.activations(2, 512, seed=3)
    A = torch.from_numpy(x[None]).cuda()
    C = torch.empty((2, 2, 1024), dtype=torch.float, device="cuda")
    A_had = torch.empty((2, 2, 512), dtype=torch.half, device="cuda")
    tag = ad.exl3_mgemm(A, B, C, suh, A_had, svh, None, None, 4.0, -1, 0, 0, -1, -1, 0, 1, None, None, None, None, 0)
    torch.cuda.synchronize()
    assert tag == 90
    for q, L in enumerate(layers):
        ref = orc.linear(x, L.trellis, L.suh, L.svh, 4, y_fp32=True)
        assert rel_err(C[q].cpu().numpy(), ref) < TOL


@pytest.mark.gpu
def test_adapter_exl3_moe_coop(ad, orc):
    """Mixed-K MoE through the adapter: same routing semantics and tolerance as test_gpu_moe."""
    gpu()
    from tests import moe_ref
    from tests.test_gpu_moe import check_runs, routing, run
    rng = np.random.default_rng(5)
    es = moe_ref.ExpertSet(torch, orc, 16, 256, 1024, 1024, rng.choice([2, 3, 4], 16), 2, seed=5, bias=True)
    rng = np.random.default_rng(108)
    sel, rw = routing(rng, 8, 16, 8)
    x = rng.standard_normal((8, 256)).astype(np.float16)
    y, runs = run(torch, es, x, sel, rw, moe_fn=ad.exl3_moe_coop)
    ref = moe_ref.reference(es, x, sel, rw, -1, -1, 0, True, 0.0, 1024)
    assert rel_err(y, ref) < TOL
    check_runs(runs, sel, rw, -1, -1)


def test_adapter_moe_rejects_bad_arguments(ad):
    h = lambda *s: torch.zeros(s, dtype=torch.half)
    L = lambda *s: torch.zeros(s, dtype=torch.long)
    tabs = [L(4) for _ in range(9)]
    with pytest.raises(RuntimeError, match="output_scratch needs fused_base"):
        ad.exl3_moe(h(2, 128), torch.zeros((2, 128)), L(5), L(4), h(4), h(1, 4, 128), h(1, 4, 128), h(1, 4, 128),
                    h(1, 4, 128), 0, 3.0, 3.0, 3.0, *tabs, True, False, True, False, True, False, 0.0, 1,
                    torch.zeros((4, 128)), None, 0, 1 << 30, 16, None, None, None)
    with pytest.raises(RuntimeError, match="output_state is incorrect datatype"):
        ad.exl3_moe(h(2, 128), h(2, 128), L(5), L(4), h(4), h(1, 4, 128), h(1, 4, 128), h(1, 4, 128),
                    h(1, 4, 128), 0, 3.0, 3.0, 3.0, *tabs, True, False, True, False, True, False, 0.0, 1,
                    None, None, 0, 1 << 30, 16, None, None, None)
    with pytest.raises(RuntimeError, match="weight_sorted is incorrect datatype"):
        ad.exl3_moe_gather(torch.zeros((2, 128)), torch.zeros((4, 128)), L(4), L(4), L(3), L(3), L(3), L(4))


@pytest.mark.gpu
def test_adapter_exl3_moe_and_gather(ad, orc):
    """Slot mode through the adapter: bit-identical to the same call through the C ABI's
    Python front end, then the fixed-order gather (also bit-identical)."""
    from ampstein_amd import ops
    from tests.moe_ref import ExpertSet
    from tests.test_gpu_moe_sorted import routing
    E, H, I, T, topk = 6, 256, 256, 24, 2
    es = ExpertSet(torch, orc, E, H, I, H, [3] * E, 1, seed=5)
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((T, H)).astype(np.float16)).cuda()
    flat, order, inv, tok, ws, count, start = routing(T, E, topk, seed=4)
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    fb = dv(start[:E])
    tb = es.tables
    tabs = [tb[n] for n in ("g_trellis", "g_suh", "g_svh", "u_trellis", "u_suh", "u_svh", "d_trellis", "d_suh", "d_svh")]
    outs = []
    for fn in (ad.exl3_moe, ops.exl3_moe):
        tmp = [torch.zeros((1, 64, w), dtype=torch.half, device="cuda") for w in (H, H, I, I)]
        out = torch.zeros((T, H), dtype=torch.float, device="cuda")
        scr = torch.zeros((T * topk, H), dtype=torch.float, device="cuda")
        fn(x, out, dv(count), dv(tok), dv(ws), *tmp, 0, 3.0, 3.0, 3.0, *tabs, True, False, True, False, True, False,
           0.0, E, scr, fb, 0, 1 << 30, 16, None, None, None)
        kind = dv(np.ones(E, np.int64))
        g = ad.exl3_moe_gather if fn is ad.exl3_moe else ops.exl3_moe_gather
        g(out, scr, dv(flat), dv(inv), dv(start), fb, kind, dv(ws))
        torch.cuda.synchronize()
        outs.append((scr.cpu().numpy(), out.cpu().numpy()))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    assert np.abs(outs[0][1]).max() > 0
    assert ad.exl3_moe_max_concurrency(0) == ops.exl3_moe_max_concurrency(0)


@pytest.mark.gpu
def test_adapter_decode_neighbours(ad):
    from ampstein_amd import ops
    rng = np.random.default_rng(8)
    x, r = (torch.from_numpy(rng.standard_normal((2, 1024)).astype(np.float16)).cuda() for _ in range(2))
    w = torch.from_numpy((rng.standard_normal(1024) * 0.1 + 1).astype(np.float16)).cuda()
    y, n = torch.empty_like(x), torch.empty_like(x)
    ad.rms_norm_res(x, r, w, y, n, 1e-6)
    y2, n2 = ops.rms_norm_res(x, r, w, 1e-6)
    assert torch.equal(y, y2) and torch.equal(n, n2)
    out = torch.empty_like(x)
    ad.silu_mul(x, r, out)
    assert torch.equal(out, ops.silu_mul(x, r))
