"""GPU parity of the HIP path (through the C ABI, via ampstein_amd.ops) against the CPU oracle.

Bars: reconstruct / reconstruct_had / had_r_128 bit-exact; GEMV outputs within 2e-3 of the
oracle's fp32-accumulated reference, measured as max|y - y_ref| / max|y_ref| (elementwise
relative error is undefined near zero outputs).
"""
import numpy as np
import pytest

from ampstein_amd import synth

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ampstein_amd import ops
    ops.init(0)
    return torch


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def to_gpu(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


KS = list(range(1, 9))


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("K", KS)
def test_reconstruct_bit_exact(torch_cuda, orc, K, cb):
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(256, 384, K, cb, seed=100 * K + cb)
    ref = orc.reconstruct(L.trellis, K, cb=cb)
    W = torch.empty((256, 384), dtype=torch.half, device="cuda")
    ops.reconstruct(W, to_gpu(torch, L.trellis, torch.int16), K, mcg=cb == 1, mul1=cb == 2)
    got = W.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("K", [1.5, 2.5, 3.5])
def test_reconstruct_half_rate_bit_exact(torch_cuda, orc, K):
    """Half-integer bitrates (mul1, 16K + 8 u16 per tile): reconstruct, a column slice,
    the transposed layout and the original-basis form, bit for bit against the oracle."""
    torch = torch_cuda
    from ampstein_amd import ops
    b = int(K)
    L = synth.layer(256, 384, K, 2, seed=int(40 * K))
    t, s, v = L.torch()
    ref = orc.reconstruct(L.trellis, b, half=True, cb=2)
    W = torch.empty((256, 384), dtype=torch.half, device="cuda")
    ops.reconstruct(W, t, K, mul1=True)
    assert np.array_equal(W.cpu().numpy().view(np.uint16), ref.view(np.uint16))
    Ws = torch.empty((256, 256), dtype=torch.half, device="cuda")
    ops.reconstruct_slice(Ws, t, K, False, True, 128)
    assert np.array_equal(Ws.cpu().numpy().view(np.uint16), ref[:, 128:].view(np.uint16))
    WT = torch.empty((384, 256), dtype=torch.half, device="cuda")
    ops.reconstruct_t(WT, t, K, False, True)
    assert np.array_equal(WT.cpu().numpy().view(np.uint16), np.ascontiguousarray(ref.T).view(np.uint16))
    ref_had = orc.reconstruct_had(L.trellis, L.suh, L.svh, b, half=True, cb=2)
    Wh = torch.empty((256, 384), dtype=torch.half, device="cuda")
    ops.reconstruct_had_slice(Wh, t, s, v, K, False, True, 0)
    assert np.array_equal(Wh.cpu().numpy().view(np.uint16), ref_had.view(np.uint16))


def test_reconstruct_slice_bit_exact(torch_cuda, orc):
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(128, 512, 3, 1, seed=7)
    ref = orc.reconstruct(L.trellis, 3, cb=1, n=256, n_offset=128)
    W = torch.empty((128, 256), dtype=torch.half, device="cuda")
    ops.reconstruct_slice(W, to_gpu(torch, L.trellis, torch.int16), 3, True, False, 128)
    assert np.array_equal(W.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8])
def test_reconstruct_had_bit_exact(torch_cuda, orc, K, cb):
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(256, 256, K, cb, seed=200 + 10 * K + cb)
    ref = orc.reconstruct_had(L.trellis, L.suh, L.svh, K, cb=cb)
    W = torch.empty((256, 256), dtype=torch.half, device="cuda")
    t, s, v = L.torch()
    ops.reconstruct_had_slice(W, t, s, v, K, cb == 1, cb == 2, 0)
    got = W.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), \
        f"{np.sum(got.view(np.uint16) != ref.view(np.uint16))} mismatches"


@pytest.mark.parametrize("dtype", ["half", "float"])
@pytest.mark.parametrize("scales", ["none", "pre", "post"])
def test_had_r_128_bit_exact(torch_cuda, orc, dtype, scales):
    torch = torch_cuda
    from ampstein_amd import ops
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 384)).astype(np.float16 if dtype == "half" else np.float32)
    s = synth.signs(rng, 384) * np.float16(1.5)
    pre = s if scales == "pre" else None
    post = s if scales == "post" else None
    ref = orc.had128(x, pre=pre, post=post, scale=0.5)
    xt = to_gpu(torch, x)
    yt = torch.empty_like(xt)
    ops.had_r_128(xt, yt, None if pre is None else to_gpu(torch, pre),
                  None if post is None else to_gpu(torch, post), 0.5)
    got = yt.cpu().numpy()
    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8))
    ops.had_r_128(xt, xt, None, None, 1.0)          # in place
    assert np.array_equal(xt.cpu().numpy().view(np.uint8), orc.had128(x).view(np.uint8))


def run_gemm(torch, L, x, y_fp32, suh=True, svh=True):
    from ampstein_amd import ops
    t, s, v = L.torch()
    A = to_gpu(torch, x)
    C = torch.empty((x.shape[0], L.n), dtype=torch.float if y_fp32 else torch.half, device="cuda")
    tag = ops.exl3_gemm(A, t, C, s if suh else None, torch.empty_like(A), v if svh else None,
                        0, L.cb == 1, L.cb == 2)
    return tag, C.cpu().numpy()


@pytest.mark.parametrize("y_fp32", [False, True])
@pytest.mark.parametrize("m", [1, 2, 5, 8])
@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("K", KS)
def test_gemv_parity(torch_cuda, orc, K, cb, m, y_fp32):
    torch = torch_cuda
    L = synth.layer(512, 384, K, cb, seed=300 + 10 * K + cb)
    x = synth.activations(m, 512, seed=K)
    ref = orc.linear(x, L.trellis, L.suh, L.svh, K, cb=cb, y_fp32=y_fp32)
    tag, y = run_gemm(torch, L, x, y_fp32)
    assert tag == 90
    assert rel_err(y, ref) < TOL
    ref64 = orc.linear_f64(x, L.trellis, L.suh, L.svh, K, cb=cb)
    assert rel_err(y, ref64) < TOL


@pytest.mark.parametrize("suh,svh", [(False, False), (True, False), (False, True)])
def test_gemv_optional_rotations(torch_cuda, orc, suh, svh):
    torch = torch_cuda
    L = synth.layer(256, 256, 4, 0, seed=11)
    x = synth.activations(3, 256, seed=11)
    ref = orc.linear(x, L.trellis, L.suh if suh else None, L.svh if svh else None, 4, y_fp32=True)
    _, y = run_gemm(torch, L, x, True, suh, svh)
    assert rel_err(y, ref) < TOL


@pytest.mark.parametrize("k,n", [(4096, 4096), (14336, 1024), (4096, 14336), (128, 128)])
def test_gemv_shapes_and_splits(torch_cuda, orc, k, n):
    """Config-1 / Llama shapes: many k-splits, the cross-workgroup reduction, and the counter
    re-arm (a second call must reproduce the first bit for bit)."""
    torch = torch_cuda
    L = synth.layer(k, n, 4, 0, seed=1000 + k + n)
    x = synth.activations(1, k, seed=1)
    ref = orc.linear(x, L.trellis, L.suh, L.svh, 4)
    _, y1 = run_gemm(torch, L, x, False)
    _, y2 = run_gemm(torch, L, x, False)
    assert rel_err(y1, ref) < TOL
    assert np.array_equal(y1.view(np.uint16), y2.view(np.uint16))
