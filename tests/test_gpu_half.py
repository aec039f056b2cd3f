"""GPU parity at half-integer bitrates (1.5 / 2.5 / 3.5 bits, mul1 codebook: tiles of 16K + 8
u16, bits_k.cuh:8-27) for the GEMV paths against the CPU oracle's fp64 linear.  The oracle's
half-rate window extraction is pinned against a bit-string model in tests/test_oracle.py.

Covers exl3_gemm at 1..8 rows (streaming M = 1 kernel and the multi-row GEMV), more rows (the
MFMA GEMM's half-rate tile decode, tag 91), fp16 / fp32 outputs, and exl3_mgemm stacked bundles on the XCD hand-off
(1024 columns) and the finish-kernel path (384 columns).  Bar: max|y - ref| / max|ref| < 2e-3.
"""
import numpy as np
import pytest

from ampstein_amd import synth

pytestmark = pytest.mark.gpu

TOL = 2e-3
HALF_KS = [1.5, 2.5, 3.5]


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


@pytest.mark.parametrize("K", HALF_KS)
@pytest.mark.parametrize("m", [1, 5, 8, 20, 300])
@pytest.mark.parametrize("y_fp32", [False, True])
def test_gemm_half_rate(torch_cuda, orc, K, m, y_fp32):
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(512, 1024, K, 2, seed=int(100 * K) + m)
    x = synth.activations(m, 512, seed=m)
    t, s, v = L.torch()
    A = torch.from_numpy(x).cuda()
    C = torch.empty((m, 1024), dtype=torch.float if y_fp32 else torch.half, device="cuda")
    # m > 8: force the MFMA GEMM (the library routes these small shapes to the GEMV)
    tag = ops.exl3_gemm(A, t, C, s, torch.empty_like(A), v, 0 if m <= 8 else 2, False, True)
    torch.cuda.synchronize()
    assert tag == (90 if m <= 8 else 91)
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=True, cb=2)
    assert rel_err(C.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("K", HALF_KS)
@pytest.mark.parametrize("n", [1024, 384])
@pytest.mark.parametrize("m", [1, 3])
def test_mgemm_half_rate(torch_cuda, orc, K, n, m):
    torch = torch_cuda
    from ampstein_amd import ops
    layers = [synth.layer(256, n, K, 2, seed=int(10 * K) + i + n) for i in range(3)]
    dev = [L.torch() for L in layers]
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    B, suh, svh = P([d[0].data_ptr() for d in dev]), P([d[1].data_ptr() for d in dev]), P([d[2].data_ptr() for d in dev])
    x = synth.activations(m, 256, seed=m + 11)
    C = torch.empty((3, m, n), dtype=torch.half, device="cuda")
    A_had = torch.empty((3, m, 256), dtype=torch.half, device="cuda")
    ops.mgemm(torch.from_numpy(x[None]).cuda(), B, C, suh, A_had, svh, K, False, True)
    torch.cuda.synchronize()
    got = C.cpu().numpy()
    for q, L in enumerate(layers):
        ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=True, cb=2)
        assert rel_err(got[q], ref) < TOL, q
