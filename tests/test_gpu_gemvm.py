"""GPU parity of the row-batched matrix-core GEMV (gemvm_kernel: 2..16 rows, and single rows
when the policy EXL3_AMD_GEMV_ROWS_MFMA_ALL routes them there) against the CPU oracle.

Covers every integer K and codebook, the half rates, fp16 / fp32 outputs, column-chunk counts
that take the XCD hand-off (8 chunks) and the finish kernel (3 chunks), one to sixteen rows
(mgemm row groups), and a second call that must reproduce the first bit for bit.
Bar (tests/tol.py): max relative error 2e-3, norm-wise and element-wise, against the fp64 linear.
"""
import numpy as np
import pytest

from ampstein_amd import _lib, synth
from tests.tol import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ampstein_amd import ops
    ops.init(0)
    return torch


def run(torch, L, x, y_fp32):
    from ampstein_amd import ops
    t, s, v = L.torch()
    A = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    C = torch.full((x.shape[0], L.n), float("nan"), dtype=torch.float if y_fp32 else torch.half, device="cuda")
    tag = ops.exl3_gemm(A, t, C, s, torch.empty_like(A), v, 0, L.cb == 1, L.cb == 2)
    torch.cuda.synchronize()
    return tag, C.cpu().numpy()


@pytest.mark.parametrize("K,cb", [(k, c) for k in range(1, 9) for c in range(3)] + [(1.5, 2), (2.5, 2), (3.5, 2)])
@pytest.mark.parametrize("m", [1, 2, 5, 8])
def test_gemvm_parity(torch_cuda, orc, kernel_policy, K, cb, m):
    kernel_policy(_lib.POLICY_GEMV_ROWS, _lib.GEMV_ROWS_MFMA_ALL)
    torch = torch_cuda
    L = synth.layer(1024, 1024, K, cb, seed=900 + int(10 * K) + cb)
    x = synth.activations(m, 1024, seed=m + int(K))
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)
    tag, y = run(torch, L, x, False)
    assert tag == 90
    assert_close(y, ref, what=f"K{K} cb{cb} m{m}")
    _, y2 = run(torch, L, x, False)
    assert np.array_equal(y.view(np.uint16), y2.view(np.uint16))


@pytest.mark.parametrize("k,n", [(256, 384), (4096, 1024), (14336, 4096), (5120, 17408)])
@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("y_fp32", [False, True])
def test_gemvm_shapes(torch_cuda, orc, kernel_policy, k, n, m, y_fp32):
    kernel_policy(_lib.POLICY_GEMV_ROWS, _lib.GEMV_ROWS_MFMA_ALL)
    torch = torch_cuda
    L = synth.layer(k, n, 4, 0, seed=950 + k + n)
    x = synth.activations(m, k, seed=951)
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, 4)
    tag, y = run(torch, L, x, y_fp32)
    assert tag == 90
    assert_close(y, ref, what=f"{k}x{n} m{m}")


@pytest.mark.parametrize("m", [12, 16, 20])
def test_gemvm_mgemm_row_groups(torch_cuda, orc, m):
    """exl3_mgemm with more than 8 rows: row groups through the matrix-core kernel."""
    torch = torch_cuda
    from ampstein_amd import ops
    layers = [synth.layer(512, 1024, 3, 1, seed=970 + i) for i in range(2)]
    dev = [L.torch() for L in layers]
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    B, suh, svh = (P([d[i].data_ptr() for d in dev]) for i in range(3))
    x = synth.activations(m, 512, seed=971)
    C = torch.full((2, m, 1024), float("nan"), dtype=torch.half, device="cuda")
    A_had = torch.empty((2, m, 512), dtype=torch.half, device="cuda")
    ops.exl3_mgemm(torch.from_numpy(x[None]).cuda(), B, C, suh, A_had, svh, None, None, 3, mcg=1)
    torch.cuda.synchronize()
    got = C.cpu().numpy()
    for q, L in enumerate(layers):
        assert_close(got[q], orc.linear_f64(x, L.trellis, L.suh, L.svh, 3, cb=1), what=f"slot {q}")

