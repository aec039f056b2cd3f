"""GEMV row groups of 9..16 rows whose matrix-core plan does not fit the split-partial workspace,
and the forced GEMV route for any row count.

A 16-row group on the matrix-core GEMV needs (k/16 / SB) * slots * 16 * n * 4 bytes of fp32
split partials (SB <= 32 k-slices per workgroup).  When that exceeds the workspace (64 MiB for
exl3_amd_gemm / exl3_amd_mgemm, 16 MiB for exl3_amd_gemm_noalloc), or the matrix-core GEMV is
switched off by policy, the group runs as two launches of at most 8 rows on the LDS kernel
(rows [row0, row0 + 8) and the rest of the group, same slabs).  force_shape_idx = 1 routes any
row count through the GEMV in such groups.

Bar: max relative error 2e-3 (tests/tol.py) against the fp64 linear of the oracle; at the large
shapes on two 128-column chunks of the output (column chunks are independent: the output
rotation acts within a chunk), and against exl3_amd_gemm on the whole output.
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


def ref_cols(orc, L, x, c0, width=256):
    """fp64 linear of output columns [c0, c0 + width) (whole 128-column chunks)."""
    t = np.ascontiguousarray(L.trellis[:, c0 // 16:(c0 + width) // 16, :])
    return orc.linear_f64(x, t, L.suh, np.ascontiguousarray(L.svh[c0:c0 + width]), int(L.K),
                          half=L.K != int(L.K), cb=L.cb)


def call(torch, entry, L, x, force=0):
    t, s, v = L.torch()
    A = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    A_had = torch.empty_like(A)
    C = torch.full((x.shape[0], L.n), float("nan"), dtype=torch.half, device="cuda")
    rc = getattr(_lib.lib(), entry)(A.data_ptr(), t.data_ptr(), C.data_ptr(), 0, s.data_ptr(), A_had.data_ptr(),
                                    v.data_ptr(), x.shape[0], L.k, L.n, float(L.K), int(L.cb == 1),
                                    int(L.cb == 2), force, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return rc, C.cpu().numpy()


def test_noalloc_16_rows_over_scratch(torch_cuda, orc):
    """16 rows of 20480 -> 8192: the matrix-core plan needs >= 20 MiB of partials (16 MiB of
    scratch), so the group runs as 8 + 8 rows."""
    torch = torch_cuda
    L = synth.layer(20480, 8192, 2, 0, seed=8101)
    x = synth.activations(16, 20480, seed=8102)
    rc1, y1 = call(torch, "exl3_amd_gemm_noalloc", L, x)
    rc0, y0 = call(torch, "exl3_amd_gemm", L, x)
    assert rc1 == 90 and rc0 == 90, (rc0, rc1)
    assert np.isfinite(y1.astype(np.float32)).all()
    assert_close(y1, y0, what="noalloc (split groups) vs gemm")
    for c0 in (0, 8192 - 256):
        assert_close(y1[:, c0:c0 + 256], ref_cols(orc, L, x, c0), what=f"noalloc columns {c0}")


@pytest.mark.parametrize("m", [9, 12, 16])
def test_lds_policy_splits_groups(torch_cuda, orc, kernel_policy, m):
    """The matrix-core GEMV off: exl3_mgemm with 9..16 rows per group runs 8 + (m - 8) rows."""
    torch = torch_cuda
    from ampstein_amd import ops
    kernel_policy(_lib.POLICY_GEMV_ROWS, _lib.GEMV_ROWS_LDS)
    layers = [synth.layer(1024, 512, 3, 0, seed=8200 + i) for i in range(2)]
    dev = [L.torch() for L in layers]
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    B, suh, svh = (P([d[i].data_ptr() for d in dev]) for i in range(3))
    x = synth.activations(m, 1024, seed=8210 + m)
    A = torch.from_numpy(x).cuda().unsqueeze(0)
    C = torch.full((2, m, 512), float("nan"), dtype=torch.half, device="cuda")
    A_had = torch.empty((2, m, 1024), dtype=torch.half, device="cuda")
    tag = ops.exl3_mgemm(A, B, C, suh, A_had, svh, None, None, 3)
    torch.cuda.synchronize()
    assert tag == 90
    y = C.cpu().numpy()
    for q, L in enumerate(layers):
        assert_close(y[q], orc.linear_f64(x, L.trellis, L.suh, L.svh, 3), what=f"slab {q}, {m} rows")


def test_mgemm_16_rows_over_workspace(torch_cuda, orc):
    """Four slots of 20480 -> 8192 at 16 rows need >= 80 MiB of matrix-core partials (64 MiB
    workspace): 8 + 8 rows on the LDS kernel, every slot against the fp64 linear on two chunks."""
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(20480, 8192, 2, 0, seed=8301)
    t, s, v = L.torch()
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    B, suh, svh = P([t.data_ptr()] * 4), P([s.data_ptr()] * 4), P([v.data_ptr()] * 4)
    x = synth.activations(16 * 4, 20480, seed=8302).reshape(4, 16, 20480)
    A = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    C = torch.full((4, 16, 8192), float("nan"), dtype=torch.half, device="cuda")
    A_had = torch.empty_like(A)
    tag = ops.exl3_mgemm(A, B, C, suh, A_had, svh, None, None, 2)
    torch.cuda.synchronize()
    assert tag == 90
    y = C.cpu().numpy()
    assert np.isfinite(y.astype(np.float32)).all()
    for q in range(4):
        for c0 in (0, 4096):
            assert_close(y[q][:, c0:c0 + 256], ref_cols(orc, L, x[q], c0), what=f"slot {q} columns {c0}")


@pytest.mark.parametrize("m", [12, 40])
def test_force_gemv_any_rows(torch_cuda, orc, m):
    """force_shape_idx = 1: the GEMV in 16-row groups for any row count (A_had still written)."""
    torch = torch_cuda
    L = synth.layer(1024, 768, 4, 1, seed=8400 + m)
    x = synth.activations(m, 1024, seed=8401)
    rc, y = call(torch, "exl3_amd_gemm", L, x, force=1)
    assert rc == 90
    assert_close(y, orc.linear_f64(x, L.trellis, L.suh, L.svh, 4, cb=1), what=f"forced GEMV, {m} rows")
