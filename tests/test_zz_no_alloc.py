"""exl3_amd_gemm_noalloc (the allocation-free variant of exl3_amd_gemm, scratch in a file-scope
device array) against exl3_amd_gemm through the C ABI, and both against the CPU oracle.

Two calls in a row on the same GPU, the second with a smaller input, so the second runs on the
scratch the first left behind (counters re-armed, partials overwritten).  Shapes cover the M = 1
stream kernel with a split k (the XCD hand-off after exl3_amd_init), the row-batched kernel
(m = 5), a half rate, the MFMA GEMM with its k split (m = 96: partial tiles in the scratch, fewer
splits than exl3_amd_gemm's 64 MiB workspace allows, so the two agree to the bar, not bit for bit)
and 16-row GEMV groups (m = 40).  A shape whose split partials exceed the 16 MiB scratch is
refused with EXL3_AMD_EUNSUPPORTED.
Bar: max relative error 2e-3 (tests/tol.py) against exl3_amd_gemm and against the fp64 linear.
"""
import numpy as np
import pytest

from ampstein_amd import synth
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


def call(torch, entry, L, x):
    from ampstein_amd import _lib
    t, s, v = L.torch()
    A = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    A_had = torch.empty_like(A)
    C = torch.full((x.shape[0], L.n), float("nan"), dtype=torch.half, device="cuda")
    lib = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    rc = getattr(lib, entry)(A.data_ptr(), t.data_ptr(), C.data_ptr(), 0, s.data_ptr(), A_had.data_ptr(),
                             v.data_ptr(), x.shape[0], L.k, L.n, float(L.K), int(L.cb == 1), int(L.cb == 2), 0, st)
    torch.cuda.synchronize()
    return rc, C.cpu().numpy()


CASES = [
    # (k, n, K, cb, m) first call, then a smaller one
    ((4096, 14336, 4, 0, 1), (4096, 1024, 4, 0, 1)),
    ((14336, 4096, 3, 1, 1), (1024, 1024, 2, 1, 1)),
    ((5120, 5120, 4, 0, 5), (2048, 1024, 3, 0, 2)),
    ((2048, 2048, 2.5, 2, 1), (512, 512, 2.5, 2, 1)),
    ((1024, 1024, 4, 0, 40), (512, 768, 4, 0, 20)),
    ((4096, 4096, 4, 0, 96), (1024, 1024, 4, 0, 40)),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_gemm(torch_cuda, orc, first, second):
    torch = torch_cuda
    for i, (k, n, K, cb, m) in enumerate((first, second)):
        L = synth.layer(k, n, K, cb, seed=7000 + 13 * i + k + n)
        x = synth.activations(m, k, seed=7001 + i)
        rc0, y0 = call(torch, "exl3_amd_gemm", L, x)
        rc1, y1 = call(torch, "exl3_amd_gemm_noalloc", L, x)
        assert rc0 == rc1 and rc1 in (90, 91), (rc0, rc1)
        assert_close(y1, y0, what=f"call {i}: noalloc vs gemm")
        ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)
        assert_close(y1, ref, what=f"call {i}: noalloc vs fp64")


def test_noalloc_rejects_oversized(torch_cuda):
    """8 rows of a 14336 -> 65536 matrix need more split partials than the scratch holds."""
    torch = torch_cuda
    from ampstein_amd import _lib
    k, n, m = 14336, 65536, 8
    t = torch.zeros((k // 16, n // 16, 64), dtype=torch.int16, device="cuda")
    s = torch.ones(k, dtype=torch.half, device="cuda")
    v = torch.ones(n, dtype=torch.half, device="cuda")
    A = torch.zeros((m, k), dtype=torch.half, device="cuda")
    C = torch.empty((m, n), dtype=torch.half, device="cuda")
    lib = _lib.lib()
    rc = lib.exl3_amd_gemm_noalloc(A.data_ptr(), t.data_ptr(), C.data_ptr(), 0, s.data_ptr(), None, v.data_ptr(),
                                   m, k, n, 4.0, 0, 0, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.EUNSUPPORTED, rc
    assert b"scratch" in lib.exl3_amd_last_error() or b"workspace" in lib.exl3_amd_last_error()
