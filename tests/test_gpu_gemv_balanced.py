"""The balanced single-row GEMV (exl3_gemv.hip gemv1b_kernel: every wave streams the same number
of k-slices, every SIMD holds the same number of waves) against the fp64 linear of the oracle,
on shapes whose slice count splits evenly over the device's SIMDs (the Llama-3-8B gate / up,
down and q / o shapes), alone and as the stacked gate / up exl3_mgemm; selected by the policy
EXL3_AMD_GEMV_SPLIT_BALANCED; and the default per-chunk split on the same inputs.  Bar: 2e-3 (tests/tol.py)."""
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


@pytest.mark.parametrize("k,n", [(4096, 14336), (14336, 4096), (4096, 4096)])
@pytest.mark.parametrize("K,cb", [(4, 0), (2, 0), (3, 1), (8, 0)])
@pytest.mark.parametrize("split", ["balanced", "per_chunk"])
def test_gemv_m1_balanced(torch_cuda, orc, kernel_policy, k, n, K, cb, split):
    torch = torch_cuda
    from ampstein_amd import ops
    if split == "balanced":
        kernel_policy(_lib.POLICY_GEMV_SPLIT, _lib.GEMV_SPLIT_BALANCED)
    L = synth.layer(k, n, K, cb, seed=9300 + k // 1024 + n // 1024 + K)
    x = synth.activations(1, k, seed=9301)
    t, s, v = L.torch()
    A = torch.from_numpy(x).cuda()
    for rep in range(2):                      # the second call runs on re-armed counters
        C = torch.full((1, n), float("nan"), dtype=torch.half, device="cuda")
        assert ops.exl3_gemm(A, t, C, s, torch.empty_like(A), v, 0, cb == 1, cb == 2) == 90
        torch.cuda.synchronize()
        y = C.cpu().numpy()
        assert np.isfinite(y.astype(np.float32)).all()
        assert_close(y, orc.linear_f64(x, L.trellis, L.suh, L.svh, K, cb=cb), what=f"{k}x{n} K{K} cb{cb} rep{rep}")


@pytest.mark.parametrize("split", ["balanced", "per_chunk"])
def test_gate_up_stacked_balanced(torch_cuda, orc, kernel_policy, split):
    torch = torch_cuda
    from ampstein_amd import ops
    if split == "balanced":
        kernel_policy(_lib.POLICY_GEMV_SPLIT, _lib.GEMV_SPLIT_BALANCED)
    layers = [synth.layer(4096, 14336, 4, 0, seed=9400 + i) for i in range(2)]
    dev = [L.torch() for L in layers]
    P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
    B, suh, svh = (P([d[i].data_ptr() for d in dev]) for i in range(3))
    x = synth.activations(1, 4096, seed=9401)
    A = torch.from_numpy(x).cuda().unsqueeze(0)
    C = torch.full((2, 1, 14336), float("nan"), dtype=torch.half, device="cuda")
    A_had = torch.empty((2, 1, 4096), dtype=torch.half, device="cuda")
    assert ops.exl3_mgemm(A, B, C, suh, A_had, svh, None, None, 4) == 90
    torch.cuda.synchronize()
    y = C.cpu().numpy()
    for q, L in enumerate(layers):
        assert_close(y[q], orc.linear_f64(x, L.trellis, L.suh, L.svh, 4), what=f"slab {q}")
