"""GPU parity of the MFMA prefill GEMM (exl3_amd_gemm with m > 8, exl3_gemm_kernel semantics:
the output Hadamard reads fp32 sums) against the CPU oracle's fp64 linear.

Bar: max|y - ref| / max|ref| < 2e-3.  Covers every K and codebook, ragged row counts (row
blocks of 256 with a partial last block), column-chunk counts that do and do not take the
XCD-grouped tile order, fp16 / fp32 outputs, and the optional rotations.  A_had must hold the
rotated input afterwards, bit-exact with had_r_128(A, pre=suh).
"""
import numpy as np
import pytest

from ampstein_amd import _lib, synth

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


def run_gemm(torch, L, x, y_fp32, suh=True, svh=True, force=2):
    """force 2 (default here): the MFMA GEMM whatever m; 0: the library's routing."""
    from ampstein_amd import ops
    t, s, v = L.torch()
    A = torch.from_numpy(x).cuda()
    A_had = torch.empty_like(A)
    C = torch.empty((x.shape[0], L.n), dtype=torch.float if y_fp32 else torch.half, device="cuda")
    tag = ops.exl3_gemm(A, t, C, s if suh else None, A_had, v if svh else None, force, L.cb == 1, L.cb == 2)
    return tag, C.cpu().numpy(), A_had.cpu().numpy()


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("K", list(range(1, 9)))
def test_gemm_parity_all_bitrates(torch_cuda, orc, K, cb):
    torch = torch_cuda
    L = synth.layer(256, 256, K, cb, seed=500 + 10 * K + cb)
    x = synth.activations(40, 256, seed=K + 3 * cb)
    tag, y, _ = run_gemm(torch, L, x, False)
    assert tag == 91
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, K, cb=cb)
    assert rel_err(y, ref) < TOL


@pytest.mark.parametrize("K,cb,m,k,n", [(4, 0, 300, 512, 2048), (2, 1, 513, 1024, 384), (8, 2, 256, 256, 1024),
                                         (2.5, 2, 40, 384, 256), (3, 0, 9, 128, 128)])
def test_gemm_dma_and_register_staging(torch_cuda, orc, kernel_policy, K, cb, m, k, n):
    """The LDS-DMA kernel (without the split k: policy EXL3_AMD_GEMM_STAGING_NO_SPLIT) and the
    register-staged kernel (EXL3_AMD_GEMM_STAGING_REGS) do the same arithmetic in the same order:
    bit-identical outputs.  The default (LDS DMA, k split where the tiles fill at most half the
    CUs: partial tiles summed in k order by the fixup kernel) and both forms within the bar."""
    torch = torch_cuda
    L = synth.layer(k, n, K, cb, seed=900 + int(10 * K) + cb)
    x = synth.activations(m, k, seed=901 + int(10 * K))
    ys = []
    for staging in (_lib.GEMM_STAGING_NO_SPLIT, _lib.GEMM_STAGING_REGS, 0):
        kernel_policy(_lib.POLICY_GEMM_STAGING, staging)
        tag, y, _ = run_gemm(torch, L, x, False)
        assert tag == 91
        ys.append(y)
    assert np.array_equal(ys[0].view(np.uint16), ys[1].view(np.uint16))
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)
    assert rel_err(ys[0], ref) < TOL
    assert rel_err(ys[2], ref) < TOL


@pytest.mark.parametrize("K,cb,m,k,n", [(4, 0, 64, 14336, 4096), (3, 1, 200, 4096, 4096), (2.5, 2, 33, 2048, 1152),
                                         (8, 0, 256, 4096, 8192), (4, 2, 17, 512, 256)])
@pytest.mark.parametrize("y_fp32", [False, True])
def test_gemm_split_k(torch_cuda, orc, kernel_policy, K, cb, m, k, n, y_fp32):
    """The fused GEMM with its k split in S ranges per tile (force_shape_idx 2 keeps the tiled GEMM;
    tiles filling at most half the CUs split; n = 1152 ends on a half column block, 512 x 256 has
    too few stages to split): within the bar of the fp64 linear, as the unsplit kernel."""
    torch = torch_cuda
    L = synth.layer(k, n, K, cb, seed=950 + m + int(10 * K) + cb)
    x = synth.activations(m, k, seed=951 + m)
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)
    for staging in (0, _lib.GEMM_STAGING_NO_SPLIT):
        kernel_policy(_lib.POLICY_GEMM_STAGING, staging)
        tag, y, _ = run_gemm(torch, L, x, y_fp32, force=2)
        assert tag == 91
        assert rel_err(y, ref) < TOL, (staging, m, k, n)


@pytest.mark.parametrize("m,k,n", [(9, 128, 128), (256, 512, 1024), (300, 256, 384), (513, 1024, 1024)])
@pytest.mark.parametrize("y_fp32", [False, True])
def test_gemm_shapes(torch_cuda, orc, m, k, n, y_fp32):
    torch = torch_cuda
    L = synth.layer(k, n, 4, 0, seed=600 + m + k + n)
    x = synth.activations(m, k, seed=m)
    tag, y, A_had = run_gemm(torch, L, x, y_fp32)
    assert tag == 91
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, 4, cb=0)
    assert rel_err(y, ref) < TOL
    assert np.array_equal(A_had.view(np.uint16), orc.had128(x, pre=L.suh).view(np.uint16))


@pytest.mark.parametrize("m,k,n,K,cb,route", [(9, 5120, 17408, 2, 0, 90), (16, 17408, 5120, 4, 1, 90),
                                                (33, 4096, 14336, 3, 2, 91), (64, 5120, 5120, 2.5, 2, 91),
                                                (100, 4096, 1024, 4, 0, 91)])
def test_gemm_medium_batch_routing(torch_cuda, orc, m, k, n, K, cb, route):
    """m > 8 with few 256-row tiles per CU: one or two 16-row groups of the matrix-core GEMV (tag
    90) against the MFMA GEMM with its k split (tag 91, from ~32 rows), by the library's time
    model; the rotated input written into A_had either way; the call forced onto the MFMA GEMM
    agrees."""
    torch = torch_cuda
    L = synth.layer(k, n, K, cb, seed=650 + m + n)
    x = synth.activations(m, k, seed=651 + m)
    tag, y, A_had = run_gemm(torch, L, x, False, force=0)
    assert tag == route
    assert np.array_equal(A_had.view(np.uint16), orc.had128(x, pre=L.suh).view(np.uint16))
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)
    assert rel_err(y, ref) < TOL
    tag2, y2, _ = run_gemm(torch, L, x, False, force=2)
    assert tag2 == 91
    assert rel_err(y2, ref) < TOL


@pytest.mark.parametrize("suh,svh", [(False, False), (True, False), (False, True)])
def test_gemm_optional_rotations(torch_cuda, orc, suh, svh):
    torch = torch_cuda
    L = synth.layer(256, 256, 3, 1, seed=77)
    x = synth.activations(64, 256, seed=77)
    _, y, _ = run_gemm(torch, L, x, True, suh, svh)
    ref = orc.linear(x, L.trellis, L.suh if suh else None, L.svh if svh else None, 3, cb=1, y_fp32=True)
    assert rel_err(y, ref) < TOL


def test_gemm_forced_kernel_and_rows(torch_cuda, orc):
    """force_shape_idx 2 runs the MFMA kernel for m <= 8; 1 forces the GEMV for any row count."""
    torch = torch_cuda
    from ampstein_amd import ops, _lib
    L = synth.layer(256, 128, 4, 0, seed=88)
    x = synth.activations(5, 256, seed=88)
    t, s, v = L.torch()
    A = torch.from_numpy(x).cuda()
    C = torch.empty((5, 128), dtype=torch.float, device="cuda")
    assert ops.exl3_gemm(A, t, C, s, torch.empty_like(A), v, 2) == 91
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, 4, cb=0)
    assert rel_err(C.cpu().numpy(), ref) < TOL
    x9 = synth.activations(9, 256, seed=89)
    A9 = torch.from_numpy(x9).cuda()
    C9 = torch.empty((9, 128), dtype=torch.float, device="cuda")
    assert ops.exl3_gemm(A9, t, C9, s, torch.empty_like(A9), v, 1) == 90
    assert rel_err(C9.cpu().numpy(), orc.linear_f64(x9, L.trellis, L.suh, L.svh, 4, cb=0)) < TOL
    with pytest.raises(_lib.Exl3Error, match="A_had"):
        ops.exl3_gemm(A9, t, torch.empty((9, 128), dtype=torch.half, device="cuda"), s, None, v)


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("K", list(range(1, 9)))
def test_reconstruct_t_bit_exact(torch_cuda, orc, K, cb):
    """The transposed reconstruct (recon GEMM layout): WT == oracle W_hat transposed, bit for bit."""
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(256, 384, K, cb, seed=700 + 10 * K + cb)
    t, _, _ = L.torch()
    WT = torch.empty((384, 256), dtype=torch.half, device="cuda")
    ops.reconstruct_t(WT, t, K, cb == 1, cb == 2)
    ref = orc.reconstruct(L.trellis, K, cb=cb)
    assert np.array_equal(WT.cpu().numpy().view(np.uint16), np.ascontiguousarray(ref.T).view(np.uint16))
    # a column block (the recon pipeline's unit): columns [128, 384) into rows 0..255
    WB = torch.empty((256, 256), dtype=torch.half, device="cuda")
    ops.reconstruct_t(WB, t, K, cb == 1, cb == 2, n_offset=128)
    assert np.array_equal(WB.cpu().numpy().view(np.uint16), np.ascontiguousarray(ref[:, 128:].T).view(np.uint16))


@pytest.mark.parametrize("branch", ["rotated", "fused_w"])
@pytest.mark.parametrize("K,cb", [(4, 0), (3, 1), (2, 2)])
def test_gemm_recon(torch_cuda, orc, branch, K, cb):
    """exl3_gemm_recon (amp_torch.cpp:11149-11230): both branches of the reference's row policy,
    dense GEMM on hipBLASLt, within 2e-3 of the fp64 linear."""
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(512, 384, K, cb, seed=800 + K)
    x = synth.activations(300, 512, seed=K)
    t, s, v = L.torch()
    y = ops.exl3_gemm_recon(torch.from_numpy(x).cuda(), t, s, v, float(K), mul1=cb == 2, mcg=cb == 1,
                            fused_rows=0 if branch == "fused_w" else 1 << 30)
    torch.cuda.synchronize()
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, K, cb=cb)
    assert rel_err(y.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("K,cb", [(4, 0), (3, 1), (2, 2), (2.5, 2), (8, 0)])
def test_reconstruct_t_had(orc, K, cb):
    """W' = W_hat H128 diag(svh) / sqrt(128), transposed: within one fp16 ulp of the fp64 product
    of the oracle's bit-exact W_hat (fp32 butterflies, one rounding), and the recon GEMM's rotated
    branch with the fold against fp64 within 2e-3."""
    import torch
    from ampstein_amd import ops
    from scipy.linalg import hadamard
    k, n = 256, 384
    L = synth.layer(k, n, K, cb, seed=int(K * 10) + cb)
    t, s, v = L.torch("cuda")
    wt = torch.empty((n, k), dtype=torch.half, device="cuda")
    ops.reconstruct_t(wt, t, K, cb == 1, cb == 2, svh=v)
    W = orc.reconstruct(L.trellis, int(K), half=K != int(K), cb=cb).astype(np.float64)
    H = hadamard(128) / np.sqrt(128.0)
    ref = (W.reshape(k, n // 128, 128) @ H).reshape(k, n) * L.svh.astype(np.float64)
    got = wt.cpu().numpy().T.astype(np.float64)
    ulp = np.abs(ref).clip(min=2.0 ** -14) * 2.0 ** -10
    assert np.all(np.abs(got - ref) <= ulp + 1e-12)
    x = synth.activations(300, k, seed=1)
    xd = torch.from_numpy(x).cuda()
    xh = torch.empty_like(xd)
    ops.had_r_128(xd, xh, s, None, 1.0)
    y = torch.empty((300, n), dtype=torch.half, device="cuda")
    ops.recon_mm(xh, wt, y)                                  # the folded weight: no output rotation left
    yr = orc.linear(x, L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb, y_fp32=True).astype(np.float64)
    assert np.abs(y.float().cpu().numpy() - yr).max() / np.abs(yr).max() < 2e-3
