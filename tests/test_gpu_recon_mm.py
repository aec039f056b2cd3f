"""The recon route's hand-written dense GEMM (exl3_amd_recon_mm, exl3_dense.hip) and the
transposed original-basis reconstruct (exl3_amd_reconstruct_had_t) through the C ABI.

recon_mm is a floating-point kernel: it is checked against a plain PyTorch fp32 matmul of the same
fp16 operands (and the output rotation against the fp64 Hadamard), bar max |y - ref| / max |ref|
< 2e-3 (fp16 output) or 1e-5 (fp32 output, only the summation order differs).
reconstruct_had_t must equal reconstruct_had transposed, bit for bit.
"""
import numpy as np
import pytest
from scipy.linalg import hadamard

from ampstein_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ampstein_amd import ops
    ops.init(0)
    return torch


def rel(y, ref):
    y = np.asarray(y, np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("m,k,n", [(1, 128, 128), (37, 256, 384), (256, 1024, 1024), (300, 512, 640),
                                   (513, 2048, 256), (1024, 96, 2048)])
@pytest.mark.parametrize("out", ["fp16", "fp32"])
@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("variant", [0, 1, 3], ids=["4waves", "8waves", "4waves-global-dma"])
def test_recon_mm_matches_torch_fp32(torch_cuda, kernel_policy, m, k, n, out, rot, variant):
    torch = torch_cuda
    from ampstein_amd import ops, _lib
    kernel_policy(_lib.POLICY_RECON_MM, variant)
    g = torch.Generator(device="cuda")
    g.manual_seed(m * 7 + k + n)
    a = torch.randn((m, k), generator=g, device="cuda").half()
    wt = (torch.randn((n, k), generator=g, device="cuda") * 0.05).half()
    svh = (torch.randint(0, 2, (n,), generator=g, device="cuda") * 2 - 1).half() if rot else None
    c = torch.full((m, n), float("nan"), dtype=torch.half if out == "fp16" else torch.float, device="cuda")
    ops.recon_mm(a, wt, c, svh)
    ref = (a.float() @ wt.float().t()).double().cpu().numpy()
    if rot:
        H = hadamard(128) / np.sqrt(128.0)
        ref = (ref.reshape(m, n // 128, 128) @ H).reshape(m, n) * svh.double().cpu().numpy()
    y = c.float().cpu().numpy()
    assert np.isfinite(y).all()
    assert rel(y, ref) < (2e-3 if out == "fp16" else 1e-5), (m, k, n, out, rot)


def half_tile_cases(cus):
    """(m, k, n) whose 256 x 256 tiles leave a last round at most half full, so that the four-wave
    form runs the remaining column blocks as 256 x 128 half tiles: one row block with cus + 44
    column blocks, two row blocks (partial rows) with cus / 2 + 2, and the 8192 -> 28672 prefill
    shape (configs[3], 896 tiles)."""
    return [(256, 64, 256 * (cus + 44)), (300, 96, 256 * (cus // 2 + 2)), (2048, 8192, 28672)]


@pytest.mark.parametrize("case", [0, 1, 2])
@pytest.mark.parametrize("rot", [False, True])
def test_recon_mm_half_tiles(torch_cuda, kernel_policy, case, rot):
    """The grid with half tiles in its last round against the same GEMM with whole tiles only
    (policy EXL3_AMD_RECON_MM_WHOLE_TILES) and against torch's fp32 matmul, bar 2e-3 (fp16 out)."""
    torch = torch_cuda
    from ampstein_amd import ops, _lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    m, k, n = half_tile_cases(cus)[case]
    nmb, nbn = (m + 255) // 256, n // 256
    rem = nbn * nmb % cus
    assert nbn * nmb > cus and 0 < 2 * rem <= cus and rem % nmb == 0     # the half-tile grid applies
    g = torch.Generator(device="cuda")
    g.manual_seed(m + k + n + case)
    a = torch.randn((m, k), generator=g, device="cuda").half()
    wt = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
    svh = (torch.randint(0, 2, (n,), generator=g, device="cuda") * 2 - 1).half() if rot else None
    outs = []
    for variant in (0, _lib.RECON_MM_WHOLE_TILES, _lib.RECON_MM_GLOBAL_DMA):
        kernel_policy(_lib.POLICY_RECON_MM, variant)
        c = torch.full((m, n), float("nan"), dtype=torch.half, device="cuda")
        ops.recon_mm(a, wt, c, svh)
        torch.cuda.synchronize()
        outs.append(c)
    # the same tile arithmetic every way (one k order per output): bit-identical
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = a.float() @ wt.float().t()
    if rot:
        H = torch.from_numpy(hadamard(128) / np.sqrt(128.0)).float().cuda()
        ref = (ref.view(m, n // 128, 128) @ H).view(m, n) * svh.float()
    y = outs[0].float()
    assert torch.isfinite(y).all()
    err = float((y - ref).abs().max() / ref.abs().max())
    assert err < 2e-3, (m, k, n, rot, err)


@pytest.mark.parametrize("m,k,n", [(16, 4096, 4096), (64, 14336, 4096), (300, 2048, 1152), (2048, 14336, 4096)])
@pytest.mark.parametrize("out", ["fp16", "fp32"])
@pytest.mark.parametrize("rot", [False, True])
def test_recon_mm_split_k(torch_cuda, kernel_policy, m, k, n, out, rot):
    """Launches whose 256 x 256 tiles fill at most half the CUs split k (partial tiles in the
    library workspace, summed in k order by the fixup kernel, which also rotates and stores):
    against the same GEMM without the split (policy EXL3_AMD_RECON_MM_NO_SPLIT) and against
    torch's fp32 matmul, bar 2e-3 (fp16 out) or 1e-5 (fp32 out); n = 1152 ends on a half column
    block.  Slab operands give the split's result bit for bit."""
    torch = torch_cuda
    from ampstein_amd import ops, _lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = ((m + 255) // 256) * ((n + 255) // 256)
    assert 2 * tiles <= cus                                                  # the split applies
    g = torch.Generator(device="cuda")
    g.manual_seed(m + k + n + 5)
    a = torch.randn((m, k), generator=g, device="cuda").half()
    wt = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
    svh = (torch.randint(0, 2, (n,), generator=g, device="cuda") * 2 - 1).half() if rot else None
    dt = torch.half if out == "fp16" else torch.float
    ref = a.float() @ wt.float().t()
    if rot:
        H = torch.from_numpy(hadamard(128) / np.sqrt(128.0)).float().cuda()
        ref = (ref.view(m, n // 128, 128) @ H).view(m, n) * svh.float()
    ys = {}
    for variant in (0, _lib.RECON_MM_NO_SPLIT):
        kernel_policy(_lib.POLICY_RECON_MM, variant)
        c = torch.full((m, n), float("nan"), dtype=dt, device="cuda")
        ops.recon_mm(a, wt, c, svh)
        torch.cuda.synchronize()
        y = c.float()
        assert torch.isfinite(y).all()
        err = float((y - ref).abs().max() / ref.abs().max())
        assert err < (2e-3 if out == "fp16" else 1e-5), (m, k, n, out, rot, variant, err)
        ys[variant] = c
    kernel_policy(_lib.POLICY_RECON_MM, 0)
    c = torch.full((m, n), float("nan"), dtype=dt, device="cuda")
    ops.recon_mm(ops.slabs_of(a), ops.slabs_of(wt), c, svh)
    torch.cuda.synchronize()
    assert torch.equal(c, ys[0])


def test_recon_mm_rejects(torch_cuda):
    torch = torch_cuda
    from ampstein_amd import _lib
    lib = _lib.lib()
    a = torch.zeros((4, 64), dtype=torch.half, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert lib.exl3_amd_recon_mm(a.data_ptr(), a.data_ptr(), a.data_ptr(), 0, None, 4, 48, 128, st) == _lib.EINVAL
    assert lib.exl3_amd_recon_mm(a.data_ptr(), a.data_ptr(), a.data_ptr(), 0, None, 4, 64, 100, st) == _lib.EINVAL
    assert lib.exl3_amd_recon_mm(None, a.data_ptr(), a.data_ptr(), 0, None, 4, 64, 128, st) == _lib.EINVAL
    assert lib.exl3_amd_recon_mm(None, None, None, 0, None, 0, 64, 128, st) == 0      # empty: nothing to do


@pytest.mark.parametrize("K,cb", [(4, 0), (3, 1), (2, 2), (2.5, 2), (8, 0)])
def test_reconstruct_had_t_bit_exact(torch_cuda, orc, K, cb):
    torch = torch_cuda
    from ampstein_amd import ops
    k, n = 256, 384
    L = synth.layer(k, n, K, cb, seed=5100 + int(10 * K) + cb)
    t, s, v = L.torch()
    w = torch.empty((k, n), dtype=torch.half, device="cuda")
    wt = torch.empty((n, k), dtype=torch.half, device="cuda")
    ops.reconstruct_had_slice(w, t, s, v, K, cb == 1, cb == 2, 0)
    ops.reconstruct_had_t(wt, t, s, v, K, cb == 1, cb == 2, 0)
    W = w.cpu().numpy().view(np.uint16)
    assert np.array_equal(wt.cpu().numpy().view(np.uint16), W.T)
    ref = orc.reconstruct_had(L.trellis, L.suh, L.svh, int(K), half=K != int(K), cb=cb)
    assert np.array_equal(W, ref.view(np.uint16))


@pytest.mark.parametrize("branch", ["rotated", "fused_w"])
def test_recon_hip_matches_library(torch_cuda, orc, branch):
    """exl3_gemm_recon on this build's GEMM and on the vendor library (the comparison path):
    both within 2e-3 of the fp64 linear on the same reconstructed weights, 2048 rows."""
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(1024, 768, 4, 0, seed=5200)
    x = synth.activations(2048, 1024, seed=5201)
    t, s, v = L.torch()
    xd = torch.from_numpy(x).cuda()
    fr = 2048 if branch == "fused_w" else 1 << 30
    yh = ops.exl3_gemm_recon(xd, t, s, v, 4.0, fused_rows=fr).float().cpu().numpy()
    yl = ops.exl3_gemm_recon(xd, t, s, v, 4.0, fused_rows=fr, gemm="library").float().cpu().numpy()
    if branch == "fused_w":
        W = orc.reconstruct_had(L.trellis, L.suh, L.svh, 4).astype(np.float64)
        ref = x.astype(np.float64) @ W
    else:
        ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, 4)
    assert rel(yh, ref) < 2e-3
    assert rel(yl, ref) < 2e-3


# ------------------------------------------------------------------ k-slab operand layout
@pytest.mark.parametrize("m,k,n", [(37, 96, 384), (300, 512, 640), (513, 256, 1024), (2048, 1024, 768)])
@pytest.mark.parametrize("variant", [0, 1, 3], ids=["4waves", "8waves", "4waves-global-dma"])
def test_recon_mm_slabs_bit_identical(torch_cuda, kernel_policy, m, k, n, variant):
    """recon_mm on A and / or WT in the k-slab layout equals recon_mm on the row-major operands
    bit for bit (same tiles, same k order), fp16 and fp32 output, with and without svh."""
    torch = torch_cuda
    from ampstein_amd import ops, _lib
    kernel_policy(_lib.POLICY_RECON_MM, variant)
    g = torch.Generator(device="cuda")
    g.manual_seed(m + 3 * k + n)
    a = torch.randn((m, k), generator=g, device="cuda").half()
    wt = (torch.randn((n, k), generator=g, device="cuda") * 0.05).half()
    svh = (torch.randint(0, 2, (n,), generator=g, device="cuda") * 2 - 1).half()
    a_s, wt_s = ops.slabs_of(a), ops.slabs_of(wt)
    for dt in (torch.half, torch.float):
        for sv in (None, svh):
            ref = torch.full((m, n), float("nan"), dtype=dt, device="cuda")
            ops.recon_mm(a, wt, ref, sv)
            for aa, ww in ((a_s, wt), (a, wt_s), (a_s, wt_s)):
                c = torch.full((m, n), float("nan"), dtype=dt, device="cuda")
                ops.recon_mm(aa, ww, c, sv)
                torch.cuda.synchronize()
                assert torch.equal(c, ref), (m, k, n, dt, sv is None, aa.dim(), ww.dim())


def test_recon_mm_slabs_half_tiles(torch_cuda):
    """The half-tile grid (8192 -> 28672 at 2048 rows) on slab operands: bit-identical to the
    row-major call."""
    torch = torch_cuda
    from ampstein_amd import ops
    m, k, n = 2048, 8192, 28672
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    a = torch.randn((m, k), generator=g, device="cuda").half()
    wt = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
    ref = torch.empty((m, n), dtype=torch.half, device="cuda")
    ops.recon_mm(a, wt, ref)
    c = torch.full((m, n), float("nan"), dtype=torch.half, device="cuda")
    ops.recon_mm(ops.slabs_of(a), ops.slabs_of(wt), c)
    torch.cuda.synchronize()
    assert torch.equal(c, ref)


@pytest.mark.parametrize("K,cb", [(4, 0), (3, 1), (2.5, 2), (8, 0)])
@pytest.mark.parametrize("original", [False, True])
def test_reconstruct_t_slabs_bit_exact(torch_cuda, K, cb, original):
    """reconstruct_t_slabs equals the row-major reconstruct_t / reconstruct_had_t laid out in k
    slabs, bit for bit, on a column slice (n_offset 128) of a wider packed tensor."""
    torch = torch_cuda
    from ampstein_amd import ops
    k, n_packed, n, off = 384, 512, 256, 128
    L = synth.layer(k, n_packed, K, cb, seed=5300 + int(10 * K) + cb + 7 * original)
    t, s, v = L.torch()
    ref = torch.empty((n, k), dtype=torch.half, device="cuda")
    if original:
        ops.reconstruct_had_t(ref, t, s, v, K, cb == 1, cb == 2, off)
    else:
        ops.reconstruct_t(ref, t, K, cb == 1, cb == 2, off)
    ws = torch.full((k // 32, n, 32), float("nan"), dtype=torch.half, device="cuda")
    ops.reconstruct_t_slabs(ws, t, K, cb == 1, cb == 2, s if original else None, v if original else None, off)
    torch.cuda.synchronize()
    assert torch.equal(ws.view(torch.int16), ops.slabs_of(ref).view(torch.int16))


@pytest.mark.parametrize("rows,cols", [(1, 128), (37, 384), (2048, 1024), (5, 96), (300, 160)])
def test_to_slabs(torch_cuda, rows, cols):
    """to_slabs: the copy is exact (any multiple of 32 columns); the rotation (multiples of 128)
    equals had_r_128 (pre scale) laid out in slabs."""
    torch = torch_cuda
    from ampstein_amd import ops
    g = torch.Generator(device="cuda")
    g.manual_seed(rows + cols)
    x = torch.randn((rows, cols), generator=g, device="cuda").half()
    pre = (torch.randint(0, 2, (cols,), generator=g, device="cuda") * 2 - 1).half()
    y = torch.full((cols // 32, rows, 32), float("nan"), dtype=torch.half, device="cuda")
    ops.to_slabs(x, y)
    torch.cuda.synchronize()
    assert torch.equal(y, ops.slabs_of(x))
    if cols % 128:
        return
    h = torch.empty_like(x)
    ops.had_r_128(x, h, pre, None, 1.0)
    ops.to_slabs(x, y, True, pre, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), ops.slabs_of(h).view(torch.int16))


@pytest.mark.parametrize("branch", ["rotated", "fused_w"])
@pytest.mark.parametrize("n", [768, 16384])
def test_recon_slabs_route_bit_identical(torch_cuda, orc, branch, n):
    """exl3_gemm_recon with slab operands (the default; n = 16384: the fused branch copies x into
    slabs) equals the row-major route bit for bit, and the fp64 linear within 2e-3."""
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(1024, n, 4, 0, seed=5400 + n)
    x = synth.activations(300, 1024, seed=5401)
    t, s, v = L.torch()
    xd = torch.from_numpy(x).cuda()
    fr = 1 if branch == "fused_w" else 1 << 30
    ys = ops.exl3_gemm_recon(xd, t, s, v, 4.0, fused_rows=fr)
    yr = ops.exl3_gemm_recon(xd, t, s, v, 4.0, fused_rows=fr, slabs=False)
    torch.cuda.synchronize()
    assert torch.equal(ys, yr)
    if branch == "fused_w":
        W = orc.reconstruct_had(L.trellis, L.suh, L.svh, 4).astype(np.float64)
        ref = x.astype(np.float64) @ W
    else:
        ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, 4)
    assert rel(ys.float().cpu().numpy(), ref) < 2e-3


def test_slab_entry_points_reject(torch_cuda):
    torch = torch_cuda
    from ampstein_amd import _lib
    lib = _lib.lib()
    a = torch.zeros((4, 256), dtype=torch.half, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    p = a.data_ptr()
    assert lib.exl3_amd_recon_mm_slabs(p, p, p, 0, None, 4, 48, 128, 1, 1, 128, st) == _lib.EINVAL     # k % 32
    assert lib.exl3_amd_recon_mm_slabs(p, p, p, 0, None, 4, 64, 128, 1, 1, 120, st) == _lib.EINVAL     # ldc < n
    assert lib.exl3_amd_recon_mm_slabs(p, p, p, 0, None, 4, 64, 128, 1, 1, 132, st) == _lib.EINVAL     # ldc % 8
    assert lib.exl3_amd_to_slabs(p, p, 4, 256, 0, None, 1.0, st) == _lib.EINVAL                    # in place
    assert lib.exl3_amd_to_slabs(p, p + 4096, 4, 96, 1, None, 1.0, st) == _lib.EINVAL              # rotation: cols % 128
    assert lib.exl3_amd_to_slabs(p, p + 4096, 4, 48, 0, None, 1.0, st) == _lib.EINVAL              # copy: cols % 32
    assert lib.exl3_amd_to_slabs(p, p + 4096, 4, 256, 0, p, 1.0, st) == _lib.EINVAL                # pre without rotation
    assert lib.exl3_amd_reconstruct_t_slabs(p, p, None, None, 48, 128, 128, 0, 4.0, 0, 0, 0, st) == _lib.EINVAL   # k % 32
