"""GPU parity of the multi-matrix GEMV (exl3_amd_mgemm through the C ABI) against the CPU
oracle, one oracle linear per selected matrix.

Covers the modes of exl3_mgemm (quant/exl3_gemm.cu:352-394): stacked bundle (broadcast input,
as the decode step's gate/up), sliced bundle (q/k/v column slices with per-source suh, strided
outputs), indexed selection with skipped slots, per-matrix widths, routing-weighted reduction
over token groups, and expert-range filtering.  Widths of 1024 columns (8 chunks) take the
XCD-local hand-off; 384 columns (3 chunks) the finish-kernel path.  Bar: max|y - ref| /
max|ref| < 2e-3 per output slab.
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


class Bundle:
    """Synthetic matrices on the GPU with their pointer tables."""

    def __init__(self, torch, k, widths, K, cb, seed):
        self.layers = [synth.layer(k, n, K, cb, seed=seed + i) for i, n in enumerate(widths)]
        self.dev = [L.torch() for L in self.layers]
        self.K, self.cb, self.k = K, cb, k
        ptr = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
        self.B = ptr([t.data_ptr() for t, _, _ in self.dev])
        self.suh = ptr([s.data_ptr() for _, s, _ in self.dev])
        self.svh = ptr([v.data_ptr() for _, _, v in self.dev])

    def ref(self, orc, q, x, y_fp32):
        L = self.layers[q]
        return orc.linear(x, L.trellis, L.suh, L.svh, self.K, cb=self.cb, y_fp32=y_fp32)


def cuda_x(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("n", [1024, 384])
@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("y_fp32", [False, True])
@pytest.mark.parametrize("K,cb", [(4, 0), (2, 1), (3, 2), (6, 0)])
def test_mgemm_stacked(torch_cuda, orc, n, m, y_fp32, K, cb):
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 512, [n, n, n], K, cb, seed=50 + K + 7 * cb)
    x = synth.activations(m, 512, seed=m)
    C = torch.empty((3, m, n), dtype=torch.float if y_fp32 else torch.half, device="cuda")
    A_had = torch.empty((3, m, 512), dtype=torch.half, device="cuda")
    out = ops.mgemm(cuda_x(torch, x[None]), bd.B, C, bd.suh, A_had, bd.svh, K, cb == 1, cb == 2)
    got = out.cpu().numpy()
    for q in range(3):
        assert rel_err(got[q], bd.ref(orc, q, x, y_fp32)) < TOL, q


@pytest.mark.parametrize("width", [256, 128])
@pytest.mark.parametrize("m", [1, 12])
def test_mgemm_sliced_qkv(torch_cuda, orc, width, m):
    """q 1024 / k 256 / v 256 cut into equal-width column slices (models.uc:367-430); 12 rows
    run as row groups of 8 and 4 with the slices' row stride."""
    torch = torch_cuda
    from ampstein_amd import ops
    widths = [1024, 256, 256]
    bd = Bundle(torch, 1024, widths, 4, 0, seed=70)
    x = synth.activations(m, 1024, seed=3)
    outs = [torch.full((m, w), float("nan"), dtype=torch.half, device="cuda") for w in widths]
    t_ptr, svh_ptr, c_ptr, strides, srcs = [], [], [], [], []
    for i, w in enumerate(widths):
        t, s, v = bd.dev[i]
        tw = t.size(2)
        for n0 in range(0, w, width):
            t_ptr.append(t.data_ptr() + (n0 // 16) * tw * 2)
            svh_ptr.append(v.data_ptr() + n0 * 2)
            c_ptr.append(outs[i].data_ptr() + n0 * 2)
            strides.append(w)
            srcs.append(i)
    ns = len(t_ptr)
    P = lambda v: torch.tensor(v, dtype=torch.long, device="cuda")
    I = lambda v: torch.tensor(v, dtype=torch.int32, device="cuda")
    carrier = torch.zeros((ns, m, width), dtype=torch.half, device="cuda")
    A_had = torch.zeros((3, m, 1024), dtype=torch.half, device="cuda")
    opts = {"size_n_list": I([width] * ns), "c_ptrs": P(c_ptr), "n_stride_list": I(strides),
            "had_src_list": I(srcs), "num_had_src": 3}
    ops.mgemm(cuda_x(torch, x[None]), P(t_ptr), carrier, bd.suh, A_had, P(svh_ptr), 4, False, False, opts)
    torch.cuda.synchronize()
    for i in range(3):
        assert rel_err(outs[i].cpu().numpy(), bd.ref(orc, i, x, False)) < TOL, i


@pytest.mark.parametrize("n", [1024, 384])
@pytest.mark.parametrize("m", [9, 20])
@pytest.mark.parametrize("slabs", [1, 3])
@pytest.mark.parametrize("y_fp32", [False, True])
def test_mgemm_many_rows(torch_cuda, orc, n, m, slabs, y_fp32):
    """More than 8 rows per matrix (batched decode): row groups of 8 over one broadcast input or
    one input slab per matrix, with an index that skips a slot."""
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 256, [n] * 3, 4, 0, seed=130 + n)
    xs = [synth.activations(m, 256, seed=m + 17 * i) for i in range(slabs)]
    A = cuda_x(torch, np.stack(xs))
    C = torch.full((3, m, n), 7.0, dtype=torch.float if y_fp32 else torch.half, device="cuda")
    idx = torch.tensor([[1, -1, 0]], dtype=torch.long, device="cuda")
    A_had = torch.empty((3, m, 256), dtype=torch.half, device="cuda")
    ops.exl3_mgemm(A, bd.B, C, bd.suh, A_had, bd.svh, idx, None, 4)
    torch.cuda.synchronize()
    got = C.cpu().numpy()
    assert rel_err(got[0], bd.ref(orc, 1, xs[0], y_fp32)) < TOL
    assert np.all(got[1] == 7.0)
    assert rel_err(got[2], bd.ref(orc, 0, xs[2 if slabs == 3 else 0], y_fp32)) < TOL


@pytest.mark.parametrize("n", [1024, 384])
def test_mgemm_indices_skip(torch_cuda, orc, n):
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 256, [n] * 4, 3, 0, seed=90)
    x = synth.activations(2, 256, seed=5)
    C = torch.full((3, 2, n), 7.0, dtype=torch.half, device="cuda")
    idx = torch.tensor([[2, -1, 0]], dtype=torch.long, device="cuda")
    A_had = torch.empty((3, 2, 256), dtype=torch.half, device="cuda")
    ops.exl3_mgemm(cuda_x(torch, x[None]), bd.B, C, bd.suh, A_had, bd.svh, idx, None, 3)
    got = C.cpu().numpy()
    assert rel_err(got[0], bd.ref(orc, 2, x, False)) < TOL
    assert np.all(got[1] == 7.0)                       # skipped slot left untouched
    assert rel_err(got[2], bd.ref(orc, 0, x, False)) < TOL


def test_mgemm_per_matrix_widths(torch_cuda, orc):
    torch = torch_cuda
    from ampstein_amd import ops
    widths = [1024, 256, 512]
    bd = Bundle(torch, 512, widths, 4, 1, seed=110)
    x = synth.activations(1, 512, seed=9)
    outs = [torch.empty((1, w), dtype=torch.float, device="cuda") for w in widths]
    C = torch.empty((3, 1, 1024), dtype=torch.float, device="cuda")
    A_had = torch.empty((3, 1, 512), dtype=torch.half, device="cuda")
    ops.exl3_mgemm(cuda_x(torch, x[None]), bd.B, C, bd.suh, A_had, bd.svh, None, None, 4, mcg=1,
                   size_n_list=torch.tensor(widths, dtype=torch.int32, device="cuda"),
                   c_ptrs=torch.tensor([o.data_ptr() for o in outs], dtype=torch.long, device="cuda"))
    for i in range(3):
        assert rel_err(outs[i].cpu().numpy(), bd.ref(orc, i, x, True)) < TOL, i


def weighted_ref(bd, orc, x_rows, sel, w, num_tokens, y_fp32):
    """Per-token sums of w_j * linear(x_j, B[sel_j]) over each group's slots (fp64)."""
    stride = len(sel) // num_tokens
    out = []
    for t in range(num_tokens):
        acc = 0.0
        for jj in range(stride):
            j = t * stride + jj
            if sel[j] < 0:
                continue
            acc = acc + np.float64(w[j]) * bd.ref(orc, sel[j], x_rows[j], True).astype(np.float64)
        out.append(acc)
    return out


@pytest.mark.parametrize("n", [1024, 384])
@pytest.mark.parametrize("y_fp32", [False, True])
@pytest.mark.parametrize("bszm_in", [1, 4])
def test_mgemm_weighted_tokens(torch_cuda, orc, n, y_fp32, bszm_in):
    """MoE-style fan-out: 2 tokens x 2 experts each, routing weights, one skipped selection."""
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 256, [n] * 6, 2, 2, seed=130)
    xs = synth.activations(bszm_in, 256, seed=11)
    sel = [4, 1, -1, 5]
    w = np.array([0.75, 0.25, 0.5, 0.625], np.float16)
    C = torch.full((4, 1, n), 3.0, dtype=torch.float if y_fp32 else torch.half, device="cuda")
    A = cuda_x(torch, xs[:, None, :])
    A_had = torch.empty((4, 1, 256), dtype=torch.half, device="cuda")
    idx = torch.tensor([sel], dtype=torch.long, device="cuda")
    wt = torch.from_numpy(w[None]).cuda()
    ops.exl3_mgemm(A, bd.B, C, bd.suh, A_had, bd.svh, idx, wt, 2, mul1=1, num_tokens=2)
    got = C.cpu().numpy()
    x_rows = [xs[j if bszm_in > 1 else 0][None] for j in range(4)]
    ref = weighted_ref(bd, orc, x_rows, sel, w.astype(np.float64), 2, y_fp32)
    for t in range(2):
        assert rel_err(got[t], ref[t]) < TOL, t


@pytest.mark.parametrize("m", [12, 20])
@pytest.mark.parametrize("num_tokens", [1, 2])
@pytest.mark.parametrize("y_fp32", [False, True])
def test_mgemm_weighted_many_rows(torch_cuda, orc, m, num_tokens, y_fp32):
    """Weighted reduction with more than 8 rows per slot: the rows run in groups (16 on the
    matrix-core GEMV) and each group reduces its own rows of every slot."""
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 256, [1024] * 6, 3, 2, seed=140)
    xs = synth.activations(4 * m, 256, seed=14).reshape(4, m, 256)
    sel = [4, 1, -1, 5]
    w = np.array([0.75, 0.25, 0.5, 0.625], np.float16)
    C = torch.full((4, m, 1024), 3.0, dtype=torch.float if y_fp32 else torch.half, device="cuda")
    A_had = torch.empty((4, m, 256), dtype=torch.half, device="cuda")
    idx = torch.tensor([sel], dtype=torch.long, device="cuda")
    wt = torch.from_numpy(w[None]).cuda()
    ops.exl3_mgemm(cuda_x(torch, xs), bd.B, C, bd.suh, A_had, bd.svh, idx, wt, 3, mul1=1, num_tokens=num_tokens)
    got = C.cpu().numpy()
    ref = weighted_ref(bd, orc, [xs[j] for j in range(4)], sel, w.astype(np.float64), num_tokens, y_fp32)
    for t in range(num_tokens):
        assert rel_err(got[t], ref[t]) < TOL, t


@pytest.mark.parametrize("num_tokens", [1, 2])
def test_mgemm_range_filter(torch_cuda, orc, num_tokens):
    """Expert-range filtering: selections outside [2, 6) dropped, kept ones rebased (the local
    tables hold experts 2..5)."""
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 256, [1024] * 4, 4, 0, seed=150)    # local experts 2, 3, 4, 5
    x = synth.activations(1, 256, seed=13)
    sel = [5, 1, 7, 3]
    w = np.array([0.5, 0.25, 0.125, 1.0], np.float16)
    C = torch.zeros((4, 1, 1024), dtype=torch.float, device="cuda")
    A_had = torch.empty((4, 1, 256), dtype=torch.half, device="cuda")
    idx = torch.tensor([sel], dtype=torch.long, device="cuda")
    wt = torch.from_numpy(w[None]).cuda()
    ops.exl3_mgemm(cuda_x(torch, x[None]), bd.B, C, bd.suh, A_had, bd.svh, idx, wt, 4,
                   min_index=2, max_index=6, num_tokens=num_tokens)
    got = C.cpu().numpy()
    loc = [s - 2 if 2 <= s < 6 else -1 for s in sel]
    if num_tokens == 1:
        kept = [(l, wi) for l, wi in zip(loc, w) if l >= 0]
        ref = sum(np.float64(wi) * bd.ref(orc, l, x, True).astype(np.float64) for l, wi in kept)
        assert rel_err(got[0], ref) < TOL
    else:
        ref = weighted_ref(bd, orc, [x] * 4, loc, w.astype(np.float64), 2, True)
        for t in range(2):
            assert rel_err(got[t], ref[t]) < TOL, t


def test_mgemm_repeat_deterministic(torch_cuda, orc):
    """Counters re-arm: repeated launches reproduce the same bits."""
    torch = torch_cuda
    from ampstein_amd import ops
    bd = Bundle(torch, 4096, [1024, 1024], 4, 0, seed=170)
    x = synth.activations(1, 4096, seed=17)
    A = cuda_x(torch, x[None])
    A_had = torch.empty((2, 1, 4096), dtype=torch.half, device="cuda")
    res = []
    for _ in range(3):
        C = torch.empty((2, 1, 1024), dtype=torch.half, device="cuda")
        ops.mgemm(A, bd.B, C, bd.suh, A_had, bd.svh, 4, False, False)
        res.append(C.cpu().numpy())
    assert np.array_equal(res[0].view(np.uint16), res[1].view(np.uint16))
    assert np.array_equal(res[0].view(np.uint16), res[2].view(np.uint16))
    for q in range(2):
        assert rel_err(res[0][q], bd.ref(orc, q, x, False)) < TOL
