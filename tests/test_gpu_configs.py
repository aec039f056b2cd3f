"""GPU parity at the benchmark configurations' own sizes (BASELINE.json configs[1..4]).

Every case runs the HIP path through the C ABI on the full-size synthetic layer and compares
with the CPU oracle (fp64 accumulation on the oracle's bit-exact W_hat) on the same bytes.
Bar (tests/tol.py): max relative error 2e-3, norm-wise and element-wise.

- configs[1] Llama-3-8B decode shapes at 4 bpw 3INST, M = 1: every linear alone, plus the q/k/v
  sliced bundle and the gate/up stacked bundle the decode step launches.
- configs[2] Qwen-27B-class shapes x K {2, 3, 5, 8} x {3INST, MCG} x M {1, 4, 8}.
- configs[3] prefill, 2048 rows through 8192 -> 28672 and 28672 -> 8192: the MFMA GEMM and both
  branches of exl3_gemm_recon, on 32 sampled rows.
- configs[4] MoE: 256 experts (4096 -> 2048 -> 4096), per-expert K in {2, 3, 4}, mul1, softmax
  top-8, M {1, 8, 16}; the routed outputs against an fp64 model, the run table bit for bit.
"""
import numpy as np
import pytest

from ampstein_amd import synth
from tests import moe_ref
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


def gemm(torch, L, x):
    from ampstein_amd import ops
    t, s, v = L.torch()
    A = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    C = torch.full((x.shape[0], L.n), float("nan"), dtype=torch.half, device="cuda")
    tag = ops.exl3_gemm(A, t, C, s, torch.empty_like(A), v, 0, L.cb == 1, L.cb == 2)
    torch.cuda.synchronize()
    return tag, C.cpu().numpy()


# ------------------------------------------------------------------ configs[1]
@pytest.mark.parametrize("name,k,n", synth.LLAMA3_8B_SHAPES)
def test_llama3_8b_linear_m1(torch_cuda, orc, name, k, n):
    L = synth.layer(k, n, 4, 0, seed=1000 + k + n)
    x = synth.activations(1, k, seed=1001)
    tag, y = gemm(torch_cuda, L, x)
    assert tag == 90
    assert_close(y, orc.linear_f64(x, L.trellis, L.suh, L.svh, 4), what=name)


def _linears(torch, specs, seed):
    from ampstein_amd.bundles import Linear
    layers = [synth.layer(k, n, 4, 0, seed=seed + i) for i, (k, n) in enumerate(specs)]
    lins = []
    for L in layers:
        t, s, v = L.torch()
        lins.append(Linear(t, s, v, 4.0))
    return layers, lins


def test_llama3_8b_qkv_sliced_bundle(torch_cuda, orc):
    torch = torch_cuda
    from ampstein_amd import bundles
    layers, lins = _linears(torch, [(4096, 4096), (4096, 1024), (4096, 1024)], 1100)
    outs = [torch.full((1, 1, L.n), float("nan"), dtype=torch.half, device="cuda") for L in layers]
    x = synth.activations(1, 4096, seed=1101)
    bundles.Sliced(lins, outs).run(torch.from_numpy(x[None]).cuda())
    torch.cuda.synchronize()
    for i, L in enumerate(layers):
        assert_close(outs[i].cpu().numpy()[0], orc.linear_f64(x, L.trellis, L.suh, L.svh, 4), what="qkv"[i])


def test_llama3_8b_gate_up_stacked_bundle(torch_cuda, orc):
    torch = torch_cuda
    from ampstein_amd import bundles
    layers, lins = _linears(torch, [(4096, 14336), (4096, 14336)], 1200)
    out = torch.full((2, 1, 14336), float("nan"), dtype=torch.half, device="cuda")
    x = synth.activations(1, 4096, seed=1201)
    bundles.Multi(lins, out).run(torch.from_numpy(x[None]).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, L in enumerate(layers):
        assert_close(got[i], orc.linear_f64(x, L.trellis, L.suh, L.svh, 4), what=("gate", "up")[i])


# ------------------------------------------------------------------ configs[2]
QWEN_SHAPES = [(5120, 5120), (5120, 1024), (5120, 17408), (17408, 5120)]


@pytest.mark.parametrize("k,n", QWEN_SHAPES)
@pytest.mark.parametrize("K", [2, 3, 5, 8])
@pytest.mark.parametrize("cb", [0, 1])
def test_qwen27b_shapes(torch_cuda, orc, k, n, K, cb):
    """M = 1 (stream kernel), 4 and 8 (row kernels; 8 = a 1 + 7 draft-token verify batch); the
    rows are independent, so one oracle call on 8 rows checks all three."""
    L = synth.layer(k, n, K, cb, seed=2000 + 10 * K + cb + k // 128 + n)
    x = synth.activations(8, k, seed=2001 + K)
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, K, cb=cb)
    for m in (1, 4, 8):
        tag, y = gemm(torch_cuda, L, x[:m])
        assert tag == 90
        assert_close(y, ref[:m], what=f"{k}x{n} K{K} cb{cb} M{m}")


# ------------------------------------------------------------------ configs[3]
PREFILL_ROWS = np.array([0, 1, 2, 3, 127, 128, 255, 256, 511, 700, 1023, 1024, 1025, 1300, 1535, 1536,
                         1600, 1777, 1800, 1900, 2000, 2016, 2030, 2040, 2044, 2045, 2046, 2047, 64, 900, 1200, 333])


@pytest.mark.parametrize("k,n", [(8192, 28672), (28672, 8192)])
def test_prefill_2048_rows(torch_cuda, orc, k, n):
    """2048 rows at 4 bpw 3INST: the hand-written MFMA GEMM (exl3_gemm, m > 8), the reference's
    fused-W recon branch (rows >= 2048) and the rotated recon branch."""
    torch = torch_cuda
    from ampstein_amd import ops
    L = synth.layer(k, n, 4, 0, seed=3000 + k)
    x = synth.activations(2048, k, seed=3001)
    ref = orc.linear_f64(x[PREFILL_ROWS], L.trellis, L.suh, L.svh, 4)
    tag, y = gemm(torch, L, x)
    assert tag == 91
    assert_close(y[PREFILL_ROWS], ref, what="mfma gemm")
    t, s, v = L.torch()
    xd = torch.from_numpy(x).cuda()
    yr = ops.exl3_gemm_recon(xd, t, s, v, 4.0, fused_rows=1 << 30)
    torch.cuda.synchronize()
    assert_close(yr.cpu().numpy()[PREFILL_ROWS], ref, what="rotated")
    del yr
    # The fused-W branch multiplies by W = diag(suh) H W_hat H diag(svh) rounded to fp16 by the
    # reference's reconstruct_had sequence (several fp16 butterfly roundings per element).  Its
    # reference result is x @ W on that fp16 W (the oracle's reconstruct_had, bit-exact with the
    # kernel's) in fp64; against the exact linear it stays within 1e-2.
    yf = ops.exl3_gemm_recon(xd, t, s, v, 4.0, fused_rows=2048)
    torch.cuda.synchronize()
    yf = yf.cpu().numpy()[PREFILL_ROWS]
    W = orc.reconstruct_had(L.trellis, L.suh, L.svh, 4).astype(np.float64)
    assert_close(yf, x[PREFILL_ROWS].astype(np.float64) @ W, what="fused_w vs x @ W_fp16")
    assert_close(yf, ref, tol=1e-2, what="fused_w vs exact")


# ------------------------------------------------------------------ configs[4]
class Experts256:
    """256 experts, gate/up 4096 -> 2048 and down 2048 -> 4096, per-expert K in {2, 3, 4}, mul1.
    Trellis words and signs are drawn on the GPU from a seeded generator; the oracle reads back
    only the routed experts (the model reconstructs one expert at a time)."""

    def __init__(self, torch, seed=4000):
        self.n, self.Hi, self.I, self.Ho, self.cb = 256, 4096, 2048, 4096, 2
        rng = np.random.default_rng(seed)
        self.K = [int(k) for k in rng.choice([2, 3, 4], self.n)]
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.dev = []
        for e in range(self.n):
            trio = []
            for (k, n) in ((self.Hi, self.I), (self.Hi, self.I), (self.I, self.Ho)):
                t = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * self.K[e]), dtype=torch.int16,
                                  device="cuda", generator=g)
                s = (torch.randint(0, 2, (k,), device="cuda", generator=g) * 2 - 1).half()
                v = (torch.randint(0, 2, (n,), device="cuda", generator=g) * 2 - 1).half()
                trio.append((t, s, v))
            self.dev.append(tuple(trio))
        P = lambda vals: torch.tensor(vals, dtype=torch.long, device="cuda")
        self.tables = {}
        for pi, name in enumerate("gud"):
            self.tables[name + "_trellis"] = P([self.dev[e][pi][0].data_ptr() for e in range(self.n)])
            self.tables[name + "_suh"] = P([self.dev[e][pi][1].data_ptr() for e in range(self.n)])
            self.tables[name + "_svh"] = P([self.dev[e][pi][2].data_ptr() for e in range(self.n)])
        self.bits = {name: torch.tensor(self.K, dtype=torch.uint8, device="cuda") for name in "gud"}

    def host(self, e, pi):
        t, s, v = self.dev[e][pi]
        return (t.cpu().numpy().view(np.uint16), s.cpu().numpy().astype(np.float64),
                v.cpu().numpy().astype(np.float64))

    def reference(self, orc, x, sel, rw):
        """Sum over k (in order) of rw_k * down(silu(gate(x)) * up(x)) with the fused kernel's fp16
        rounding points (tests/moe_ref.py), one routed expert at a time."""
        bsz, topk = sel.shape
        slot = np.zeros((bsz, topk, self.Ho))
        for e in np.unique(sel):
            W, sv = [], []
            for pi in range(3):
                t, s, v = self.host(int(e), pi)
                W.append(orc.reconstruct(t, self.K[e], cb=2).astype(np.float64))
                sv.append((s, v))
            for tk in zip(*np.nonzero(sel == e)):
                xr = x[tk[0]].astype(np.float64)
                proj = lambda i, inp: moe_ref.had(moe_ref.f16(moe_ref.had(inp * sv[i][0])) @ W[i]) * sv[i][1]
                a = moe_ref.act_fn(0, True, proj(0, xr), proj(1, xr), 0.0)
                slot[tk] = proj(2, a)
            del W
        out = np.zeros((bsz, self.Ho))
        for k in range(topk):
            out += rw[:, k].astype(np.float64)[:, None] * slot[:, k]
        return out


@pytest.fixture(scope="module")
def experts256(torch_cuda):
    return Experts256(torch_cuda)


@pytest.mark.parametrize("bsz", [1, 8, 16])
def test_moe_256_experts(torch_cuda, orc, experts256, bsz):
    from tests.test_gpu_moe import check_runs, routing, run
    rng = np.random.default_rng(4100 + bsz)
    sel, rw = routing(rng, bsz, 256, 8)
    x = rng.standard_normal((bsz, 4096)).astype(np.float16)
    y, runs = run(torch_cuda, experts256, x, sel, rw)
    check_runs(runs, sel, rw, -1, -1)
    assert_close(y, experts256.reference(orc, x, sel, rw), what=f"moe M{bsz}")
