"""GPU parity of the fused MoE (exl3_amd_moe_coop through the C ABI) against the fp64 model in
tests/moe_ref.py (the reference semantics on the oracle's bit-exact weights), plus a bit-exact
check of the gather: the run table the kernel writes must equal the host's (token, expert) list
sorted by expert.  Bar: max|y - ref| / max|ref| < 2e-3."""
import numpy as np
import pytest

from tests import moe_ref

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


def routing(rng, bsz, n_experts, topk):
    """Router logits ~ N(0, 1), softmax, top-k (ties to the lower index); rw = top-k probabilities."""
    logits = rng.standard_normal((bsz, n_experts))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    sel = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    rw = np.take_along_axis(p, sel, 1).astype(np.float16)
    return sel.astype(np.int64), rw


def run(torch, es, x, sel, rw, *, mn=-1, mx=-1, act=0, limit=0.0, gated=True, mixed=True, H_out=None,
        sh_out=None, sh_gate_w=None, bias=False, slots_max=None, rows_max=None, moe_fn=None):
    from ampstein_amd import ops
    moe_fn = moe_fn or ops.exl3_moe_coop
    bsz, topk = sel.shape
    H = x.shape[1]
    H_out = H_out or es.Ho
    slots_max = slots_max or bsz * topk
    rows_max = rows_max or bsz
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    z = lambda *shape, dt=torch.half: torch.zeros(shape, dtype=dt, device="cuda")
    had_g, had_u = z(slots_max, es.Hi), z(slots_max, es.Hi)
    gu_g, gu_u = z(slots_max, es.I, dt=torch.float), z(slots_max, es.I, dt=torch.float)
    act_out = z(slots_max, es.I)
    d_out = z(slots_max, es.Ho, dt=torch.float)
    ctr = torch.zeros(ops.moe_coop_ctr_len(slots_max, rows_max, es.I, es.Ho), dtype=torch.int32, device="cuda")
    out = torch.full((rows_max, H_out), float("nan"), dtype=torch.float, device="cuda")
    T = es.tables
    K = es.K[0]
    moe_fn(dev(x), dev(sel), dev(rw), mn, mx, es.Hi,
                      T["g_trellis"], T["g_suh"], T["g_svh"], T["u_trellis"], T["u_suh"], T["u_svh"],
                      T["d_trellis"], T["d_suh"], T["d_svh"],
                      T.get("g_bias") if bias else None, T.get("u_bias") if bias else None,
                      T.get("d_bias") if bias else None,
                      K, K, K, es.cb == 1, es.cb == 2, act, limit, gated,
                      had_g, had_u, gu_g, gu_u, act_out, d_out, ctr, out,
                      None if sh_out is None else dev(sh_out), None if sh_gate_w is None else dev(sh_gate_w),
                      *((es.bits["g"], es.bits["u"], es.bits["d"]) if mixed else (None, None, None)))
    torch.cuda.synchronize()
    off = slots_max * (es.I // 128) + rows_max * (es.Ho // 128)
    c = ctr.cpu().numpy()
    runs = (int(c[off]), c[off + 2: off + 2 + slots_max + 1], c[off + 2 + slots_max + 1:])
    return out.cpu().numpy()[:bsz], runs


@pytest.fixture(scope="module")
def experts_mixed(torch_cuda, orc):
    """16 experts, mixed K in {2,3,4} by seed, mul1; Hi 256, I 1024, Ho 1024 (8 chunks: XCD hand-off)."""
    rng = np.random.default_rng(5)
    return moe_ref.ExpertSet(torch_cuda, orc, 16, 256, 1024, 1024, rng.choice([2, 3, 4], 16), 2, seed=5, bias=True)


@pytest.fixture(scope="module")
def experts_small(torch_cuda, orc):
    """12 experts, uniform K = 3, 3INST; I = Ho = 256 (2 chunks: device-scope hand-off)."""
    return moe_ref.ExpertSet(torch_cuda, orc, 12, 256, 256, 256, [3] * 12, 0, seed=6, bias=True)


def check_runs(runs, sel, rw, mn, mx):
    n, starts, order = runs
    hn, hstarts, horder = moe_ref.host_runs(sel, rw, mn, mx)
    assert n == hn
    assert list(starts[: n + 1]) == hstarts
    assert list(order[: len(horder)]) == horder


@pytest.mark.parametrize("bsz", [1, 8, 16])
def test_moe_mixed_k_routing(torch_cuda, experts_mixed, bsz):
    """Config-5 semantics at test scale: mixed K, SiLU, top-8 of softmax routing."""
    rng = np.random.default_rng(100 + bsz)
    sel, rw = routing(rng, bsz, 16, 8)
    x = rng.standard_normal((bsz, 256)).astype(np.float16)
    y, runs = run(torch_cuda, experts_mixed, x, sel, rw)
    ref = moe_ref.reference(experts_mixed, x, sel, rw, -1, -1, 0, True, 0.0, 1024)
    assert rel_err(y, ref) < TOL
    check_runs(runs, sel, rw, -1, -1)


@pytest.mark.parametrize("act", [0, 1, 2, 3])
@pytest.mark.parametrize("gated", [True, False])
def test_moe_activations(torch_cuda, experts_small, act, gated):
    rng = np.random.default_rng(7 + act)
    sel, rw = routing(rng, 3, 12, 4)
    x = rng.standard_normal((3, 256)).astype(np.float16)
    limit = 7.0 if act == 3 else 0.0
    y, runs = run(torch_cuda, experts_small, x, sel, rw, act=act, gated=gated, limit=limit, mixed=False)
    ref = moe_ref.reference(experts_small, x, sel, rw, -1, -1, act, gated, limit, 256)
    assert rel_err(y, ref) < TOL


def test_moe_bias_shared_padding(torch_cuda, experts_small):
    """Biases, a gated shared expert, input narrower than Hi (zero padding), trimmed output."""
    rng = np.random.default_rng(11)
    sel, rw = routing(rng, 4, 12, 4)
    H = 200
    x = rng.standard_normal((4, H)).astype(np.float16)
    sh_out = rng.standard_normal((4, H)).astype(np.float32)
    sh_gate_w = (rng.standard_normal(H) * 0.05).astype(np.float16)
    y, _ = run(torch_cuda, experts_small, x, sel, rw, mixed=False, H_out=H, sh_out=sh_out, sh_gate_w=sh_gate_w,
               bias=True)
    ref = moe_ref.reference(experts_small, x, sel, rw, -1, -1, 0, True, 0.0, H, sh_out, sh_gate_w, use_bias=True)
    assert rel_err(y, ref) < TOL


def test_moe_range_filter_and_empty_rows(torch_cuda, experts_mixed):
    """Expert-parallel shard [4, 12): out-of-range picks and zero weights are inactive; a token
    with no active pick gets only the shared-expert term."""
    rng = np.random.default_rng(13)
    sel = np.array([[4, 5, 20, 11], [0, 1, 2, 3], [7, 7, 9, 4]], np.int64)
    rw = np.array([[0.5, 0.25, 0.125, 0.125], [0.4, 0.3, 0.2, 0.1], [0.5, 0.0, 0.25, 0.25]], np.float16)
    x = rng.standard_normal((3, 256)).astype(np.float16)
    sh_out = rng.standard_normal((3, 256)).astype(np.float32)
    # local tables: experts 4..11 of the 16 (shard)
    y, runs = run(torch_cuda, experts_mixed, x, sel + 0, rw, mn=4, mx=12, H_out=256, sh_out=sh_out, slots_max=16)
    ref = np.zeros((3, 256))
    ok = moe_ref.active(sel, rw, 4, 12)
    for t in range(3):
        acc = np.zeros(1024)
        for k in range(4):
            if ok[t, k]:
                acc += float(rw[t, k]) * experts_mixed.slot_out(x[t].astype(np.float64), int(sel[t, k]) - 4, 0, True, 0.0)
        acc[:256] += sh_out[t]
        ref[t] = acc[:256]
    assert rel_err(y, ref) < TOL
    assert np.allclose(y[1], sh_out[1], atol=0, rtol=0)
    check_runs(runs, sel, rw, 4, 12)


@pytest.mark.parametrize("case", ["bsz1", "bsz8", "bias", "filter", "hi512"])
def test_moe_epilogue_forms_bit_identical(torch_cuda, orc, experts_mixed, experts_small, kernel_policy, case):
    """The gate/up and down epilogues' prefetched forms (every load issued first) and their
    general loops give the same bits: same operations in the same order."""
    from ampstein_amd import _lib
    rng = np.random.default_rng(300 + len(case))
    kw = {}
    if case == "bias":
        es, (sel, rw) = experts_small, routing(rng, 4, 12, 4)
        kw = dict(mixed=False, bias=True)
    elif case == "hi512":
        # Hi = 512 at one token: 4 gate/up k-splits (the widest prefetched form)
        es = moe_ref.ExpertSet(torch_cuda, orc, 8, 512, 256, 256, [3] * 8, 0, seed=31)
        sel, rw = routing(rng, 1, 8, 8)
        kw = dict(mixed=False)
    else:
        es, (sel, rw) = experts_mixed, routing(rng, 8 if case == "bsz8" else 1, 16, 8)
        if case == "filter":
            kw = dict(mn=4, mx=12)
    x = rng.standard_normal((sel.shape[0], 256)).astype(np.float16)
    y1, _ = run(torch_cuda, es, x, sel, rw, **kw)
    kernel_policy(_lib.POLICY_MOE_EPILOGUE, _lib.MOE_EPILOGUE_SERIAL)
    y2, _ = run(torch_cuda, es, x, sel, rw, **kw)
    assert np.array_equal(np.asarray(y1).view(np.uint32), np.asarray(y2).view(np.uint32))


def test_moe_repeat_deterministic(torch_cuda, experts_mixed):
    rng = np.random.default_rng(17)
    sel, rw = routing(rng, 16, 16, 8)
    x = rng.standard_normal((16, 256)).astype(np.float16)
    y1, _ = run(torch_cuda, experts_mixed, x, sel, rw)
    y2, _ = run(torch_cuda, experts_mixed, x, sel, rw)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("bsz", [1, 4])
def test_moe_repeated_expert(torch_cuda, experts_mixed, bsz):
    """A token that picks one expert twice: the run holds both slots (one token: the single-row
    launch takes it in two passes; several tokens: the multi-row launch)."""
    rng = np.random.default_rng(19 + bsz)
    sel, rw = routing(rng, bsz, 16, 8)
    sel[0, 1] = sel[0, 0]
    sel[bsz - 1, 5] = sel[bsz - 1, 2]
    x = rng.standard_normal((bsz, 256)).astype(np.float16)
    y, runs = run(torch_cuda, experts_mixed, x, sel, rw)
    ref = moe_ref.reference(experts_mixed, x, sel, rw, -1, -1, 0, True, 0.0, 1024)
    assert rel_err(y, ref) < TOL
    check_runs(runs, sel, rw, -1, -1)


@pytest.mark.parametrize("K", [1.5, 2.5, 3.5])
def test_moe_half_rate(torch_cuda, orc, K):
    """Uniform half-integer bitrate (mul1): gate/up and down at K + 0.5 bits."""
    es = moe_ref.ExpertSet(torch_cuda, orc, 8, 256, 1024, 1024, [K] * 8, 2, seed=int(4 * K))
    rng = np.random.default_rng(int(10 * K))
    for bsz in (1, 4):
        sel, rw = routing(rng, bsz, 8, 4)
        x = rng.standard_normal((bsz, 256)).astype(np.float16)
        y, runs = run(torch_cuda, es, x, sel, rw, mixed=False)
        ref = moe_ref.reference(es, x, sel, rw, -1, -1, 0, True, 0.0, 1024)
        assert rel_err(y, ref) < TOL, bsz
        check_runs(runs, sel, rw, -1, -1)
