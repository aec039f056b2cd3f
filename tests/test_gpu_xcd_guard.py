"""The per-launch check of the XCD-local split-k hand-off on the GPU (exl3_xcd.cuh, XcdGuard).

1. The tests that ran before this module in the same process (every hand-off path of the GEMV
   and the MoE) raised no alarm, and the hand-off is still on.
2. The flag path, per hand-off kernel (single-row per-chunk split, balanced single-row split,
   LDS multi-row kernel, and the coop MoE's gate/up and down stages): with the test policy EXL3_AMD_POLICY_XCD_FAKE, workgroup X (X = the
   device's XCD count) reports XCC + 1, as if dispatch had put it on another XCD than workgroup 0
   of its counter.  The launch's output stays right (real dispatch is unchanged), the alarm is
   seen, the library turns the hand-off off, the next calls (finish-kernel path) are right too,
   and exl3_amd_xcd_rearm restores the probe's XCD count.
3. With the hand-off off, the split residual norm's producer (exl3_gemm_res) runs its epilogue
   in the finish kernel: bit-identical to exl3_gemm + res_sq.
Bar of every output: the oracle's fp64 linear, 2e-3 (tests/tol.py).
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


def test_no_alarm_before(torch_cuda):
    probe, active, alarms = _lib.xcd_status(0)
    assert alarms == 0
    assert active == probe


PATHS = {
    "m1-per-chunk": (1, 4096, 4096, None),
    "m1-balanced": (1, 4096, 14336, (_lib.POLICY_GEMV_SPLIT, _lib.GEMV_SPLIT_BALANCED)),
    "m4-lds": (4, 4096, 4096, (_lib.POLICY_GEMV_ROWS, _lib.GEMV_ROWS_LDS)),
}


@pytest.mark.parametrize("path", list(PATHS))
def test_flag_path(torch_cuda, orc, kernel_policy, path):
    torch = torch_cuda
    from ampstein_amd import ops
    m, k, n, pol = PATHS[path]
    probe, active, alarms0 = _lib.xcd_status(0)
    if probe == 0:
        pytest.skip("the XCD-local hand-off is off on this device")
    assert active == probe
    if pol:
        kernel_policy(*pol)
    L = synth.layer(k, n, 4, 0, seed=9700 + m + n // 1024)
    x = synth.activations(m, k, seed=9701)
    t, s, v = L.torch()
    A = torch.from_numpy(x).cuda()
    ref = orc.linear_f64(x, L.trellis, L.suh, L.svh, 4)

    def run(what):
        C = torch.full((m, n), float("nan"), dtype=torch.half, device="cuda")
        assert ops.exl3_gemm(A, t, C, s, torch.empty_like(A), v, 0, False, False) == 90
        torch.cuda.synchronize()
        y = C.cpu().numpy()
        assert np.isfinite(y.astype(np.float32)).all(), what
        assert_close(y, ref, what=f"{path} {what}")

    try:
        run("hand-off on")
        assert _lib.xcd_status(0) == (probe, probe, alarms0)
        kernel_policy(_lib.POLICY_XCD_FAKE, probe + 1)
        print(f"[xcd guard] {path}: workgroup {probe} reports another XCC", flush=True)
        run("reported mix")
        assert _lib.xcd_status(0) == (probe, 0, alarms0 + 1)
        run("hand-off off")
        run("hand-off off, again")
        assert _lib.xcd_status(0) == (probe, 0, alarms0 + 1)
    finally:
        _lib.check(_lib.lib().exl3_amd_xcd_rearm(0))
    assert _lib.xcd_status(0)[:2] == (probe, probe)


def test_flag_path_moe_coop(torch_cuda, orc, kernel_policy):
    """The same on exl3_amd_moe_coop (gate/up and down hand-offs of moe_a / moe_b, I = Ho = 1024:
    8 column chunks, XCD mode): workgroup X shares chunk 0's row counters with workgroup 0."""
    torch = torch_cuda
    from tests import moe_ref
    from tests.test_gpu_moe import rel_err, routing, run
    probe, active, alarms0 = _lib.xcd_status(0)
    if probe == 0:
        pytest.skip("the XCD-local hand-off is off on this device")
    rng = np.random.default_rng(9800)
    es = moe_ref.ExpertSet(torch, orc, 16, 256, 1024, 1024, rng.choice([2, 3, 4], 16), 2, seed=9801)
    sel, rw = routing(rng, 8, 16, 8)
    x = rng.standard_normal((8, 256)).astype(np.float16)
    ref = moe_ref.reference(es, x, sel, rw, -1, -1, 0, True, 0.0, 1024)
    try:
        y, _ = run(torch, es, x, sel, rw)
        assert rel_err(y, ref) < 2e-3
        assert _lib.xcd_status(0) == (probe, probe, alarms0)
        kernel_policy(_lib.POLICY_XCD_FAKE, probe + 1)
        print(f"[xcd guard] moe_coop: workgroup {probe} reports another XCC", flush=True)
        y, _ = run(torch, es, x, sel, rw)
        assert rel_err(y, ref) < 2e-3
        assert _lib.xcd_status(0) == (probe, 0, alarms0 + 1)
        y, _ = run(torch, es, x, sel, rw)                  # agent-scope hand-off
        assert rel_err(y, ref) < 2e-3
    finally:
        _lib.check(_lib.lib().exl3_amd_xcd_rearm(0))
    assert _lib.xcd_status(0)[:2] == (probe, probe)


def test_gemm_res_finish_kernel(torch_cuda, kernel_policy):
    """The hand-off turned off by the hook: the split partials are summed by the finish kernel,
    whose epilogue does the split norm's residual add and chunk sums."""
    from tests.test_gpu_split_norm import _check_gemm_res, _gemm_res_case
    torch = torch_cuda
    from ampstein_amd import ops
    probe, active, alarms0 = _lib.xcd_status(0)
    if probe == 0:
        pytest.skip("the XCD-local hand-off is off on this device")
    case = _gemm_res_case(4096, 4096, False, 1, 77)
    try:
        kernel_policy(_lib.POLICY_XCD_FAKE, probe + 1)
        C = torch.empty((1, 4096), dtype=torch.half, device="cuda")
        ops.exl3_gemm(case[3], case[0], C, case[1], torch.empty_like(case[3]), case[2])   # raises the alarm
        torch.cuda.synchronize()
        assert _lib.xcd_status(0) == (probe, 0, alarms0 + 1)
        print("[xcd guard] gemm_res with the finish kernel", flush=True)
        _check_gemm_res(*case, 1, 4096)
    finally:
        _lib.check(_lib.lib().exl3_amd_xcd_rearm(0))
    assert _lib.xcd_status(0)[:2] == (probe, probe)
