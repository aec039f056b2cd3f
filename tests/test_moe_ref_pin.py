"""Pins the MoE test model (tests/moe_ref.py) against the reference's own CPU MoE forward.

tests/golden/ref_moe_cpu_forward.npz holds the outputs of exl3_moe_cpu_forward_raw
(vendor/exl3/exllamav3_ext/cpu/moe_mul1.cpp:2529-2654), compiled from the reference source and run
on its scalar tier (fp32 throughout, no int8 activations) by tests/golden/make_ref_vectors.py, on
4 mul1 experts at K 2 / 3 / 4 with 6 routed rows (top-2, a repeated expert, a zero weight).

The model runs with its fp16 rounding points off (round16=False: the CPU forward has none) and the
CPU forward's fp32 mul1 values (golden mul1_f32, the reference's decode_mul1_scalar) so that the
two differ only by fp32 vs fp64 accumulation.  The bar is 1e-5, two orders below the MoE kernels'
2e-3: it pins the activation functions and constants, the act_limit clamps (up symmetric, the
activated gate from above, before the multiply), swiglu_oai's +1 and 1.702, gateless relu2, the
bias placement (after the output transform), and the routing-weighted sum.

The CPU forward's GELU is the erf form (moe_mul1.cpp:2196-2201); the reference's GPU kernels use
the tanh approximation (activation_kernels.cuh:44-57, exl3_moe_coop_kernel.cuh:86-91), which the
GPU tests follow.  The model's tanh form is checked against scipy's erf GELU at the approximation's
known accuracy, and the golden comparison shows the two are told apart at this bar.
"""
import numpy as np
import pytest
import scipy.special

from tests import moe_ref
from tests.tol import assert_close

CASES = {"silu": (0, 0.0, True, False), "silu_limit": (0, 10.0, True, False),
         "gelu": (1, 0.0, True, False), "swiglu_oai": (3, 7.0, True, False),
         "relu2": (2, 0.0, False, False), "silu_bias": (0, 0.0, True, True)}


@pytest.fixture(scope="module")
def cpu_moe(orc, golden):
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "ref_moe_cpu_forward.npz")
    g = dict(np.load(path))
    perm = orc.tile_perm()
    mul1 = golden["mul1_f32"].astype(np.float64)
    E, H, I = int(g["E"]), int(g["H"]), int(g["I"])
    W = []
    for e in range(E):
        K = int(g["bits"][e])
        mats = []
        for p, (k, n) in enumerate(((H, I), (H, I), (I, H))):
            tr = g[f"trellis_{e}_{p}"]
            Wp = np.empty((k, n))
            for tk in range(k // 16):
                for tn in range(n // 16):
                    tile = np.ascontiguousarray(tr[tk, tn])
                    vals = np.empty(256)
                    for t in range(256):
                        vals[perm[t]] = mul1[orc.state(tile, K, False, t)]
                    Wp[16 * tk:16 * tk + 16, 16 * tn:16 * tn + 16] = vals.reshape(16, 16)
            mats.append(Wp)
        W.append(tuple(mats))
    g["W"] = W
    return g


class CpuSet:
    """moe_ref.reference's expert-set interface over the golden experts."""

    def __init__(self, g, gelu_erf):
        self.g, self.gelu_erf, self.Ho = g, gelu_erf, int(g["H"])

    def slot_out(self, x_row, e, act, gated, limit, use_bias=False):
        g = self.g
        sv = [(g[f"suh_{e}_{p}"].astype(np.float64), g[f"svh_{e}_{p}"].astype(np.float64)) for p in range(3)]
        bias = [g[f"bias_{e}_{p}"].astype(np.float64) if use_bias else None for p in range(3)]
        return moe_ref.expert_out(x_row, g["W"][e], sv, bias, act, gated, limit,
                                  round16=False, gelu_erf=self.gelu_erf)


@pytest.mark.parametrize("case", list(CASES))
def test_model_vs_reference_cpu_forward(cpu_moe, case):
    act, limit, gated, bias = CASES[case]
    g = cpu_moe
    x, sel, w = g["x"], g["sel"].astype(np.int64), g["w"]
    ref = g[f"out_{case}"].astype(np.float64)
    got = moe_ref.reference(CpuSet(g, gelu_erf=True), x, sel, w, -1, -1, act, gated, limit, int(g["H"]),
                            use_bias=bias)
    assert_close(got, ref, tol=1e-5, what=case)


def test_limits_are_active(cpu_moe):
    """The clamped cases differ from their unclamped forms, so the clamps are exercised."""
    g = cpu_moe
    assert np.abs(g["out_silu_limit"] - g["out_silu"]).max() > 1e-2 * np.abs(g["out_silu"]).max()
    x, sel, w = g["x"], g["sel"].astype(np.int64), g["w"]
    unclamped = moe_ref.reference(CpuSet(g, True), x, sel, w, -1, -1, 3, True, 0.0, int(g["H"]))
    assert np.abs(unclamped - g["out_swiglu_oai"]).max() > 1e-2 * np.abs(unclamped).max()


def test_gelu_tanh_form(cpu_moe):
    """The tanh form (the reference's GPU GELU) is within its known 5e-4 absolute accuracy of the erf
    GELU, and the golden comparison tells the two apart."""
    v = np.linspace(-8, 8, 20001)
    erf_gelu = 0.5 * v * (1 + scipy.special.erf(v / np.sqrt(2)))
    tanh_gelu = moe_ref.act_fn(1, True, v, np.ones_like(v), 0.0)
    assert np.abs(tanh_gelu - erf_gelu).max() < 5e-4
    assert np.array_equal(moe_ref.act_fn(1, True, v, np.ones_like(v), 0.0, gelu_erf=True), erf_gelu)
    g = cpu_moe
    x, sel, w = g["x"], g["sel"].astype(np.int64), g["w"]
    tanh_out = moe_ref.reference(CpuSet(g, False), x, sel, w, -1, -1, 1, True, 0.0, int(g["H"]))
    ref = g["out_gelu"].astype(np.float64)
    with pytest.raises(AssertionError):
        assert_close(tanh_out, ref, tol=1e-5, what="tanh gelu at the golden bar")
    assert_close(tanh_out, ref, tol=2e-3, what="tanh gelu")


def test_activation_special_points():
    """Closed forms: silu(0) = 0, silu(g) -> g and -> 0 at the tails, relu2, swiglu_oai at g = 0
    and with u clamped to -limit (the +1 makes it (1 - limit) glu)."""
    f = moe_ref.act_fn
    one = np.array([1.0])
    assert f(0, True, np.array([0.0]), one, 0.0)[0] == 0.0
    assert abs(f(0, True, np.array([40.0]), one, 0.0)[0] - 40.0) < 1e-15
    assert abs(f(0, True, np.array([-40.0]), one, 0.0)[0]) < 1e-15
    assert f(0, True, np.array([np.log(3.0)]), one, 0.0)[0] == pytest.approx(0.75 * np.log(3.0), rel=1e-15)
    assert f(2, False, np.array([-3.0]), np.array([-3.0]), 0.0)[0] == 0.0
    assert f(2, False, np.array([3.0]), np.array([3.0]), 0.0)[0] == 9.0
    assert f(3, True, np.array([0.0]), np.array([5.0]), 7.0)[0] == 0.0
    g = np.array([20.0])
    glu = 7.0 / (1.0 + np.exp(-1.702 * 7.0))
    assert f(3, True, g, np.array([-50.0]), 7.0)[0] == pytest.approx((1.0 - 7.0) * glu, rel=1e-15)
    # gated act with limit: the activated gate is clamped from above, u symmetrically
    assert f(0, True, np.array([30.0]), np.array([-50.0]), 10.0)[0] == pytest.approx(-100.0, rel=1e-12)
