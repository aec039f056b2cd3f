"""CPU checks of the C-ABI library: it loads, exports every entry point include/exl3_amd.h
declares, and rejects bad arguments before touching a GPU (tests/bindings_errors.uc of the
reference requires every binding to raise on bad arguments)."""
import ctypes
import os
import re

import pytest

from ampstein_amd import _lib


def header_symbols():
    text = open(_lib.HEADER).read()
    return sorted(set(re.findall(r"\b(exl3_amd_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    assert set(header_symbols()) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in header_symbols():
        assert hasattr(L, name), name
    assert L.exl3_amd_version() >= 100


def call_err(fn, *args):
    rc = fn(*args)
    return rc, _lib.lib().exl3_amd_last_error().decode()


def test_reconstruct_rejects_bad_arguments():
    L = _lib.lib()
    f = ctypes.c_float
    rc, msg = call_err(L.exl3_amd_reconstruct, 1, 1, 16, 128, 128, 0, f(9.0), 0, 0, None)
    assert rc == _lib.EINVAL and "bitrate" in msg
    rc, msg = call_err(L.exl3_amd_reconstruct, 1, 1, 16, 128, 128, 0, f(2.5), 0, 0, None)
    assert rc == _lib.EINVAL and "mul1" in msg
    rc, msg = call_err(L.exl3_amd_gemm, 1, 1, 1, 0, 1, None, 1, 1, 256, 256, f(4.0), 1, 1, 0, None)
    assert rc == _lib.EINVAL and "both" in msg
    rc, msg = call_err(L.exl3_amd_reconstruct, 1, 1, 16, 256, 64, 0, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "128" in msg
    rc, msg = call_err(L.exl3_amd_reconstruct, 1, 1, 16, 256, 128, 64, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "n_offset" in msg
    rc, msg = call_err(L.exl3_amd_reconstruct, 1, 1, 16, 256, 256, 128, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "bounds" in msg
    rc, msg = call_err(L.exl3_amd_reconstruct, None, 1, 16, 128, 128, 0, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "null" in msg
    # empty output is a successful no-op (reconstruct.cu:169-170)
    assert L.exl3_amd_reconstruct(None, None, 0, 128, 128, 0, f(4.0), 0, 0, None) == 0


def test_reconstruct_had_rejects_bad_arguments():
    L = _lib.lib()
    f = ctypes.c_float
    rc, msg = call_err(L.exl3_amd_reconstruct_had, 1, 1, 1, 1, 144, 128, 128, 0, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "K dimension" in msg
    rc, msg = call_err(L.exl3_amd_reconstruct_had, 1, 1, None, 1, 128, 128, 128, 0, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "null" in msg


def test_had_rejects_bad_arguments():
    L = _lib.lib()
    rc, msg = call_err(L.exl3_amd_had_r_128, 1, 1, 4, 100, 0, None, None, ctypes.c_float(1.0), None)
    assert rc == _lib.EINVAL and "128" in msg
    rc, msg = call_err(L.exl3_amd_had_r_128, 1, 1, 4, 128, 0, 1, 1, ctypes.c_float(1.0), None)
    assert rc == _lib.EINVAL


def test_gemm_rejects_bad_arguments():
    L = _lib.lib()
    f = ctypes.c_float
    args = lambda **kw: [kw.get(x, d) for x, d in (
        ("A", 1), ("B", 1), ("C", 1), ("fp32", 0), ("suh", 1), ("ahad", None), ("svh", 1),
        ("m", 1), ("k", 256), ("n", 256), ("K", f(4.0)), ("mcg", 0), ("mul1", 0), ("force", 0),
        ("stream", None))]
    rc, msg = call_err(L.exl3_amd_gemm, *args(n=100))
    assert rc == _lib.EINVAL and "n must" in msg
    rc, msg = call_err(L.exl3_amd_gemm, *args(k=24))
    assert rc == _lib.EINVAL and "k must" in msg
    rc, msg = call_err(L.exl3_amd_gemm, *args(K=f(0.5)))
    assert rc == _lib.EINVAL
    rc, msg = call_err(L.exl3_amd_gemm, *args(A=None))
    assert rc == _lib.EINVAL and "null" in msg
    rc, msg = call_err(L.exl3_amd_gemm, *args(force=7))
    assert rc == _lib.EINVAL and "force_shape_idx" in msg
    # m == 0 is an empty product: nothing to launch
    assert L.exl3_amd_gemm(*args(m=0)) == _lib.TAG_GEMV


def test_python_ops_raise_like_torch_check():
    import torch
    from ampstein_amd import ops
    W = torch.empty((32, 128), dtype=torch.half)
    T = torch.zeros((2, 8, 64), dtype=torch.int16)
    with pytest.raises(_lib.Exl3Error, match="bitrate"):
        ops.reconstruct(W, T, 9.0)
    with pytest.raises(_lib.Exl3Error, match="both"):
        ops.exl3_gemm(torch.empty((1, 32), dtype=torch.half), T, torch.empty((1, 128), dtype=torch.half),
                      None, None, None, mcg=True, mul1=True)
    with pytest.raises(_lib.Exl3Error, match="tile size"):
        ops.reconstruct(W, T, 3.0)
    with pytest.raises(_lib.Exl3Error, match="datatype"):
        ops.reconstruct(W.float(), T, 4.0)
    with pytest.raises(_lib.Exl3Error, match="incompatible"):
        ops.exl3_gemm(torch.empty((1, 64), dtype=torch.half), T, torch.empty((1, 128), dtype=torch.half), None, None, None)
    with pytest.raises(_lib.Exl3Error, match="128"):
        ops.had_r_128(torch.empty((2, 100), dtype=torch.half), torch.empty((2, 100), dtype=torch.half))


def mgemm_args(**kw):
    f = ctypes.c_float
    order = (("A", 1), ("bszm_in", 1), ("m", 1), ("k", 256), ("B", 1), ("num_B", 2), ("C", 1),
             ("bszm_out", 2), ("n", 256), ("fp32", 0), ("suh", 1), ("num_suh", 2), ("ahad", 1),
             ("ahad_n", 1 << 20), ("svh", 1), ("num_svh", 2), ("idx", None), ("num_idx", 0),
             ("w", None), ("K", f(4.0)), ("force", -1), ("mcg", 0), ("mul1", 0), ("min", -1),
             ("max", -1), ("sms", 0), ("tokens", 1), ("size_n", None), ("c_ptrs", None),
             ("num_c", 0), ("stride", None), ("num_stride", 0), ("src", None), ("num_src", 0),
             ("nsrc", 0), ("stream", None))
    return [kw.get(name, d) for name, d in order]


def test_mgemm_rejects_bad_arguments():
    """The TORCH_CHECKs of exl3_mgemm_gr (quant/exl3_gemm.cu:424-542) as error codes."""
    L = _lib.lib()
    f = ctypes.c_float
    cases = [
        (dict(mcg=1, mul1=1), "both"),
        (dict(num_suh=3), "same length"),
        (dict(size_n=1), "requires c_ptrs"),
        (dict(c_ptrs=1, size_n=1, num_c=2, w=1), "incompatible"),
        (dict(src=1), "sliced mode requires"),
        (dict(src=1, size_n=1, c_ptrs=1, num_c=2, stride=1, num_stride=2, num_src=2, nsrc=3), "one suh entry"),
        (dict(src=1, size_n=1, c_ptrs=1, num_c=2, stride=1, num_stride=1, num_src=2, nsrc=1), "one entry per slice"),
        (dict(stride=1), "n_stride_list requires"),
        (dict(ahad_n=100), "A_had"),
        (dict(idx=1, num_idx=3), "too many indices"),
        (dict(n=200), "n must"),
        (dict(min=0), "requires indices"),
        (dict(tokens=0), "num_tokens"),
        (dict(w=1, idx=1, num_idx=2, tokens=3), "token groups"),
        (dict(K=f(2.5), mul1=0), "mul1"),
    ]
    for kw, text in cases:
        rc, msg = call_err(L.exl3_amd_mgemm, *mgemm_args(**kw))
        assert rc < 0 and text in msg, (kw, msg)
    # nothing to do: empty batch rows
    assert L.exl3_amd_mgemm(*mgemm_args(m=0)) == _lib.TAG_GEMV


def moe_args(**kw):
    f = ctypes.c_float
    order = (("x", 1), ("bsz", 2), ("H", 256), ("xs", 256), ("sel", 1), ("rw", 1), ("topk", 4),
             ("min", -1), ("max", -1), ("Hi", 256),
             ("gt", 1), ("gs", 1), ("gv", 1), ("ut", 1), ("us", 1), ("uv", 1), ("dt", 1), ("ds", 1), ("dv", 1),
             ("n_local", 16), ("gb", None), ("ub", None), ("db", None),
             ("Kg", f(3.0)), ("Ku", f(3.0)), ("Kd", f(3.0)), ("mcg", 0), ("mul1", 1), ("act", 0),
             ("limit", f(0.0)), ("gated", 1),
             ("hg", 1), ("hg_n", 8 * 256), ("hu", 1), ("hu_n", 8 * 256),
             ("gug", 1), ("guu", 1), ("gu_n", 8 * 256), ("gu32", 1), ("I", 256),
             ("ao", 1), ("ao_n", 8 * 256), ("do", 1), ("do_n", 8 * 256), ("Ho", 256),
             ("ctr", 1), ("ctr_n", 1 << 16),
             ("out", 1), ("rows_max", 2), ("H_out", 256), ("ostride", 256),
             ("sh", None), ("shg", None), ("shg_n", 0), ("bg", None), ("bu", None), ("bd", None),
             ("stream", None))
    return [kw.get(name, d) for name, d in order]


def test_moe_coop_rejects_bad_arguments():
    """The TORCH_CHECKs of exl3_moe_coop_prepare / _run (quant/exl3_moe_coop.cu:185-305)."""
    L = _lib.lib()
    f = ctypes.c_float
    cases = [
        (dict(mcg=1), "both"),
        (dict(Kd=f(9.0)), "K out of range"),
        (dict(Kg=f(2.0)), "share a bit width"),
        (dict(act=4), "unknown activation"),
        (dict(I=200), "Hi/I/Ho"),
        (dict(H_out=512), "Hi/I/Ho"),
        (dict(hg_n=100), "1..256 slots"),
        (dict(ctr_n=10), "counter scratch"),
        (dict(bg=1), "all three"),
        (dict(H=258), "H/Hi"),
        (dict(bsz=3), "exceeds the scratch"),
        (dict(min=0, max=40), "expert range"),
        (dict(sh=1, H=128), "shared expert output width"),
        (dict(bg=1, bu=1, bd=1, mul1=0), "mul1"),
        (dict(gt=None), "pointer tables"),
    ]
    for kw, text in cases:
        rc, msg = call_err(L.exl3_amd_moe_coop, *moe_args(**kw))
        assert rc < 0 and text in msg, (kw, msg)
    assert L.exl3_amd_moe_coop(*moe_args(bsz=0)) == 0          # no tokens: nothing to do


def _moe_args(**kw):
    """exl3_amd_moe argument list (fake non-null addresses: every call here fails validation
    before any device access)."""
    a = dict(hidden=1, bsz=4, hidden_dim=256, out=1, count=1, count_len=9, tok=1, w=1, n=8,
             tsg=1, tsu=1, conc=1, max_tok=16, tig=1, tiu=1, I=256, act=0, Kg=3.0, Ku=3.0, Kd=3.0,
             tables=[1] * 9, num_ptrs=8, cbs=[1, 0, 1, 0, 1, 0], limit=0.0, num_active=3,
             scratch=None, scratch_rows=0, scratch_cols=0, fused_base=None, lo=0, hi=1 << 30, m_tile=16,
             bits=[None, None, None], bits_len=0)
    a.update(kw)
    f = ctypes.c_float
    return [a["hidden"], a["bsz"], a["hidden_dim"], a["out"], a["count"], a["count_len"], a["tok"], a["w"], a["n"],
            a["tsg"], a["tsu"], a["conc"], a["max_tok"], a["tig"], a["tiu"], a["I"], a["act"],
            f(a["Kg"]), f(a["Ku"]), f(a["Kd"]), *a["tables"], a["num_ptrs"], *a["cbs"], f(a["limit"]),
            a["num_active"], a["scratch"], a["scratch_rows"], a["scratch_cols"], a["fused_base"],
            a["lo"], a["hi"], a["m_tile"], *a["bits"], a["bits_len"], None]


def test_moe_sorted_rejects_bad_arguments():
    """exl3_moe's checks (exl3_moe.cu:186-323) in the reference's order and wording."""
    L = _lib.lib()
    assert L.exl3_amd_moe(*_moe_args(num_active=0, hidden=None)) == 0       # nothing to do: returns first
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(scratch=1, scratch_cols=256))
    assert rc == _lib.EINVAL and "needs fused_base" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(scratch=1, scratch_cols=128, fused_base=1))
    assert rc == _lib.EINVAL and "[slots, hidden]" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(cbs=[1, 0, 0, 1, 1, 0]))
    assert rc == _lib.EINVAL and "same codebook" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(cbs=[0, 0, 0, 0, 0, 0]))
    assert rc == _lib.EINVAL and "Only mcg and mul1" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(Kg=2.5))
    assert rc == _lib.EINVAL and "half-integer" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(bits=[1, None, None], cbs=[0, 1, 0, 1, 0, 1]))
    assert rc == _lib.EINVAL and "all three" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(bits=[1, 1, 1], bits_len=8))
    assert rc == _lib.EINVAL and "mul1" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(num_ptrs=7))
    assert rc == _lib.EINVAL and "num_experts" in msg
    rc, msg = call_err(L.exl3_amd_moe, *_moe_args(n=9))
    assert rc == _lib.EINVAL and "bsz" in msg


def test_moe_gather_rejects_bad_arguments():
    L = _lib.lib()
    rc, msg = call_err(L.exl3_amd_moe_gather, 1, 4, 256, 1, 128, 1, 8, 1, 1, 4, 1, 4, 1, 4, 1, None)
    assert rc == _lib.EINVAL and "[slots, hidden]" in msg
    rc, msg = call_err(L.exl3_amd_moe_gather, 1, 4, 256, 1, 256, 1, 9, 1, 1, 4, 1, 4, 1, 4, 1, None)
    assert rc == _lib.EINVAL and "assignments / tokens" in msg
    rc, msg = call_err(L.exl3_amd_moe_gather, 1, 4, 256, 1, 256, 1, 8, 1, 1, 3, 1, 4, 1, 4, 1, None)
    assert rc == _lib.EINVAL and "table sizes" in msg
    rc, msg = call_err(L.exl3_amd_moe_gather, 1, 1, 256, 1, 256, 1, 33, 1, 1, 4, 1, 4, 1, 4, 1, None)
    assert rc == _lib.EINVAL and "top-k" in msg
    assert L.exl3_amd_moe_gather(1, 0, 256, 1, 256, 1, 0, 1, 1, 4, 1, 4, 1, 4, 1, None) == 0


def test_decode_neighbours_reject_bad_arguments():
    """rms_norm_res's checks (amp_torch.cpp:10106-10131: last dim a multiple of 4, 8-byte
    aligned operands), silu_mul's null check, and exl3_gemm's shape checks in the fused entry
    points, all before any device access."""
    L = _lib.lib()
    f = ctypes.c_float
    rc, msg = call_err(L.exl3_amd_rms_norm_res, 8, 8, 8, 8, 8, 1, 130, f(1e-5), None)
    assert rc == _lib.EINVAL and "multiple of 4" in msg
    rc, msg = call_err(L.exl3_amd_rms_norm_res, 8, 12, 8, 8, 8, 1, 128, f(1e-5), None)
    assert rc == _lib.EINVAL and "8-byte aligned" in msg
    rc, msg = call_err(L.exl3_amd_rms_norm_res, None, 8, 8, 8, 8, 1, 128, f(1e-5), None)
    assert rc == _lib.EINVAL and "null" in msg
    assert L.exl3_amd_rms_norm_res(None, None, None, None, None, 0, 128, f(1e-5), None) == 0
    rc, msg = call_err(L.exl3_amd_silu_mul, None, 8, 8, 16, None)
    assert rc == _lib.EINVAL and "null" in msg
    assert L.exl3_amd_silu_mul(None, None, None, 0, None) == 0
    rc, msg = call_err(L.exl3_amd_gemm_silu_mul, 8, 8, 8, 8, 8, 0, None, None, None, 1, 128, 100, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "n must" in msg
    rc, msg = call_err(L.exl3_amd_gemm_silu_mul, 8, 8, 8, 8, 8, 0, None, None, None, 1, 136, 128, f(4.0), 0, 0, None)
    assert rc == _lib.EINVAL and "k must" in msg
    rc, msg = call_err(L.exl3_amd_gemm_silu_mul, 8, 8, 8, 8, 8, 0, None, None, None, 1, 128, 128, f(9.0), 0, 0, None)
    assert rc == _lib.EINVAL and "bitrate" in msg
    rc, msg = call_err(L.exl3_amd_gemm_norm, 16, None, None, 16, 16, None, None, None, 1, 128, 128, f(4.0), 0, 0,
                       16, 16, 8, f(1e-5), None)
    assert rc == _lib.EINVAL and "16-byte aligned" in msg
    rc, msg = call_err(L.exl3_amd_gemm_norm, 16, 16, None, 16, 16, None, None, None, 1, 128, 128, f(4.0), 0, 0,
                       16, 16, 16, f(1e-5), None)
    assert rc == _lib.EINVAL and "null" in msg
    rc, msg = call_err(L.exl3_amd_gemm_norm, 16, None, None, 16, 16, None, None, None, 1, 128, 120, f(4.0), 0, 0,
                       16, 16, 16, f(1e-5), None)
    assert rc == _lib.EINVAL and "n must" in msg


def test_header_constants_match_python():
    """Every integer constant _lib.py mirrors (return codes, tags, policy keys and values) has the
    value include/exl3_amd.h defines, and every policy key of the header has a Python name."""
    import re
    from ampstein_amd import _lib
    defs = {}
    for line in open(_lib.HEADER):
        m = re.match(r"#define\s+EXL3_AMD_(\w+)\s+(-?\d+)\b", line)
        if m:
            defs[m.group(1)] = int(m.group(2))
    assert defs, "no constants parsed from the header"
    checked = 0
    for name, val in vars(_lib).items():
        if name.isupper() and isinstance(val, int) and not isinstance(val, bool) and name in defs:
            assert defs[name] == val, (name, defs[name], val)
            checked += 1
    keys = [n for n in defs if n.startswith("POLICY_") and n != "POLICY_COUNT"]
    assert len(keys) == defs["POLICY_COUNT"]
    for n in keys:
        assert hasattr(_lib, n), f"no Python name for EXL3_AMD_{n}"
    assert checked >= len(keys)
