"""numpy front end of the CPU oracle (liboracle_exl3.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load this module as the checker; the product path
(ampstein_amd) never imports it.

Arrays of IEEE binary16 values are passed as numpy float16 (bit patterns are
identical to the reference's `half`).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_exl3.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_moe_mul1.so")

_lib = None


def build(force: bool = False) -> None:
    """Compile liboracle_exl3.so with oracle/Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", HERE, "-B" if force else "all", "liboracle_exl3.so"],
                       check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.exl3o_decode.restype = ctypes.c_uint16
        L.exl3o_decode.argtypes = [ctypes.c_uint32, i32]
        L.exl3o_state.restype = ctypes.c_uint32
        L.exl3o_state.argtypes = [vp, i32, i32, i32]
        for name in ("exl3o_hadd", "exl3o_hsub", "exl3o_hmul"):
            getattr(L, name).restype = ctypes.c_uint16
            getattr(L, name).argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.exl3o_hfma.restype = ctypes.c_uint16
        L.exl3o_hfma.argtypes = [ctypes.c_uint16] * 3
        L.exl3o_h_from_f64.restype = ctypes.c_uint16
        L.exl3o_h_from_f64.argtypes = [ctypes.c_double]
        L.exl3o_h_from_f32.restype = ctypes.c_uint16
        L.exl3o_h_from_f32.argtypes = [f32]
        L.exl3o_tile_perm.argtypes = [vp]
        L.exl3o_bits_from_K.argtypes = [f32, vp, vp]
        L.exl3o_reconstruct.argtypes = [vp, vp, i32, i32, i32, i32, i32, i32, i32, i32]
        L.exl3o_reconstruct_had.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32]
        L.exl3o_had_transform.argtypes = [vp, vp, vp, vp, i32, i32, i32]
        L.exl3o_had128_hf.argtypes = [vp, vp, i32, i32, vp, vp, f32]
        L.exl3o_had128_ff.argtypes = [vp, vp, i32, i32, vp, vp, f32]
        L.exl3o_had128_fh.argtypes = [vp, vp, i32, i32, vp, f32]
        L.exl3o_fwht128_f32.argtypes = [vp]
        L.exl3o_linear.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32]
        L.exl3o_linear_f64.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32]
        L.exl3o_matmul_h.argtypes = [vp, vp, vp, i32, i32, i32, i32]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _threads(n):
    return n if n else min(16, os.cpu_count() or 1)


def bits_from_K(K: float):
    b, h = ctypes.c_int(), ctypes.c_int()
    if lib().exl3o_bits_from_K(float(K), ctypes.byref(b), ctypes.byref(h)):
        raise ValueError(f"Unsupported EXL3 bitrate {K}")
    return b.value, bool(h.value)


def tile_u16(bits: int, half: bool) -> int:
    return 16 * bits + (8 if half else 0)


def decode(state: int, cb: int) -> int:
    return lib().exl3o_decode(state, cb)


def decode_all(cb: int) -> np.ndarray:
    """fp16 codebook value of every 16-bit state (uint16 bit patterns)."""
    return np.array([lib().exl3o_decode(s, cb) for s in range(65536)], dtype=np.uint16)


def state(tile: np.ndarray, bits: int, half: bool, t: int) -> int:
    tile = np.ascontiguousarray(tile, dtype=np.uint16)
    return lib().exl3o_state(_p(tile), bits, int(half), t)


def tile_perm() -> np.ndarray:
    p = np.zeros(256, np.uint16)
    lib().exl3o_tile_perm(_p(p))
    return p


def _check_trellis(trellis, bits, half):
    trellis = np.ascontiguousarray(trellis, dtype=np.uint16)
    assert trellis.ndim == 3 and trellis.shape[2] == tile_u16(bits, half), trellis.shape
    return trellis


def reconstruct(trellis, bits, half=False, cb=0, n=None, n_offset=0, nthreads=0):
    trellis = _check_trellis(trellis, bits, half)
    k, n_packed = trellis.shape[0] * 16, trellis.shape[1] * 16
    n = n_packed - n_offset if n is None else n
    W = np.empty((k, n), np.float16)
    rc = lib().exl3o_reconstruct(_p(W), _p(trellis), k, n, n_packed, n_offset, bits, int(half),
                                 cb, _threads(nthreads))
    if rc:
        raise ValueError("reconstruct: bad arguments")
    return W


def reconstruct_had(trellis, suh, svh, bits, half=False, cb=0, n=None, n_offset=0, nthreads=0):
    trellis = _check_trellis(trellis, bits, half)
    k, n_packed = trellis.shape[0] * 16, trellis.shape[1] * 16
    n = n_packed - n_offset if n is None else n
    suh = np.ascontiguousarray(suh, np.float16)
    svh = np.ascontiguousarray(svh, np.float16)
    W = np.empty((k, n), np.float16)
    rc = lib().exl3o_reconstruct_had(_p(W), _p(trellis), _p(suh), _p(svh), k, n, n_packed,
                                     n_offset, bits, int(half), cb, _threads(nthreads))
    if rc:
        raise ValueError("reconstruct_had: bad arguments")
    return W


def had_transform(W_hat, suh, svh, nthreads=0):
    """reconstruct_had's per-block transform on a given fp16 W_hat (k, n)."""
    W_hat = np.ascontiguousarray(W_hat, np.float16)
    k, n = W_hat.shape
    W = np.empty((k, n), np.float16)
    rc = lib().exl3o_had_transform(_p(W), _p(W_hat), _p(np.ascontiguousarray(suh, np.float16)),
                                   _p(np.ascontiguousarray(svh, np.float16)), k, n, _threads(nthreads))
    if rc:
        raise ValueError("had_transform: bad arguments")
    return W


def had128(x, pre=None, post=None, scale=1.0):
    """had_r_128 semantics: fp16 -> fp16 (half path) or fp32 -> fp32 (float path)."""
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    pre = None if pre is None else np.ascontiguousarray(pre, np.float16)
    post = None if post is None else np.ascontiguousarray(post, np.float16)
    if x.dtype == np.float16:
        y = np.empty_like(x)
        lib().exl3o_had128_hf(_p(x), _p(y), rows, cols, _p(pre), _p(post), scale)
    elif x.dtype == np.float32:
        y = np.empty_like(x)
        lib().exl3o_had128_ff(_p(x), _p(y), rows, cols, _p(pre), _p(post), scale)
    else:
        raise TypeError(x.dtype)
    return y


def had128_fh(x, post=None, scale=1.0):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    post = None if post is None else np.ascontiguousarray(post, np.float16)
    y = np.empty((rows, cols), np.float16)
    lib().exl3o_had128_fh(_p(x), _p(y), rows, cols, _p(post), scale)
    return y


def fwht128_f32(v):
    v = np.ascontiguousarray(v, np.float32).copy()
    assert v.shape == (128,)
    lib().exl3o_fwht128_f32(_p(v))
    return v


def linear(x, trellis, suh, svh, bits, half=False, cb=0, y_fp32=False, nthreads=0):
    """Reference EXL3 linear (exl3_gemm semantics), fp64 accumulation."""
    x = np.ascontiguousarray(x, np.float16)
    trellis = _check_trellis(trellis, bits, half)
    m, k = x.shape
    n = trellis.shape[1] * 16
    assert trellis.shape[0] * 16 == k
    suh = None if suh is None else np.ascontiguousarray(suh, np.float16)
    svh = None if svh is None else np.ascontiguousarray(svh, np.float16)
    y = np.empty((m, n), np.float32 if y_fp32 else np.float16)
    rc = lib().exl3o_linear(_p(x), _p(trellis), _p(suh), _p(svh), _p(y), m, k, n, bits,
                            int(half), cb, int(y_fp32), _threads(nthreads))
    if rc:
        raise ValueError("linear: bad arguments")
    return y


def linear_f64(x, trellis, suh, svh, bits, half=False, cb=0, nthreads=0):
    x = np.ascontiguousarray(x, np.float16)
    trellis = _check_trellis(trellis, bits, half)
    m, k = x.shape
    n = trellis.shape[1] * 16
    suh = None if suh is None else np.ascontiguousarray(suh, np.float16)
    svh = None if svh is None else np.ascontiguousarray(svh, np.float16)
    y = np.empty((m, n), np.float64)
    rc = lib().exl3o_linear_f64(_p(x), _p(trellis), _p(suh), _p(svh), _p(y), m, k, n, bits,
                                int(half), cb, _threads(nthreads))
    if rc:
        raise ValueError("linear_f64: bad arguments")
    return y


def matmul_h(x, W, nthreads=0):
    x = np.ascontiguousarray(x, np.float16)
    W = np.ascontiguousarray(W, np.float16)
    m, k = x.shape
    n = W.shape[1]
    y = np.empty((m, n), np.float32)
    lib().exl3o_matmul_h(_p(x), _p(W), _p(y), m, k, n, _threads(nthreads))
    return y


def ref_lib():
    """The reference's own cpu/moe_mul1.cpp helpers (oracle/_ref), or None when not built."""
    if not os.path.exists(REF_LIB_PATH):
        return None
    import torch  # noqa: F401  (the shim links libtorch_cpu; load torch's copy first)
    L = ctypes.CDLL(REF_LIB_PATH)
    L.ref_decode_state.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    L.ref_window_end.argtypes = [ctypes.c_int, ctypes.c_int]
    L.ref_tc_perm.argtypes = [ctypes.c_void_p]
    L.ref_hadamard_128_scalar.argtypes = [ctypes.c_void_p]
    L.ref_decode_mul1_scalar.restype = ctypes.c_float
    L.ref_decode_mul1_scalar.argtypes = [ctypes.c_uint16]
    return L
