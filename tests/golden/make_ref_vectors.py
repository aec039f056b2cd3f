"""Write tests/golden/ref_moe_mul1_vectors.npz from the reference's own CPU code.

Runs only in the build container, where /root/reference exists and
oracle/_ref/libref_moe_mul1.so has been compiled from the reference source
vendor/exl3/exllamav3_ext/cpu/moe_mul1.cpp (see oracle/Makefile, target `ref`).
The vectors are data (inputs and the reference's outputs):

  tc_perm            make_tc_perm()                      moe_mul1.cpp:125-139
  state_tiles_K{b}   random packed tiles, K = 1..8       (inputs)
  state_K{b}         decode_state_scalar<K>(tile, t)     moe_mul1.cpp:190-200
  window_end_half25  window_end<HALF25>(t), t = 0..255   moe_mul1.cpp:78-83
  had_in / had_out   hadamard_128_scalar(v)              moe_mul1.cpp:223-237
  mul1_f32           decode_mul1_scalar(s), all s        moe_mul1.cpp:202-207

and tests/golden/ref_moe_cpu_forward.npz from the reference's CPU MoE forward
(exl3_moe_cpu_make_layer + exl3_moe_cpu_forward_raw, moe_mul1.cpp:2418-2654) on its scalar
tier (EXL3_MOE_CPU_MAX_ISA=scalar: fp32 activations, no int8 quantization), through the
shim's ref_moe_forward:

  E, H, I, bits, trellis_{e}_{p}, suh_{e}_{p}, svh_{e}_{p}, bias_{e}_{p}   4 mul1 experts (inputs)
  x, sel, w                                                                 routed rows (inputs)
  out_{case}    fp32 output per case (activation, limit, gated, bias)       moe_mul1.cpp:2169-2214

Usage: python tests/golden/make_ref_vectors.py
"""
import ctypes
import os
import sys

import numpy as np

# The reference's CPU MoE picks its kernel tier when the library loads: cap it at the scalar tier
os.environ["EXL3_MOE_CPU_MAX_ISA"] = "scalar"

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_moe_mul1.so not built (make -C oracle ref)")
    vp = ctypes.c_void_p
    out = {}
    p = np.zeros(256, np.uint16)
    ref.ref_tc_perm(p.ctypes.data_as(vp))
    out["tc_perm"] = p
    rng = np.random.default_rng(20261201)
    for b in range(1, 9):
        tiles = rng.integers(0, 65536, size=(4, 16 * b), dtype=np.uint16)
        st = np.zeros((4, 256), np.uint16)
        for i in range(4):
            for t in range(256):
                st[i, t] = ref.ref_decode_state(b, tiles[i].ctypes.data_as(vp), t)
        out[f"state_tiles_K{b}"] = tiles
        out[f"state_K{b}"] = st
    out["window_end_half25"] = np.array([ref.ref_window_end(25, t) for t in range(256)], np.int32)
    had_in = (rng.standard_normal((16, 128)) * rng.choice([1e-3, 1.0, 100.0], (16, 1))).astype(np.float32)
    had_out = had_in.copy()
    for i in range(16):
        row = np.ascontiguousarray(had_out[i])
        ref.ref_hadamard_128_scalar(row.ctypes.data_as(vp))
        had_out[i] = row
    out["had_in"], out["had_out"] = had_in, had_out
    out["mul1_f32"] = np.array([ref.ref_decode_mul1_scalar(s) for s in range(65536)], np.float32)
    np.savez_compressed(os.path.join(HERE, "ref_moe_mul1_vectors.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_moe_mul1_vectors.npz"))


MOE_CASES = {           # name: (activation, limit, gated, bias)
    "silu": (0, 0.0, True, False),
    "silu_limit": (0, 10.0, True, False),
    "gelu": (1, 0.0, True, False),
    "swiglu_oai": (3, 7.0, True, False),
    "relu2": (2, 0.0, False, False),
    "silu_bias": (0, 0.0, True, True),
}


def moe_cpu_forward():
    ref = oracle.ref_lib()
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    ref.ref_moe_forward.argtypes = [i32, i32, i32, vp, i32, vp, vp, vp, vp, i32, ctypes.c_float,
                                    vp, vp, vp, vp, i32, i32]
    rng = np.random.default_rng(20261202)
    E, H, I, rows, topk = 4, 256, 128, 6, 2
    bits = np.array([2, 3, 4, 2], np.int32)
    out = {"E": np.int32(E), "H": np.int32(H), "I": np.int32(I), "bits": bits}
    mats = {}
    for e in range(E):
        for p, (k, n) in enumerate(((H, I), (H, I), (I, H))):
            mats[f"trellis_{e}_{p}"] = rng.integers(0, 65536, (k // 16, n // 16, 16 * int(bits[e])), dtype=np.uint16)
            mats[f"suh_{e}_{p}"] = rng.choice([-1.0, 1.0], k).astype(np.float16)
            mats[f"svh_{e}_{p}"] = rng.choice([-1.0, 1.0], n).astype(np.float16)
            mats[f"bias_{e}_{p}"] = (rng.standard_normal(n) * 0.1).astype(np.float16)
    out.update(mats)
    x = rng.standard_normal((rows, H)).astype(np.float16)
    sel = np.array([[0, 1], [2, 3], [1, 1], [3, 0], [2, 2], [0, 3]], np.int32)
    w = rng.uniform(0.1, 1.0, (rows, topk)).astype(np.float16)
    w[4, 1] = 0.0                                      # a zero routing weight
    out.update(x=x, sel=sel, w=w)
    P = lambda name: (ctypes.c_void_p * (3 * E))(*[mats[f"{name}_{q // 3}_{q % 3}"].ctypes.data for q in range(3 * E)])
    for case, (act, limit, gated, bias) in MOE_CASES.items():
        y = np.zeros((rows, H), np.float32)
        rc = ref.ref_moe_forward(E, H, I, bits.ctypes.data, int(gated), P("trellis"), P("suh"), P("svh"),
                                 P("bias") if bias else None, act, limit, x.ctypes.data, sel.ctypes.data,
                                 w.ctypes.data, y.ctypes.data, rows, topk)
        if rc:
            raise SystemExit(f"ref_moe_forward rejected case {case}")
        out[f"out_{case}"] = y
    np.savez_compressed(os.path.join(HERE, "ref_moe_cpu_forward.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_moe_cpu_forward.npz"))


if __name__ == "__main__":
    main()
    moe_cpu_forward()
