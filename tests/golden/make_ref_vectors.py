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

Usage: python tests/golden/make_ref_vectors.py
"""
import ctypes
import os
import sys

import numpy as np

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


if __name__ == "__main__":
    main()
