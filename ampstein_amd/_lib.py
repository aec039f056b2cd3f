"""ctypes binding of libexl3_amd.so (the C ABI declared in include/exl3_amd.h).

The library is built in-tree by ampstein_amd.build (or __graft_entry__.build()).  There is
no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libexl3_amd.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "exl3_amd.h")

OK, EINVAL, EUNSUPPORTED, EHIP, ENOMEM = 0, -1, -2, -3, -4
TAG_GEMV, TAG_GEMM = 90, 91

_lib = None

_vp, _i32, _f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "exl3_amd_last_error": (ctypes.c_char_p, []),
    "exl3_amd_version": (_i32, []),
    "exl3_amd_set_policy": (_i32, [_i32, _i32]),
    "exl3_amd_get_policy": (_i32, [_i32]),
    "exl3_amd_init": (_i32, [_i32]),
    "exl3_amd_debug_read_workspace": (_i32, [_i32, ctypes.c_int64, ctypes.c_int64, _vp]),
    "exl3_amd_debug_fill_workspace": (_i32, [_i32, _i32]),
    "exl3_amd_device_info": (_i32, [_i32, _vp, _vp]),
    "exl3_amd_xcd_status": (_i32, [_i32, _vp, _vp, _vp]),
    "exl3_amd_xcd_rearm": (_i32, [_i32]),
    "exl3_amd_debug_handoff_map": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "exl3_amd_reconstruct": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
    "exl3_amd_reconstruct_t": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
    "exl3_amd_reconstruct_t_had": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
    "exl3_amd_reconstruct_had": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
    "exl3_amd_reconstruct_had_t": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
    "exl3_amd_recon_mm": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp]),
    "exl3_amd_recon_mm_slabs": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "exl3_amd_reconstruct_t_slabs": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _vp]),
    "exl3_amd_to_slabs": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _f32, _vp]),
    "exl3_amd_had_r_128": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _f32, _vp]),
    "exl3_amd_gemm": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _vp]),
    "exl3_amd_gemm_noalloc": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _vp]),
    "exl3_amd_mgemm": (_i32, [_vp, _i32, _i32, _i32,             # A, bszm_in, m, k
                              _vp, _i32,                         # B table, num_B
                              _vp, _i32, _i32, _i32,             # C, bszm_out, n, c_fp32
                              _vp, _i32,                         # suh table, num_suh
                              _vp, ctypes.c_int64,               # A_had, numel
                              _vp, _i32,                         # svh table, num_svh
                              _vp, _i32,                         # indices, num_indices
                              _vp,                               # weights
                              _f32, _i32, _i32, _i32,            # K, force_shape_idx, mcg, mul1
                              _i32, _i32, _i32, _i32,            # min/max_index, force_num_sms, num_tokens
                              _vp, _vp, _i32,                    # size_n_list, c_ptrs, num_c_ptrs
                              _vp, _i32,                         # n_stride_list, entries
                              _vp, _i32, _i32,                   # had_src_list, entries, num_had_src
                              _vp]),
    "exl3_amd_moe_coop": (_i32, [_vp, _i32, _i32, _i32,                 # x, bsz, H, x_stride
                                 _vp, _vp, _i32,                         # sel, rw, topk
                                 _i32, _i32, _i32,                       # min/max expert, Hi
                                 _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,   # tables, n_local
                                 _vp, _vp, _vp,                          # bias tables
                                 _f32, _f32, _f32, _i32, _i32, _i32, _f32, _i32,      # Kg Ku Kd mcg mul1 act limit gated
                                 _vp, ctypes.c_int64, _vp, ctypes.c_int64,            # had_g, had_u
                                 _vp, _vp, ctypes.c_int64, _i32, _i32,               # gu_g, gu_u, numel, f32, I
                                 _vp, ctypes.c_int64, _vp, ctypes.c_int64, _i32,     # act_out, d_out, Ho
                                 _vp, ctypes.c_int64,                    # ctr
                                 _vp, _i32, _i32, _i32,                  # out, rows_max, H_out, stride
                                 _vp, _vp, _i32,                         # sh_out, sh_gate_w, n
                                 _vp, _vp, _vp,                          # bits tables
                                 _vp]),
    "exl3_amd_moe_max_concurrency": (_i32, [_i32]),
    "exl3_amd_rms_norm_res": (_i32, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, _i32, _f32, _vp]),
    "exl3_amd_silu_mul": (_i32, [_vp, _vp, _vp, ctypes.c_int64, _vp]),
    "exl3_amd_gemm_silu_mul": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp,
                                      _i32, _i32, _i32, _f32, _i32, _i32, _vp]),
    "exl3_amd_gemm_norm": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _i32, _i32, _i32, _f32, _i32, _i32, _vp, _vp, _vp, _f32, _vp]),
    "exl3_amd_gemm_res": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _i32, _i32, _i32, _f32, _i32, _i32, _vp, _vp, _vp]),
    "exl3_amd_res_sq": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "exl3_amd_norm_sq": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "exl3_amd_mgemm_norm_in": (_i32, [_vp, _i32, _i32, _i32,             # h, bszm_in, m, k
                                      _vp, _i32,                         # B table, num_B
                                      _vp, _i32, _i32, _i32,             # C, bszm_out, n, c_fp32
                                      _vp, _i32,                         # suh table, num_suh
                                      _vp, ctypes.c_int64,               # A_had, numel
                                      _vp, _i32,                         # svh table, num_svh
                                      _vp, _vp, _i32,                    # size_n_list, c_ptrs, num_c_ptrs
                                      _vp, _i32,                         # n_stride_list, num
                                      _vp, _i32, _i32,                   # had_src_list, num, num_had_src
                                      _f32, _i32, _i32,                  # K, mcg, mul1
                                      _vp, _vp, _f32, _vp,               # sq, w, eps, r
                                      _vp]),
    "exl3_amd_moe": (_i32, [_vp, _i32, _i32, _vp,                       # hidden, bsz, hidden_dim, output
                            _vp, _i32, _vp, _vp, _i32,                  # expert_count (+len), token/weight_sorted, n
                            _vp, _vp, _i32, _i32,                       # temp_state_g/u, concurrency, max_tokens
                            _vp, _vp, _i32,                             # temp_intermediate_g/u, intermediate_dim
                            _i32, _f32, _f32, _f32,                     # act, K gate/up/down
                            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,   # tables, num_ptrs
                            _i32, _i32, _i32, _i32, _i32, _i32,         # codebook flags
                            _f32, _i32,                                 # act_limit, num_active
                            _vp, ctypes.c_int64, _i32, _vp,             # output_scratch (rows, cols), fused_base
                            _i32, _i32, _i32,                           # count_lo, count_hi, m_tile
                            _vp, _vp, _vp, _i32,                        # bits tables, len
                            _vp]),
    "exl3_amd_moe_gather": (_i32, [_vp, _i32, _i32, _vp, _i32,          # out, tokens, hidden, scratch, cols
                                   _vp, _i32, _vp,                      # flat_expert, num_assign, inv_order
                                   _vp, _i32, _vp, _i32,                # expert_start (+len), slot_base (+len)
                                   _vp, _i32, _vp, _vp]),               # slot_kind, num_experts, weight_sorted
}


class Exl3Error(RuntimeError):
    """Raised when a C-ABI call returns a negative code (the reference raises c10::Error)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def lib():
    """Load libexl3_amd.so (torch first, so the process shares torch's HIP runtime)."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m ampstein_amd.build` "
                               "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


# Kernel-path policy keys and values (include/exl3_amd.h EXL3_AMD_POLICY_*): 0 = the library's
# own choice; the other values select alternative paths with the same results.
POLICY_GEMV_ROWS, GEMV_ROWS_LDS, GEMV_ROWS_MFMA_ALL = 0, 1, 2
POLICY_GEMM_STAGING, GEMM_STAGING_REGS, GEMM_STAGING_NO_SPLIT = 1, 1, 2
POLICY_MOE_GEMM, MOE_GEMM_LDS = 2, 1
POLICY_MOE_TILE_ROWS = 3
POLICY_MOE_OUTPUT, MOE_OUTPUT_ATOMIC = 4, 1
POLICY_RECON_MM, RECON_MM_8WAVES, RECON_MM_WHOLE_TILES, RECON_MM_GLOBAL_DMA, RECON_MM_NO_SPLIT = 5, 1, 2, 3, 5
POLICY_GEMV_SPLIT, GEMV_SPLIT_BALANCED = 6, 1
POLICY_GEMV_SLICES = 7
POLICY_XCD_FAKE = 8
POLICY_MOE_EPILOGUE, MOE_EPILOGUE_SERIAL = 9, 1


class policy:
    """Context manager: `with policy(POLICY_MOE_OUTPUT, MOE_OUTPUT_ATOMIC): ...` sets a kernel-path
    policy for the block and restores the previous value afterwards."""

    def __init__(self, key: int, value: int):
        self.key, self.value = key, value

    def __enter__(self):
        self.prev = check(lib().exl3_amd_get_policy(self.key))
        check(lib().exl3_amd_set_policy(self.key, self.value))
        return self

    def __exit__(self, *exc):
        check(lib().exl3_amd_set_policy(self.key, self.prev))
        return False


def check(rc: int) -> int:
    if rc < 0:
        raise Exl3Error(rc, lib().exl3_amd_last_error().decode())
    return rc


def xcd_status(device: int = 0):
    """(XCD count the init probe verified, count in use, alarms serviced) of the per-launch XCD
    hand-off check; synchronises the device."""
    vals = [ctypes.c_int(0) for _ in range(3)]
    check(lib().exl3_amd_xcd_status(device, *[ctypes.byref(v) for v in vals]))
    return tuple(v.value for v in vals)


def handoff_map(kind: int, xcd: int, p0: int, p1: int, p2: int, b: int):
    """The kernels' workgroup -> hand-off coordinates, computed on the host (exl3_amd_debug_handoff_map)."""
    out = (ctypes.c_int * 4)()
    check(lib().exl3_amd_debug_handoff_map(kind, xcd, p0, p1, p2, b, out))
    return tuple(out)
