"""The at::Tensor adapter (adapter/exl3_amd_adapter.cpp) as a Python module.

`load()` returns the compiled module `exl3_amd_torch`, whose functions take the arguments of
the global C++ operators that ampstein's torch bindings call (amp_torch.cpp:3739-3896,
:11062-11081): exl3_gemm, exl3_mgemm, reconstruct, reconstruct_had_slice, had_r_128,
exl3_moe_coop.  Built in-tree by ampstein_amd.build; there is no fallback.
"""
from __future__ import annotations

import importlib.util
import os

from ampstein_amd import _lib, build

_mod = None


def load():
    global _mod
    if _mod is None:
        import torch  # noqa: F401  (the module links against torch's libraries)
        _lib.lib()    # libexl3_amd.so first, under torch's HIP runtime
        path = build.adapter_path()
        if not os.path.exists(path):
            raise ImportError(f"{path} is not built: run python -m ampstein_amd.build")
        spec = importlib.util.spec_from_file_location("exl3_amd_torch", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _mod = mod
    return _mod
