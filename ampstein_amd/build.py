"""Build libexl3_amd.so (HIP, gfx950) in-tree: ampstein_amd/lib/libexl3_amd.so.

    python -m ampstein_amd.build [-j N]

Each kernel unit is compiled separately with hipcc (the GEMV once per bitrate K) and the
objects are linked into one shared library exporting the C ABI of include/exl3_amd.h.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libexl3_amd.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # packed fp32 ops stay off on this pool; every fp32 / fp16 operation rounds once
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=off", "-fno-fast-math",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
    f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
]


def units():
    u = [
        ("exl3_capi.cpp", "exl3_capi.o", []),
        ("exl3_reconstruct.hip", "exl3_reconstruct.o", []),
        ("exl3_hadamard.hip", "exl3_hadamard.o", []),
        ("exl3_device.hip", "exl3_device.o", []),
        ("exl3_moe_sorted.hip", "exl3_moe_sorted.o", []),
        ("exl3_decode_ops.hip", "exl3_decode_ops.o", []),
        ("exl3_dense.hip", "exl3_dense.o", []),
    ]
    for cb in range(3):
        u.append(("exl3_moe.hip", f"exl3_moe_cb{cb}.o", [f"-DEXL3_MOE_CB={cb}"]))
    for k in range(1, 9):
        u.append(("exl3_gemv.hip", f"exl3_gemv_k{k}.o", [f"-DEXL3_INST_K={k}"]))
        u.append(("exl3_gemm.hip", f"exl3_gemm_k{k}.o", [f"-DEXL3_INST_K={k}"]))
    for k in (17, 18, 19):       # half rates 1.5 / 2.5 / 3.5 (rate code 16 + b, mul1 only)
        u.append(("exl3_gemv.hip", f"exl3_gemv_k{k}.o", [f"-DEXL3_INST_K={k}"]))
        u.append(("exl3_gemm.hip", f"exl3_gemm_k{k}.o", [f"-DEXL3_INST_K={k}"]))
    return u


def _compile(src, obj, extra):
    cmd = [HIPCC] + COMMON + extra + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", os.path.join(OBJ, obj)]
    t0 = time.time()
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src} {extra}:\n{p.stderr[-6000:]}")
    return obj, time.time() - t0


def _stale(src: str, obj: str) -> bool:
    """True when the object is missing or older than its source or any shared header."""
    o = os.path.join(OBJ, obj)
    if not os.path.exists(o):
        return True
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, f) for f in os.listdir(CSRC)
                                        if f.endswith((".h", ".cuh"))]
    deps.append(os.path.join(ROOT, "include", "exl3_amd.h"))
    return max(os.path.getmtime(d) for d in deps) > os.path.getmtime(o)


def build(jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> str:
    """Compile every unit (incremental: only units whose object is stale) and link."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    todo = [u for u in units() if not incremental or _stale(u[0], u[1])]
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_compile, *u) for u in todo]
        for f in cf.as_completed(futs):
            obj, dt = f.result()
            if verbose:
                print(f"  {obj}: {dt:.1f}s", flush=True)
    objs = [os.path.join(OBJ, o) for _, o, _ in units()]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr[-6000:]}")
    shutil.move(tmp, LIB)
    return LIB


PROBE_LIB = os.path.join(LIB_DIR, "libexl3_probe.so")


def build_probe(verbose: bool = False) -> str:
    """Issue-rate microbenchmarks (csrc/exl3_probe.hip) for `bench.py --rates`: a library of its
    own, not part of the C ABI."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = PROBE_LIB + ".tmp"
    cmd = [HIPCC] + COMMON + ["-shared", "-x", "hip", os.path.join(CSRC, "exl3_probe.hip"), "-o", tmp]
    t0 = time.time()
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{p.stderr[-6000:]}")
    shutil.move(tmp, PROBE_LIB)
    if verbose:
        print(f"  libexl3_probe.so: {time.time() - t0:.1f}s", flush=True)
    return PROBE_LIB


ADAPTER_DIR = os.path.join(PKG, "adapter")


def adapter_path() -> str:
    import sysconfig
    return os.path.join(LIB_DIR, "exl3_amd_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_adapter(verbose: bool = False) -> str:
    """The at::Tensor adapter (adapter/exl3_amd_adapter.cpp) and its Python module: host-only
    C++ (no device code) built by the host compiler against torch's ROCm headers, linked to
    libexl3_amd.so (rpath $ORIGIN).  __HIP_PLATFORM_AMD__ is the define hipcc itself passes;
    the HIP runtime headers that torch's headers include need it."""
    import sysconfig
    from torch.utils import cpp_extension as ce
    out = adapter_path()
    inc = ce.include_paths(device_type="cuda") + [sysconfig.get_paths()["include"], ADAPTER_DIR,
                                                    os.path.join(ROOT, "include")]
    libdirs = ce.library_paths(device_type="cuda")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-fPIC", "-shared", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1",
           "-DTORCH_EXTENSION_NAME=exl3_amd_torch", "-D_GLIBCXX_USE_CXX11_ABI=1",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-DUSE_ROCM=1", "-w"]
    cmd += [f"-I{d}" for d in inc]
    cmd += [os.path.join(ADAPTER_DIR, "exl3_amd_adapter.cpp"), os.path.join(ADAPTER_DIR, "exl3_amd_torch.cpp")]
    cmd += [f"-L{d}" for d in libdirs] + [f"-L{LIB_DIR}", "-lexl3_amd", "-lc10", "-lc10_hip", "-ltorch",
                                          "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
                                          "-Wl,-rpath,$ORIGIN"]
    tmp = out + ".tmp"
    t0 = time.time()
    p = subprocess.run(cmd + ["-o", tmp], capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"adapter build failed:\n{p.stderr[-6000:]}")
    shutil.move(tmp, out)
    if verbose:
        print(f"  {os.path.basename(out)}: {time.time() - t0:.1f}s", flush=True)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--incremental", action="store_true", help="recompile stale units only; keep the adapter")
    args = ap.parse_args(argv)
    t0 = time.time()
    path = build(args.j, verbose=True, incremental=args.incremental)
    if not args.incremental or not os.path.exists(adapter_path()):
        build_adapter(verbose=True)
    build_probe(verbose=True)
    print(f"built {path} in {time.time() - t0:.1f}s")


if __name__ == "__main__":
    sys.exit(main())
