"""Builds libapplegpu_core.so (C++ runtime + gfx950 HIP kernels) in-tree.

Every source is compiled by hipcc for --offload-arch=gfx950 into
applegpu-runtime_amd/_build/, then linked into
applegpu-runtime_amd/applegpu_runtime/libapplegpu_core.so, where the Python
package and the tests load it from.

Usage: python applegpu-runtime_amd/build.py [-j N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "applegpu_runtime", "libapplegpu_core.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-fp32 VALU ops are disabled for all device code (hipcc flag; the
# host pass warns that it does not know the feature, which is harmless).
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-command-line-argument",
]


def sources() -> list[str]:
    out = []
    for root, _, files in os.walk(CSRC):
        for f in sorted(files):
            if f.endswith((".cpp", ".hip")):
                out.append(os.path.join(root, f))
    return sorted(out)


def obj_for(src: str) -> str:
    rel = os.path.relpath(src, CSRC).replace(os.sep, "_")
    return os.path.join(BUILD, rel + ".o")


def compile_one(src: str) -> tuple[str, int, str]:
    obj = obj_for(src)
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if "packed-fp32-ops" not in l)
    return src, p.returncode, msg


def stale(src: str) -> bool:
    """True when the object is missing or older than its source or any header
    under csrc/ (a conservative stand-in for dependency tracking)."""
    obj = obj_for(src)
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    if os.path.getmtime(src) > t:
        return True
    for root, _, files in os.walk(CSRC):
        for f in files:
            if f.endswith(".hpp") and os.path.getmtime(os.path.join(root, f)) > t:
                return True
    return False


def build(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    todo = [s for s in srcs if stale(s)] if incremental else srcs
    jobs = jobs or min(8, os.cpu_count() or 4)
    failed = []
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, rc, msg in ex.map(compile_one, todo):
            if msg.strip() and (rc != 0 or verbose):
                print(f"--- {os.path.relpath(src, HERE)}\n{msg}", file=sys.stderr)
            if rc != 0:
                failed.append(src)
    if failed:
        raise RuntimeError("compile failed: " + ", ".join(os.path.relpath(f, HERE) for f in failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *[obj_for(s) for s in srcs]]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stdout + p.stderr)
    shutil.move(tmp, LIB)
    return LIB


SHIM_SRC = os.path.join(HERE, "torch_shim", "applegpu_backend.cpp")
SHIM_LIB = os.path.join(HERE, "applegpu_runtime", "applegpu_backend.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def build_torch_shim(verbose: bool = True) -> str:
    """Builds the PrivateUse1 torch extension (plain C++ against the installed
    PyTorch; it calls only the C ABI of libapplegpu_core.so, found through
    $ORIGIN next to it)."""
    import torch
    from torch.utils import cpp_extension as ce
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", SHIM_SRC, "-o", SHIM_LIB + ".tmp",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-I{INCLUDE}", "-w"]
    cmd += [f"-I{p}" for p in ce.include_paths()]
    cmd += [f"-L{p}" for p in ce.library_paths()] + ["-lc10", "-ltorch", "-ltorch_cpu"]
    cmd += [f"-L{os.path.dirname(LIB)}", "-lapplegpu_core", "-Wl,-rpath,$ORIGIN"]
    cmd += [f"-Wl,-rpath,{p}" for p in ce.library_paths()]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("torch shim build failed:\n" + p.stdout + p.stderr)
    if verbose and (p.stdout or p.stderr).strip():
        print(p.stdout + p.stderr, file=sys.stderr)
    shutil.move(SHIM_LIB + ".tmp", SHIM_LIB)
    return SHIM_LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only sources older than their object (or than any header)")
    a = ap.parse_args()
    print(build(a.j, incremental=a.incremental))
    print(build_torch_shim())
