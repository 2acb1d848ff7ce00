"""The C-ABI library loads and exports every symbol include/applegpu_ffi.h
declares; no compute call is made (runs on the CPU)."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "applegpu_ffi.h")
LIB = os.path.join(ROOT, "applegpu-runtime_amd", "applegpu_runtime", "libapplegpu_core.so")
REF_SURFACE = [  # backend_cpp/applegpu_ffi.h:11-92 of the reference
    "applegpu_ffi_init", "applegpu_ffi_last_error", "applegpu_ffi_alloc", "applegpu_ffi_free",
    "applegpu_ffi_register_tensor", "applegpu_ffi_shape", "applegpu_ffi_dtype", "applegpu_ffi_add",
    "applegpu_ffi_matmul", "applegpu_ffi_relu", "applegpu_ffi_mul", "applegpu_ffi_sub", "applegpu_ffi_neg",
    "applegpu_ffi_copy", "applegpu_ffi_add_out", "applegpu_ffi_mul_out", "applegpu_ffi_sub_out",
    "applegpu_ffi_matmul_out", "applegpu_ffi_relu_out", "applegpu_ffi_neg_out", "applegpu_ffi_div_out",
    "applegpu_ffi_threshold_backward_out", "applegpu_ffi_scalar_mul_out", "applegpu_ffi_mean_all_out",
    "applegpu_ffi_eval", "applegpu_ffi_synchronize", "applegpu_ffi_read_f32", "applegpu_eager_init",
    "applegpu_eager_last_error", "applegpu_eager_alloc", "applegpu_eager_free", "applegpu_eager_register_shape",
    "applegpu_eager_shape", "applegpu_eager_dtype", "applegpu_eager_add", "applegpu_eager_sub",
    "applegpu_eager_mul", "applegpu_eager_div", "applegpu_eager_relu", "applegpu_eager_neg",
    "applegpu_eager_matmul", "applegpu_eager_matmul_ex", "applegpu_eager_threshold_backward",
    "applegpu_eager_scalar_mul", "applegpu_eager_mean_all", "applegpu_eager_sum_dim", "applegpu_eager_create_view",
    "applegpu_eager_add_inplace", "applegpu_eager_add_scaled_inplace", "applegpu_eager_flush_and_wait",
    "applegpu_eager_synchronize", "applegpu_eager_embedding", "applegpu_eager_layer_norm", "applegpu_eager_gelu",
    "applegpu_eager_softmax", "applegpu_eager_find_by_data_ptr", "applegpu_eager_execute_graph",
]


def declared():
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(applegpu_\w+)\s*\(", text)))


def exported():
    out = subprocess.check_output(["nm", "-D", "--defined-only", LIB], text=True)
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_library_built():
    assert os.path.exists(LIB), "run `python applegpu-runtime_amd/build.py`"


def test_every_declared_symbol_is_exported():
    missing = [s for s in declared() if s not in exported()]
    assert not missing, missing


def test_reference_surface_is_declared():
    d = set(declared())
    assert [s for s in REF_SURFACE if s not in d] == []


def test_library_loads_and_binds():
    lib = ctypes.CDLL(LIB)
    for s in declared():
        getattr(lib, s)


def test_python_binding_covers_header():
    import applegpu_runtime._native as nat
    assert sorted(nat.EXPORTED) == declared()


def test_library_is_gfx950_code():
    # the code object embedded in the library targets gfx950 (hipcc --offload-arch=gfx950)
    blob = open(LIB, "rb").read()
    assert b"gfx950" in blob


def _gpu_visible():
    return os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK)


def test_init_without_gpu_reports_an_error():
    """With no GPU the runtime refuses to start and says why (no CPU fallback);
    run in a child process so this process never touches HIP."""
    code = (
        "import ctypes,sys; lib=ctypes.CDLL(sys.argv[1]);"
        "lib.applegpu_eager_init.restype=ctypes.c_bool;"
        "lib.applegpu_eager_last_error.restype=ctypes.c_char_p;"
        "ok=lib.applegpu_eager_init(); e=lib.applegpu_eager_last_error();"
        "print('OK' if ok else 'ERR:'+(e or b'').decode())"
    )
    out = subprocess.run(["python", "-c", code, LIB], capture_output=True, text=True, timeout=120).stdout.strip()
    if _gpu_visible():
        assert out == "OK", out
    else:
        assert out.startswith("ERR:") and "device" in out.lower(), out


def test_execute_graph_reports_missing_device():
    code = (
        "import ctypes,sys; lib=ctypes.CDLL(sys.argv[1]);"
        "lib.applegpu_eager_last_error.restype=ctypes.c_char_p;"
        "r=lib.applegpu_eager_execute_graph(None,0,None,0,None,0,None,None);"
        "print(r, lib.applegpu_eager_last_error().decode())"
    )
    out = subprocess.run(["python", "-c", code, LIB], capture_output=True, text=True, timeout=120).stdout.strip()
    if not _gpu_visible():
        assert out.startswith("-1") and "device" in out, out
