"""PyTorch PrivateUse1 device `applegpu` on the MI355X backend.

Same entry point as the reference's loader (python/applegpu_runtime/
cpp_backend.py:53-85): `load_cpp_backend()` installs a `torch.applegpu`
module, loads the C++ extension (applegpu_backend.so, built in-tree by
applegpu-runtime_amd/build.py next to libapplegpu_core.so), renames
PrivateUse1 to "applegpu" and generates the `.applegpu()` tensor methods.

Usage:
    from applegpu_runtime.cpp_backend import load_cpp_backend
    load_cpp_backend()
    x = torch.randn(3, 3).to("applegpu")
"""
from __future__ import annotations

import ctypes
import os
import sys
import types

HERE = os.path.dirname(os.path.abspath(__file__))
BACKEND_LIB = os.path.join(HERE, "applegpu_backend.so")

_loaded = False


def _synchronize(device=None) -> None:
    from ._native import lib
    lib.applegpu_eager_flush_and_wait()


def load_cpp_backend() -> None:
    """Registers the `applegpu` device with PyTorch (idempotent).  Raises
    ImportError when the extension is not built and RuntimeError when no
    MI355X is available: there is no silent CPU fallback."""
    global _loaded
    if _loaded:
        return
    if not os.path.exists(BACKEND_LIB):
        raise ImportError(f"applegpu_backend.so not found at {BACKEND_LIB}; build it with "
                          "`python applegpu-runtime_amd/build.py`")
    import torch

    mod = types.ModuleType("torch.applegpu")
    mod.device_count = lambda: 1
    mod.is_available = lambda: True
    mod.current_device = lambda: 0
    mod.set_device = lambda d: None
    mod.synchronize = _synchronize
    mod._exchange_device = lambda d: 0
    mod._maybe_exchange_device = lambda d: 0
    mod._is_in_bad_fork = lambda: False
    mod.manual_seed_all = lambda seed: None
    mod.manual_seed = lambda seed: None
    sys.modules["torch.applegpu"] = mod
    torch.applegpu = mod

    torch.ops.load_library(BACKEND_LIB)
    ready = ctypes.CDLL(BACKEND_LIB).applegpu_backend_ready
    ready.restype = ctypes.c_int32
    if ready() != 1:
        from ._native import lib
        err = lib.applegpu_eager_last_error()
        raise RuntimeError("applegpu backend init failed: " + (err.decode() if err else "unknown error"))
    torch.utils.rename_privateuse1_backend("applegpu")
    torch.utils.generate_methods_for_privateuse1_backend()
    _loaded = True


def fallback_count() -> int:
    """aten ops that ran through the CPU fallback since the extension loaded."""
    f = ctypes.CDLL(BACKEND_LIB).applegpu_backend_fallback_count
    f.restype = ctypes.c_uint64
    return int(f())
