"""ctypes binding of libapplegpu_core.so (the C ABI in include/applegpu_ffi.h).

The library is built in-tree by applegpu-runtime_amd/build.py.  Importing this
module without the built library raises ImportError: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_bool, c_char_p, c_double, c_float, c_int8, c_int32, c_int64, c_uint8, c_uint16, \
    c_uint32, c_uint64, c_void_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libapplegpu_core.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libapplegpu_core.so not found at {LIB_PATH}; build it with "
        "`python applegpu-runtime_amd/build.py` (hipcc, gfx950)")

lib = ctypes.CDLL(LIB_PATH)

u64p = POINTER(c_uint64)
i64p = POINTER(c_int64)
u32p = POINTER(c_uint32)
u8p = POINTER(c_uint8)

_SIGS = {
    # graph path (reference surface)
    "applegpu_ffi_init": (c_bool, []),
    "applegpu_ffi_last_error": (c_char_p, []),
    "applegpu_ffi_alloc": (c_void_p, [c_uint64, c_int8, u64p]),
    "applegpu_ffi_free": (None, [c_uint64]),
    "applegpu_ffi_register_tensor": (c_int32, [c_uint64, u64p, c_uint32, c_int8]),
    "applegpu_ffi_shape": (c_int32, [c_uint64, u64p, u32p]),
    "applegpu_ffi_dtype": (c_int8, [c_uint64]),
    "applegpu_ffi_add": (c_uint64, [c_uint64, c_uint64]),
    "applegpu_ffi_matmul": (c_uint64, [c_uint64, c_uint64]),
    "applegpu_ffi_relu": (c_uint64, [c_uint64]),
    "applegpu_ffi_mul": (c_uint64, [c_uint64, c_uint64]),
    "applegpu_ffi_sub": (c_uint64, [c_uint64, c_uint64]),
    "applegpu_ffi_neg": (c_uint64, [c_uint64]),
    "applegpu_ffi_copy": (c_int32, [c_uint64, c_uint64]),
    "applegpu_ffi_add_out": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_ffi_mul_out": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_ffi_sub_out": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_ffi_matmul_out": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_ffi_relu_out": (c_void_p, [c_uint64, u64p]),
    "applegpu_ffi_neg_out": (c_void_p, [c_uint64, u64p]),
    "applegpu_ffi_div_out": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_ffi_threshold_backward_out": (c_void_p, [c_uint64, c_uint64, c_float, u64p]),
    "applegpu_ffi_scalar_mul_out": (c_void_p, [c_uint64, c_float, u64p]),
    "applegpu_ffi_mean_all_out": (c_void_p, [c_uint64, u64p]),
    "applegpu_ffi_eval": (c_int32, [c_uint64]),
    "applegpu_ffi_eval_many": (c_int32, [POINTER(c_uint64), c_uint32]),
    "applegpu_ffi_synchronize": (None, []),
    "applegpu_ffi_read_f32": (c_int32, [c_uint64, POINTER(c_float), c_uint64]),
    # eager path (reference surface)
    "applegpu_eager_init": (c_bool, []),
    "applegpu_eager_last_error": (c_char_p, []),
    "applegpu_eager_alloc": (c_void_p, [u64p, c_uint32, c_int8, u64p]),
    "applegpu_eager_free": (None, [c_uint64]),
    "applegpu_eager_register_shape": (c_int32, [c_uint64, u64p, c_uint32]),
    "applegpu_eager_shape": (c_int32, [c_uint64, u64p, u32p]),
    "applegpu_eager_dtype": (c_int8, [c_uint64]),
    "applegpu_eager_add": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_sub": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_mul": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_div": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_relu": (c_void_p, [c_uint64, u64p]),
    "applegpu_eager_neg": (c_void_p, [c_uint64, u64p]),
    "applegpu_eager_matmul": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_matmul_ex": (c_void_p, [c_uint64, c_uint64, c_bool, c_bool, u64p]),
    "applegpu_eager_threshold_backward": (c_void_p, [c_uint64, c_uint64, c_float, u64p]),
    "applegpu_eager_scalar_mul": (c_void_p, [c_uint64, c_float, u64p]),
    "applegpu_eager_mean_all": (c_void_p, [c_uint64, u64p]),
    "applegpu_eager_sum_dim": (c_void_p, [c_uint64, c_int64, c_bool, u64p]),
    "applegpu_eager_create_view": (c_void_p, [c_uint64, u64p, u64p, c_uint32, c_uint64, u64p]),
    "applegpu_eager_add_inplace": (c_int32, [c_uint64, c_uint64]),
    "applegpu_eager_add_scaled_inplace": (c_int32, [c_uint64, c_uint64, c_float]),
    "applegpu_eager_flush_and_wait": (None, []),
    "applegpu_eager_synchronize": (None, []),
    "applegpu_eager_embedding": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_layer_norm": (c_void_p, [c_uint64, c_uint64, c_uint64, c_float, u64p]),
    "applegpu_eager_gelu": (c_void_p, [c_uint64, u64p]),
    "applegpu_eager_softmax": (c_void_p, [c_uint64, u64p]),
    "applegpu_eager_find_by_data_ptr": (c_uint64, [c_void_p]),
    "applegpu_eager_execute_graph": (c_int32, [c_void_p, c_uint32, u64p, c_uint32, POINTER(c_uint16), c_uint32,
                                              u64p, POINTER(c_void_p)]),
    # additions
    "applegpu_graph_op": (c_int32, [c_char_p, u64p, c_uint32, POINTER(c_double), c_uint32, i64p, c_uint32, u64p,
                                    c_uint32]),
    "applegpu_ffi_write_bytes": (c_int32, [c_uint64, c_void_p, c_uint64]),
    "applegpu_ffi_read_bytes": (c_int32, [c_uint64, c_void_p, c_uint64]),
    "applegpu_ffi_is_pending": (c_int32, [c_uint64]),
    "applegpu_ffi_strides": (c_int32, [c_uint64, i64p, u32p]),
    "applegpu_ffi_pool_stats": (c_int32, [u64p]),
    "applegpu_ffi_pool_drain": (None, []),
    "applegpu_ffi_set_pool_watermark": (None, [c_uint64]),
    "applegpu_ffi_memory_usage": (c_uint64, []),
    "applegpu_ffi_tensor_count": (c_uint64, []),
    "applegpu_ffi_set_limits": (None, [c_uint64, c_uint64, c_uint64]),
    "applegpu_ffi_device_name": (c_int32, [c_char_p, c_uint32]),
    "applegpu_ffi_graph_stats": (c_int32, [u64p]),
    "applegpu_ffi_graph_stats_ex": (c_uint32, [u64p, c_uint32]),
    "applegpu_ffi_inject_alloc_failures": (None, [c_int32]),
    "applegpu_kv_write": (c_int32, [c_uint64, c_uint64, c_uint64]),
    "applegpu_kv_write_pair": (c_int32, [c_uint64, c_uint64, c_uint64, c_uint64, c_uint64]),
    "applegpu_capture_begin": (c_int32, []),
    "applegpu_capture_end": (c_int64, []),
    "applegpu_capture_abort": (c_int32, []),
    "applegpu_graph_replay": (c_int32, [c_int64]),
    "applegpu_graph_destroy": (c_int32, [c_int64]),
    "applegpu_graph_bytes": (c_uint64, [c_int64]),
    "applegpu_ffi_gemm_tune": (c_int32, [c_int32, c_int32, c_int32]),
    "applegpu_ffi_gemm_skinny": (c_int32, [c_int32]),
    "applegpu_ffi_split_inkernel": (c_int32, [c_int32]),
    "applegpu_ffi_x3_rows_out": (c_int32, [c_int64, c_int64, c_int64]),
    "applegpu_ffi_gemm_plan": (c_int32, [c_int64, c_int64, c_int64, c_int64, c_int8, c_bool, c_bool, c_char_p,
                                         c_uint32]),
    "applegpu_ffi_event_record": (c_int32, [c_uint32]),
    "applegpu_ffi_event_elapsed_ms": (c_float, [c_uint32, c_uint32]),
    "applegpu_eager_op": (c_int32, [c_char_p, u64p, c_uint32, POINTER(c_double), c_uint32, i64p, c_uint32, u64p,
                                    c_uint32]),
    "applegpu_eager_copy_from_host": (c_int32, [c_uint64, c_void_p, c_uint64]),
    "applegpu_eager_copy_to_host": (c_int32, [c_uint64, c_void_p, c_uint64]),
    "applegpu_eager_copy_": (c_int32, [c_uint64, c_uint64]),
    "applegpu_eager_data_ptr": (c_void_p, [c_uint64]),
    "applegpu_eager_view_typed": (c_void_p, [c_uint64, u64p, u64p, c_uint32, c_uint64, c_int8, u64p]),
    "applegpu_eager_fill": (c_int32, [c_uint64, c_double]),
    "applegpu_eager_linear": (c_void_p, [c_uint64, c_uint64, c_uint64, c_int32, u64p]),
    "applegpu_eager_linear_noalloc": (c_int32, [c_uint64, c_uint64, c_uint64, c_int32, c_uint64]),
    "applegpu_eager_matmul_masked": (c_void_p, [c_uint64, c_uint64, c_bool, c_bool, c_uint64, u64p]),
    "applegpu_eager_mse_loss": (c_void_p, [c_uint64, c_uint64, u64p]),
    "applegpu_eager_mse_loss_backward": (c_void_p, [c_uint64, c_uint64, c_uint64, u64p]),
    "applegpu_eager_strides": (c_int32, [c_uint64, i64p, u32p]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTED = tuple(_SIGS)

# dtype wire codes (reference crates/core/src/tensor.rs:59-90)
DTYPE_CODES = {
    "float32": 0, "float16": 1, "float64": 2, "int8": 3, "int16": 4, "int32": 5, "int64": 6,
    "uint8": 7, "uint32": 8, "bool": 9, "bfloat16": 10,
}
CODE_DTYPES = {v: k for k, v in DTYPE_CODES.items()}
DTYPE_ALIASES = {
    "f32": "float32", "f16": "float16", "f64": "float64", "i8": "int8", "i16": "int16", "i32": "int32",
    "i64": "int64", "u8": "uint8", "u32": "uint32", "bool_": "bool", "bf16": "bfloat16",
}
DTYPE_SIZES = {"float32": 4, "float16": 2, "float64": 8, "int8": 1, "int16": 2, "int32": 4, "int64": 8,
               "uint8": 1, "uint32": 4, "bool": 1, "bfloat16": 2}


def canon_dtype(name: str) -> str:
    name = DTYPE_ALIASES.get(name, name)
    if name not in DTYPE_CODES:
        raise ValueError(f"Unknown dtype: {name}")
    return name


def ffi_error() -> str:
    e = lib.applegpu_ffi_last_error()
    return e.decode() if e else "unknown error"


def eager_error() -> str:
    e = lib.applegpu_eager_last_error()
    return e.decode() if e else "unknown error"
