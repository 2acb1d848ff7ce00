"""applegpu_runtime on AMD Instinct MI355X (gfx950).

The same Python surface as the reference's PyO3 module
(crates/python/src/lib.rs:1258+, re-exported by
python/applegpu_runtime/__init__.py:3-125): lazy `GpuTensor`s whose ops build a
graph that is evaluated on read (`to_numpy`, `to_list`, `eval`).  Every op
records through `applegpu_graph_op` in libapplegpu_core.so; evaluation runs the
gfx950 kernels (MFMA GEMMs with fused bias/activation/residual epilogues, fused
causal attention, wavefront-per-row softmax/layer_norm, per-row int8
quantize).  Errors raise ValueError as in the reference (lib.rs:30-33).
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_int64, c_uint32, c_uint64

import numpy as np

from . import _native
from ._native import lib, canon_dtype, ffi_error, DTYPE_CODES, CODE_DTYPES, DTYPE_SIZES

__version__ = "0.9.0+mi355x"

_initialized = False


def _check_init():
    global _initialized
    if not _initialized:
        if not lib.applegpu_ffi_init():
            raise ValueError(f"applegpu backend init failed: {ffi_error()}")
        _initialized = True


class GpuTensor:
    """A lazy tensor handle (reference: `GpuTensor`, crates/python/src/lib.rs:100-372)."""

    __slots__ = ("_id", "_destroyed", "__weakref__")

    def __init__(self, tid: int):
        self._id = tid
        self._destroyed = False

    # metadata -------------------------------------------------------------
    @property
    def id(self) -> int:
        return self._id

    @property
    def shape(self) -> list:
        dims = (c_uint64 * 8)()
        nd = c_uint32()
        if lib.applegpu_ffi_shape(self._id, dims, ctypes.byref(nd)) != 0:
            raise ValueError(ffi_error())
        return [int(dims[i]) for i in range(nd.value)]

    @property
    def dtype(self) -> str:
        code = lib.applegpu_ffi_dtype(self._id)
        if code < 0:
            raise ValueError(f"tensor {self._id} not found")
        return CODE_DTYPES[code]

    def strides(self) -> list:
        st = (c_int64 * 8)()
        nd = c_uint32()
        if lib.applegpu_ffi_strides(self._id, st, ctypes.byref(nd)) != 0:
            raise ValueError(ffi_error())
        return [int(st[i]) for i in range(nd.value)]

    def is_pending(self) -> bool:
        return lib.applegpu_ffi_is_pending(self._id) == 1

    # materialisation --------------------------------------------------------
    def eval(self) -> None:
        if lib.applegpu_ffi_eval(self._id) != 0:
            raise ValueError(ffi_error())

    def _read_raw(self) -> np.ndarray:
        dt = self.dtype
        shape = self.shape
        n = int(np.prod(shape)) if shape else 1
        if dt == "bfloat16":
            raw = np.empty(n, dtype=np.uint16)
        else:
            raw = np.empty(n, dtype=np.bool_ if dt == "bool" else np.dtype(dt))
        if lib.applegpu_ffi_read_bytes(self._id, raw.ctypes.data, raw.nbytes) != 0:
            raise ValueError(ffi_error())
        if dt == "bfloat16":
            raw = (raw.astype(np.uint32) << 16).view(np.float32)
        return raw.reshape(shape)

    def write(self, arr) -> None:
        """Overwrites this (materialised) tensor with host data of the same
        shape; bfloat16 tensors take float32 data, rounded to nearest even."""
        dt = self.dtype
        a = np.asarray(arr)
        if list(a.shape) != self.shape and a.size != int(np.prod(self.shape) if self.shape else 1):
            raise ValueError(f"write: shape {list(a.shape)} does not match {self.shape}")
        if dt == "bfloat16":
            u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
            raw = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        else:
            raw = np.ascontiguousarray(a, dtype=np.bool_ if dt == "bool" else np.dtype(dt))
        if lib.applegpu_ffi_write_bytes(self._id, raw.ctypes.data, raw.nbytes) != 0:
            raise ValueError(ffi_error())

    def to_numpy(self) -> np.ndarray:
        """Evaluates if lazy and returns a copy (bfloat16 comes back as float32)."""
        return self._read_raw()

    def to_list(self) -> list:
        return self._read_raw().reshape(-1).tolist()

    def to_torch(self):
        import torch
        if self.dtype == "bfloat16":
            return torch.from_numpy(self._read_raw()).to(torch.bfloat16)
        return torch.from_numpy(self._read_raw()).clone()

    # ops --------------------------------------------------------------------
    def neg(self): return neg(self)
    def relu(self): return relu(self)
    def exp(self): return exp(self)
    def log(self): return log(self)
    def softmax(self): return softmax(self)
    def log_softmax(self): return log_softmax(self)
    def tanh(self): return tanh(self)
    def sin(self): return sin(self)
    def cos(self): return cos(self)
    def gelu(self): return gelu(self)
    def sigmoid(self): return sigmoid(self)
    def var(self, correction=1): return var(self, correction)
    def std(self, correction=1): return std_dev(self, correction)
    def sqrt(self): return sqrt(self)
    def abs(self): return abs(self)
    def sign(self): return sign(self)
    def transpose(self): return transpose(self)
    def argmax(self): return argmax(self)
    def sum(self): return sum(self)
    def mean(self): return mean(self)
    def amax(self): return amax(self)
    def softmax_causal(self): return softmax_causal(self)
    def layer_norm(self, gamma, beta, eps=1e-5): return layer_norm(self, gamma, beta, eps)
    def transpose_dims(self, dim0, dim1): return transpose_dims(self, dim0, dim1)
    def pow(self, exponent): return pow(self, exponent)
    def clamp(self, min_val, max_val): return clamp(self, min_val, max_val)
    def masked_fill(self, mask, value): return masked_fill(self, mask, value)
    def triu(self, diagonal=0): return triu(self, diagonal)
    def tril(self, diagonal=0): return tril(self, diagonal)
    def gather(self, dim, index): return gather(self, dim, index)
    def index_select(self, dim, index): return index_select(self, dim, index)
    def scalar_mul(self, scale): return scalar_mul(self, scale)
    def reshape(self, new_shape): return reshape(self, new_shape)
    def add(self, other): return add(self, other)
    def sub(self, other): return sub(self, other)
    def mul(self, other): return mul(self, other)
    def div(self, other): return div(self, other)
    def matmul(self, other): return matmul(self, other)
    __add__ = add
    __sub__ = sub
    __mul__ = mul
    __truediv__ = div
    __matmul__ = matmul
    __neg__ = neg

    def __repr__(self):
        if self._destroyed:
            return f"GpuTensor(id={self._id}, destroyed)"
        try:
            state = "lazy" if self.is_pending() else "materialized"
            return f"GpuTensor(id={self._id}, shape={self.shape}, {state})"
        except ValueError:
            return f"GpuTensor(id={self._id}, destroyed)"

    def __del__(self):
        if not self._destroyed and lib is not None:
            try:
                lib.applegpu_ffi_free(self._id)
            except Exception:
                pass


# ── op plumbing ─────────────────────────────────────────────────────────────
def _op(name: bytes, tensors, f=(), i=(), nout=1):
    n = len(tensors)
    ins = (c_uint64 * n)(*[t._id for t in tensors])
    fa = (c_double * len(f))(*f) if f else None
    ia = (c_int64 * len(i))(*i) if i else None
    out = (c_uint64 * nout)()
    r = lib.applegpu_graph_op(name, ins, n, fa, len(f), ia, len(i), out, nout)
    if r < 0:
        raise ValueError(ffi_error())
    if nout == 1:
        return GpuTensor(out[0])
    return tuple(GpuTensor(out[k]) for k in range(r))


def _t(x) -> GpuTensor:
    if isinstance(x, GpuTensor):
        return x
    raise ValueError(f"expected GpuTensor, got {type(x).__name__}")


# ── module functions (crates/python/src/lib.rs:378-1258) ───────────────────
def version() -> str:
    return __version__


def init_backend() -> dict:
    _check_init()
    return {"backend": "mi355x-hip", "device": device_name()}


def device_name() -> str:
    _check_init()
    buf = ctypes.create_string_buffer(256)
    if lib.applegpu_ffi_device_name(buf, 256) != 0:
        raise ValueError(ffi_error())
    return buf.value.decode()


def dtype_size(name: str) -> int:
    return DTYPE_SIZES[canon_dtype(name)]


def _from_raw(raw: np.ndarray, shape, dtype: str) -> GpuTensor:
    _check_init()
    code = DTYPE_CODES[dtype]
    nbytes = raw.nbytes
    tid = c_uint64()
    lib.applegpu_ffi_alloc(max(nbytes, 1), code, ctypes.byref(tid))
    t = GpuTensor(tid.value)
    dims = (c_uint64 * len(shape))(*shape)
    if lib.applegpu_ffi_register_tensor(tid.value, dims, len(shape), code) != 0:
        raise ValueError(ffi_error())
    if nbytes and lib.applegpu_ffi_write_bytes(tid.value, raw.ctypes.data, nbytes) != 0:
        raise ValueError(ffi_error())
    return t


def from_numpy(arr) -> GpuTensor:
    """Copy a numpy array to the device (reference lib.rs:419-451)."""
    arr = np.asarray(arr)
    name = "bool" if arr.dtype == np.bool_ else arr.dtype.name
    if name not in DTYPE_CODES:
        raise ValueError(f"Unsupported numpy dtype: {name}. Supported: float16, float32, float64, int8, int16, "
                         "int32, int64, uint8, uint32, bool")
    raw = np.ascontiguousarray(arr)
    return _from_raw(raw, list(arr.shape), name)


from_numpy_shared = from_numpy


def from_torch(tensor) -> GpuTensor:
    """Copy a torch tensor to the device (reference lib.rs:454-500)."""
    import torch
    t = tensor.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        raw = t.view(torch.int16).numpy().view(np.uint16)
        return _from_raw(raw, list(t.shape), "bfloat16")
    return from_numpy(t.numpy())


from_torch_shared = from_torch


def from_bytes(data: bytes, shape, dtype: str) -> GpuTensor:
    dtype = canon_dtype(dtype)
    raw = np.frombuffer(data, dtype=np.uint8)
    expect = int(np.prod(shape)) * DTYPE_SIZES[dtype] if shape else DTYPE_SIZES[dtype]
    if raw.nbytes != expect:
        raise ValueError(f"from_bytes: {raw.nbytes} bytes for shape {list(shape)} of {dtype}")
    return _from_raw(np.ascontiguousarray(raw), list(shape), dtype)


def aligned_numpy(shape, dtype=None):
    return np.zeros(shape, dtype=np.dtype(canon_dtype(dtype or "float32")))


def tensor(data, shape, dtype=None) -> GpuTensor:
    dtype = canon_dtype(dtype or "float32")
    if dtype == "bfloat16":
        f = np.asarray(data, dtype=np.float32).reshape(shape)
        return cast(from_numpy(f), "bfloat16")
    return from_numpy(np.asarray(data, dtype=np.dtype(dtype)).reshape(shape))


def eval(t):
    _t(t).eval()


def eval_many(tensors):
    """Evaluates several lazy tensors in one walk, so that a producer several
    of them read (a GEMM writing its output, packed rows and row
    statistics) runs once with all of its outputs."""
    ts = [_t(t) for t in tensors]
    ids = (ctypes.c_uint64 * len(ts))(*[t._id for t in ts])
    if lib.applegpu_ffi_eval_many(ids, len(ts)) != 0:
        raise ValueError(ffi_error())


def to_list(t):
    return _t(t).to_list()


def shape(t):
    return _t(t).shape


def destroy(t):
    t = _t(t)
    if not t._destroyed:
        lib.applegpu_ffi_free(t._id)
        t._destroyed = True


def set_limits(max_tensor_size_mb=0, max_memory_mb=0, max_tensors=0):
    _check_init()
    mb = 1024 * 1024
    lib.applegpu_ffi_set_limits(max_tensor_size_mb * mb, max_memory_mb * mb, max_tensors)


def memory_usage() -> int:
    _check_init()
    return int(lib.applegpu_ffi_memory_usage())


def tensor_count() -> int:
    _check_init()
    return int(lib.applegpu_ffi_tensor_count())


def pool_stats() -> dict:
    _check_init()
    out = (c_uint64 * 5)()
    lib.applegpu_ffi_pool_stats(out)
    return {"hits": out[0], "misses": out[1], "pooled_bytes": out[2], "bucket_count": out[3],
            "live_bytes": out[4]}


def pool_drain():
    _check_init()
    lib.applegpu_ffi_pool_drain()


def set_pool_watermark(mb: int):
    _check_init()
    lib.applegpu_ffi_set_pool_watermark(int(mb) * 1024 * 1024)


def graph_stats() -> dict:
    """Lazy-executor counters since the library loaded: evals, nodes,
    GEMM epilogue fusions, launches saved by fusion, fused elementwise
    chains and the nodes inside them, and kernel launcher calls."""
    names = ("evals", "nodes", "fused_gemm_epilogues", "launches_saved", "fused_chains", "chain_nodes",
             "launcher_calls")
    out = (c_uint64 * len(names))()
    lib.applegpu_ffi_graph_stats_ex(out, len(names))
    return dict(zip(names, (int(v) for v in out)))


# Streaming batches (reference lib.rs:1244-1257): one HIP stream is always
# streaming here, so begin is a no-op and flush/end wait for the stream.
def begin_streaming_batch():
    _check_init()


def flush_streaming_batch():
    lib.applegpu_ffi_synchronize()


def end_streaming_batch():
    lib.applegpu_ffi_synchronize()


def synchronize():
    lib.applegpu_ffi_synchronize()


# binary
def add(a, b): return _op(b"add", [_t(a), _t(b)])
def sub(a, b): return _op(b"sub", [_t(a), _t(b)])
def mul(a, b): return _op(b"mul", [_t(a), _t(b)])
def div(a, b): return _op(b"div", [_t(a), _t(b)])
def matmul(a, b): return _op(b"matmul", [_t(a), _t(b)])
def lt(a, b): return _op(b"lt", [_t(a), _t(b)])
def gt(a, b): return _op(b"gt", [_t(a), _t(b)])
def le(a, b): return _op(b"le", [_t(a), _t(b)])
def ge(a, b): return _op(b"ge", [_t(a), _t(b)])
def eq_(a, b): return _op(b"eq", [_t(a), _t(b)])
def ne_(a, b): return _op(b"ne", [_t(a), _t(b)])
def bitwise_and(a, b): return _op(b"bitwise_and", [_t(a), _t(b)])
def bitwise_or(a, b): return _op(b"bitwise_or", [_t(a), _t(b)])
def bitwise_xor(a, b): return _op(b"bitwise_xor", [_t(a), _t(b)])
def mod_(a, b): return _op(b"mod", [_t(a), _t(b)])
def elem_min(a, b): return _op(b"elem_min", [_t(a), _t(b)])
def elem_max(a, b): return _op(b"elem_max", [_t(a), _t(b)])


# unary
def neg(t): return _op(b"neg", [_t(t)])
def relu(t): return _op(b"relu", [_t(t)])
def exp(t): return _op(b"exp", [_t(t)])
def log(t): return _op(b"log", [_t(t)])
def sqrt(t): return _op(b"sqrt", [_t(t)])
def abs(t): return _op(b"abs", [_t(t)])
def sign(t): return _op(b"sign", [_t(t)])
def tanh(t): return _op(b"tanh", [_t(t)])
def sin(t): return _op(b"sin", [_t(t)])
def cos(t): return _op(b"cos", [_t(t)])
def gelu(t): return _op(b"gelu", [_t(t)])
def gelu_exact(t): return _op(b"gelu_exact", [_t(t)])
def sigmoid(t): return _op(b"sigmoid", [_t(t)])
def bitwise_not(t): return _op(b"bitwise_not", [_t(t)])
def logical_not(t): return _op(b"logical_not", [_t(t)])
def shl(t, shift): return _op(b"shl", [_t(t)], i=(int(shift),))
def shr(t, shift): return _op(b"shr", [_t(t)], i=(int(shift),))
def pow(t, exponent): return _op(b"pow", [_t(t)], f=(float(exponent),))
def clamp(t, min_val, max_val): return _op(b"clamp", [_t(t)], f=(float(min_val), float(max_val)))
def scalar_mul(t, scale): return _op(b"scalar_mul", [_t(t)], f=(float(scale),))
def cast(t, dtype): return _op(b"cast", [_t(t)], i=(DTYPE_CODES[canon_dtype(dtype)],))


# shape / layout
def reshape(t, new_shape): return _op(b"reshape", [_t(t)], i=tuple(int(d) for d in new_shape))
def transpose(t): return _op(b"transpose", [_t(t)])
def transpose_dims(t, dim0, dim1): return _op(b"transpose_dims", [_t(t)], i=(int(dim0), int(dim1)))
def slice(t, dim, start, end): return _op(b"slice", [_t(t)], i=(int(dim), int(start), int(end)))
def concat(a, b, dim): return _op(b"concat", [_t(a), _t(b)], i=(int(dim),))
def contiguous(t): return _op(b"contiguous", [_t(t)])


def full(shape, value, dtype="float32") -> GpuTensor:
    """A new device tensor of `shape` filled with `value` (materialised)."""
    t = _op(b"full", [], f=(float(value),), i=(DTYPE_CODES[canon_dtype(dtype)],) + tuple(int(s) for s in shape))
    t.eval()
    return t


def zeros(shape, dtype="float32") -> GpuTensor:
    return full(shape, 0.0, dtype)


def concat_all(tensors, dim=0):
    tensors = list(tensors)
    if not tensors:
        raise ValueError("concat_all needs at least one tensor")
    out = tensors[0]
    for t in tensors[1:]:
        out = concat(out, t, dim)
    return out


# rows / reductions
def softmax(t): return _op(b"softmax", [_t(t)])
def log_softmax(t): return _op(b"log_softmax", [_t(t)])
def softmax_causal(t): return _op(b"softmax_causal", [_t(t)])
def layer_norm(input, gamma, beta, eps=1e-5): return _op(b"layer_norm", [_t(input), _t(gamma), _t(beta)], f=(eps,))
def argmax(t): return _op(b"argmax", [_t(t)])
def sum(t): return _op(b"sum", [_t(t)])
def mean(t): return _op(b"mean", [_t(t)])
def amax(t): return _op(b"amax", [_t(t)])
def var(t, correction=1): return _op(b"var", [_t(t)], i=(int(correction),))
def std_dev(t, correction=1): return _op(b"std", [_t(t)], i=(int(correction),))
def mean_all(t): return _op(b"mean_all", [_t(t)])
def sum_dim(t, dim, keepdim=False): return _op(b"sum_dim", [_t(t)], i=(int(dim), int(bool(keepdim))))


# transformer ops
def embedding(weights, indices): return _op(b"embedding", [_t(weights), _t(indices)])
def add_bias(input, bias): return _op(b"add_bias", [_t(input), _t(bias)])
def attention(q, k, v, scale=None):
    """softmax(q k^T * scale) v, scale 1/sqrt(d_k) by default (lib.rs:932)."""
    return _op(b"attention", [_t(q), _t(k), _t(v)], f=() if scale is None else (float(scale),))


def qkv_attention(x, w, b, n_head, causal=True, batch=1, read_partials=False):
    """Attention of a fused QKV projection: heads of (x @ w + b) split into Q,
    K, V (w [K, 3d] row-major, as GPT-2's c_attn, or those weights packed by
    pack_weight_x3), (causal) attention, heads merged back: [batch*T, d].
    read_partials (fp32): the attention kernel reads the projection's split-K
    partial sums plus the bias itself, with no reduction launch."""
    return _op(b"qkv_attention", [_t(x), _t(w), _t(b)],
               i=(int(n_head), int(bool(causal)), int(batch), int(bool(read_partials))))
def attention_causal(q, k, v, scale=None):
    """Causal attention, query i seeing keys j <= i (lib.rs:1026)."""
    return _op(b"attention_causal", [_t(q), _t(k), _t(v)], f=() if scale is None else (float(scale),))
def gather(input, dim, index): return _op(b"gather", [_t(input), _t(index)], i=(int(dim),))
def index_select(input, dim, index): return _op(b"index_select", [_t(input), _t(index)], i=(int(dim),))
def where_cond(cond, x, y): return _op(b"where", [_t(cond), _t(x), _t(y)])
def masked_fill(t, mask, value): return _op(b"masked_fill", [_t(t), _t(mask)], f=(float(value),))
def triu(t, diagonal=0): return _op(b"triu", [_t(t)], i=(int(diagonal),))
def tril(t, diagonal=0): return _op(b"tril", [_t(t)], i=(int(diagonal),))


def linear(x, weight, bias=None, activation=None):
    """y = act(x @ weight^T + bias) in one GEMM (weight in torch layout [out, in])."""
    acts = {None: 0, "relu": 1, "gelu": 2, "gelu_tanh": 2, "gelu_exact": 3}
    ins = [_t(x), _t(weight)] + ([_t(bias)] if bias is not None else [])
    return _op(b"linear", ins, i=(acts[activation],))


# backward helpers
def threshold_backward(grad_output, input, threshold):
    return _op(b"threshold_backward", [_t(grad_output), _t(input)], f=(float(threshold),))


def softmax_backward(grad_output, output): return _op(b"softmax_backward", [_t(grad_output), _t(output)])


# backward ops of the transformer blocks (crates/python/src/lib.rs:1153-1229)
def layer_norm_backward(grad_output, input, gamma, eps=1e-5):
    """dL/dx of layer_norm over the last dim (statistics recomputed from the
    input); ops.rs:690-728."""
    return _op(b"layer_norm_backward", [_t(grad_output), _t(input), _t(gamma)], f=(float(eps),))


def layer_norm_grads(grad_output, input, gamma, eps=1e-5):
    """(dx, dgamma, dbeta) of layer_norm: dx as layer_norm_backward, dgamma =
    sum over rows of dy * xhat, dbeta = sum over rows of dy."""
    return _op(b"layer_norm_grads", [_t(grad_output), _t(input), _t(gamma)], f=(float(eps),), nout=3)


def gelu_backward(grad_output, input):
    """grad * d/dx gelu_tanh(x) (ops.rs:1090-1111)."""
    return _op(b"gelu_backward", [_t(grad_output), _t(input)])


def gelu_tanh_backward(grad_output, input):
    return _op(b"gelu_tanh_backward", [_t(grad_output), _t(input)])


def gelu_exact_backward(grad_output, input):
    """grad * (Phi(x) + x phi(x)) (ops.rs:1136-1158)."""
    return _op(b"gelu_exact_backward", [_t(grad_output), _t(input)])


def embedding_backward(grad_output, indices, num_weights):
    """[num_weights, D] with row w = sum of the grad rows whose index is w,
    added in token order (ops.rs:915-960)."""
    return _op(b"embedding_backward", [_t(grad_output), _t(indices)], i=(int(num_weights),))
def mse_loss(a, b): return _op(b"mse_loss", [_t(a), _t(b)])
def mse_loss_backward(grad, a, b): return _op(b"mse_loss_backward", [_t(grad), _t(a), _t(b)])


# quantization
def quantize(t, dtype, scale=0.1, zero_point=0):
    """Per-tensor quantize, round half away from zero (reference lib.rs:1013-1018)."""
    return _op(b"quantize", [_t(t)], f=(float(scale),), i=(DTYPE_CODES[canon_dtype(dtype)], int(zero_point)))


def dequantize(t, dtype, scale=0.1, zero_point=0):
    return _op(b"dequantize", [_t(t)], f=(float(scale),), i=(DTYPE_CODES[canon_dtype(dtype)], int(zero_point)))


def quantize_per_row(t):
    """Symmetric per-row int8: returns (codes int8, scales float32[rows]);
    scale = absmax(row)/127, codes = clamp(round_half_even(x/scale), -128, 127)."""
    return _op(b"quantize_per_row", [_t(t)], nout=2)


def dequantize_per_row(q, scale, dtype="float32"):
    return _op(b"dequantize_per_row", [_t(q), _t(scale)], i=(DTYPE_CODES[canon_dtype(dtype)],))


def pack_weight(wt):
    """Decode-step weights: wt [out, in] (fp16/bf16, torch Linear layout)
    rearranged so the skinny GEMM's loads are contiguous.  Use with
    matmul_packed."""
    return _op(b"pack_weight", [_t(wt)])


def pack_weight_x3(b):
    """fp32 weights for activations of few rows: b is the B operand [in, out]
    of x @ b (any strides; in a multiple of 16), split once into bf16 hi/lo
    MFMA fragments.  Use with matmul_packed(x, packed, out)."""
    return _op(b"pack_weight_x3", [_t(b)])


def matmul_packed(x, packed, out_features):
    """x @ W for packed weights: packed = pack_weight(wt) (fp16/bf16 wt [out,
    in], x [rows <= 16, in]; the product is x @ wt^T), or packed =
    pack_weight_x3(b) (fp32 b [in, out], x [any rows, in]; x @ b)."""
    return _op(b"matmul_packed", [_t(x), _t(packed)], i=(int(out_features),))


def pack_rows_x3(x):
    """fp32 activations x [rows, cols] (cols a multiple of 16) split into
    bf16 hi/lo MFMA A-operand fragments: [ceil(rows/32), cols/16, 2, 64, 8]
    bfloat16.  Use with matmul_pp(packed_rows, rows, packed_weights, out).
    Inside a lazy graph the producer of x (a packed-weight GEMM's epilogue,
    a split-K reduction computing layer_norm, the fused embedding) writes the
    packed rows directly."""
    return _op(b"pack_rows_x3", [_t(x)])


def matmul_pp(packed_rows, rows, packed, out_features):
    """x @ b with both operands packed: packed_rows = pack_rows_x3(x) for x
    [rows, in], packed = pack_weight_x3(b) for b [in, out]; fp32 result
    [rows, out]."""
    return _op(b"matmul_pp", [_t(packed_rows), _t(packed)], i=(int(rows), int(out_features)))


def row_stats_x3(x):
    """Row statistics of fp32 x [rows, cols] (cols a multiple of 32) per
    32-column tile: [rows, cols/32, 2] = (sum, sum of squared deviations
    from the tile mean), the input of matmul_pp_norm.  Inside a lazy graph
    the packed-weight GEMM producing x writes them from its epilogue."""
    return _op(b"row_stats_x3", [_t(x)])


def x3_rows_out_ok(rows, out_features, in_features) -> bool:
    """Whether packed rows [rows, in_features] times packed fp32 weights
    [in_features, out_features] run a plan whose one launch writes the
    output, its packed rows and its row statistics (an unsplit row panel,
    or a split one whose tiles are finished in the launch)."""
    _check_init()
    r = lib.applegpu_ffi_x3_rows_out(int(rows), int(out_features), int(in_features))
    if r < 0:
        raise ValueError(ffi_error())
    return r == 1


def matmul_pp_norm(packed_rows, stats, rows, packed, cs, out_features, eps=1e-5):
    """layer_norm(x) @ W without normalising x first: packed_rows =
    pack_rows_x3(x), stats = row_stats_x3(x), packed = pack_weight_x3(gamma[:,
    None] * W), cs = column sums of gamma[:, None] * W.  Returns
    inv * (x @ (gamma W) - mean * cs) per row (mean and inv =
    1 / sqrt(var + eps) from the statistics); adding beta @ W (+ the layer's
    bias) gives layer_norm(x, gamma, beta) @ W (+ bias)."""
    return _op(b"matmul_pp_norm", [_t(packed_rows), _t(stats), _t(packed), _t(cs)],
               f=(float(eps),), i=(int(rows), int(out_features)))


def linear_int8(x, q, scale):
    """x @ (q * scale[:, None])^T with the dequantisation fused into the GEMM."""
    return _op(b"linear_int8", [_t(x), _t(q), _t(scale)])


def blit_copy(src, dst):
    """dst = src on the device, at once; dst may be a view (a slice of a
    larger tensor, any strides), which is then written in place."""
    if lib.applegpu_ffi_copy(_t(src)._id, _t(dst)._id) != 0:
        raise ValueError(ffi_error())


def kv_write(cache, rows, pos):
    """cache[b, h, pos[b] + t, :] = rows[b, h, t, :], in place, at once.

    cache [B, H, Tmax, D] and rows [B, H, T, D] share a dtype; pos is an
    int32 device tensor [B] read by the kernel (so a captured graph can be
    replayed with advancing positions).  Rows that would land outside the
    cache are not written."""
    if lib.applegpu_kv_write(_t(cache)._id, _t(rows)._id, _t(pos)._id) != 0:
        raise ValueError(ffi_error())


def kv_write_pair(k_cache, v_cache, k_rows, v_rows, pos):
    """kv_write of the K and the V rows of one layer in a single launch."""
    if lib.applegpu_kv_write_pair(_t(k_cache)._id, _t(v_cache)._id, _t(k_rows)._id, _t(v_rows)._id,
                                  _t(pos)._id) != 0:
        raise ValueError(ffi_error())


def decode_attention(q, k_cache, v_cache, lens, k_new=None, v_new=None):
    """softmax(q K^T / sqrt(D)) V of q [B, H, Tq, D] over the first lens[b]
    rows of the [B, H, Tmax, D] caches (lens: int32 device tensor [B]); query
    row i of sequence b sees cache rows j <= lens[b] - Tq + i.  With Tq = 1
    this is the reference's decode step, non-causal attention of the new
    token over the whole cache (python/applegpu_runtime/models/gpt2.py:132-135).

    k_new, v_new ([B, H, 1, D], Tq = 1): the step's own K and V rows, written
    into the caches as row lens[b] - 1 by the same kernel when the result is
    evaluated (the kv_write of the step, without a launch of its own); the
    caches must not be read by anything else of the same graph."""
    ins = [_t(q), _t(k_cache), _t(v_cache), _t(lens)]
    if k_new is not None or v_new is not None:
        ins += [_t(k_new), _t(v_new)]
    return _op(b"decode_attention", ins)


# ── graph capture ────────────────────────────────────────────────────────────
class CapturedGraph:
    """The launch sequence of one call, recorded as a HIP graph.

    `replay()` re-runs every recorded kernel (hipGraphLaunch on the library
    stream, asynchronous) from the current contents of the tensors the call
    read, into the same output buffers: write new inputs with
    `GpuTensor.write` (or eager `copy_from`) between replays, then read
    `outputs`.  The reference has no counterpart: it re-encodes every op of
    every eval (crates/core/src/lazy.rs:369-474)."""

    def __init__(self, handle: int, outputs):
        self._handle = handle
        self.outputs = outputs

    @property
    def handle(self) -> int:
        return self._handle

    def replay(self) -> None:
        if lib.applegpu_graph_replay(self._handle) != 0:
            raise ValueError(ffi_error())

    def nbytes(self) -> int:
        return int(lib.applegpu_graph_bytes(self._handle))

    def destroy(self) -> None:
        if self._handle:
            lib.applegpu_graph_destroy(self._handle)
            self._handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def capture(fn, *args, **kwargs) -> CapturedGraph:
    """Runs `fn(*args, **kwargs)` once under stream capture and returns the
    recorded graph; its `outputs` are fn's return value, with lazy tensors
    evaluated inside the capture.  Inputs must already be materialised on
    the device (no host reads or writes are allowed inside `fn`)."""
    _check_init()
    if lib.applegpu_capture_begin() != 0:
        raise ValueError(ffi_error())
    try:
        out = fn(*args, **kwargs)
        for t in (out if isinstance(out, (list, tuple)) else [out]):
            if isinstance(t, GpuTensor):
                t.eval()
    except BaseException:
        lib.applegpu_capture_abort()
        raise
    handle = lib.applegpu_capture_end()
    if handle <= 0:
        raise ValueError(ffi_error())
    return CapturedGraph(int(handle), out)
