"""Thin Python handle over the eager C ABI (`applegpu_eager_*`).

The reference drives this ABI from its PrivateUse1 shim
(backend_cpp/applegpu_backend.cpp): each aten kernel becomes one or a few
eager calls that enqueue work on the device and return at once.  `EagerTensor`
wraps an eager id; ops return new EagerTensors; `synchronize()` waits for the
stream (`applegpu_eager_flush_and_wait`).
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_int64, c_uint32, c_uint64

import numpy as np

from ._native import lib, eager_error, DTYPE_CODES, CODE_DTYPES

_ready = False


def init():
    global _ready
    if not _ready:
        if not lib.applegpu_eager_init():
            raise RuntimeError(f"applegpu eager init failed: {eager_error()}")
        _ready = True


class EagerTensor:
    __slots__ = ("id", "ptr")

    def __init__(self, tid: int, ptr: int | None):
        self.id = tid
        self.ptr = ptr

    @property
    def shape(self):
        dims = (c_uint64 * 8)()
        nd = c_uint32()
        if lib.applegpu_eager_shape(self.id, dims, ctypes.byref(nd)) != 0:
            raise RuntimeError(eager_error())
        return tuple(int(dims[i]) for i in range(nd.value))

    @property
    def dtype(self) -> str:
        return CODE_DTYPES[lib.applegpu_eager_dtype(self.id)]

    def numpy(self) -> np.ndarray:
        dt = self.dtype
        out = np.empty(self.shape, dtype=np.uint16 if dt == "bfloat16" else np.dtype("bool" if dt == "bool" else dt))
        if lib.applegpu_eager_copy_to_host(self.id, out.ctypes.data, out.nbytes) != 0:
            raise RuntimeError(eager_error())
        if dt == "bfloat16":
            out = (out.astype(np.uint32) << 16).view(np.float32)
        return out

    def copy_from(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        if lib.applegpu_eager_copy_from_host(self.id, arr.ctypes.data, arr.nbytes) != 0:
            raise RuntimeError(eager_error())

    def __del__(self):
        try:
            lib.applegpu_eager_free(self.id)
        except Exception:
            pass


def _wrap(ptr, oid: c_uint64) -> EagerTensor:
    if not ptr and oid.value == 0:
        raise RuntimeError(eager_error())
    return EagerTensor(oid.value, ptr)


def empty(shape, dtype="float32") -> EagerTensor:
    init()
    dims = (c_uint64 * len(shape))(*shape)
    oid = c_uint64()
    p = lib.applegpu_eager_alloc(dims, len(shape), DTYPE_CODES[dtype], ctypes.byref(oid))
    return _wrap(p, oid)


def from_numpy(arr: np.ndarray) -> EagerTensor:
    arr = np.ascontiguousarray(arr)
    name = "bool" if arr.dtype == np.bool_ else arr.dtype.name
    t = empty(arr.shape, name)
    t.copy_from(arr)
    return t


def _call(fn, *args) -> EagerTensor:
    oid = c_uint64()
    p = fn(*args, ctypes.byref(oid))
    if not p:
        raise RuntimeError(eager_error())
    return EagerTensor(oid.value, p)


def add(a, b): return _call(lib.applegpu_eager_add, a.id, b.id)
def sub(a, b): return _call(lib.applegpu_eager_sub, a.id, b.id)
def mul(a, b): return _call(lib.applegpu_eager_mul, a.id, b.id)
def div(a, b): return _call(lib.applegpu_eager_div, a.id, b.id)
def relu(x): return _call(lib.applegpu_eager_relu, x.id)
def neg(x): return _call(lib.applegpu_eager_neg, x.id)
def matmul(a, b): return _call(lib.applegpu_eager_matmul, a.id, b.id)
def matmul_ex(a, b, ta=False, tb=False): return _call(lib.applegpu_eager_matmul_ex, a.id, b.id, ta, tb)
def threshold_backward(g, x, thr=0.0): return _call(lib.applegpu_eager_threshold_backward, g.id, x.id, thr)
def scalar_mul(x, s): return _call(lib.applegpu_eager_scalar_mul, x.id, s)
def mean_all(x): return _call(lib.applegpu_eager_mean_all, x.id)
def sum_dim(x, dim, keepdim=False): return _call(lib.applegpu_eager_sum_dim, x.id, dim, keepdim)
def embedding(w, idx): return _call(lib.applegpu_eager_embedding, w.id, idx.id)
def layer_norm(x, g, b, eps=1e-5): return _call(lib.applegpu_eager_layer_norm, x.id, g.id, b.id, eps)
def gelu(x): return _call(lib.applegpu_eager_gelu, x.id)
def softmax(x): return _call(lib.applegpu_eager_softmax, x.id)
def mse_loss(a, b): return _call(lib.applegpu_eager_mse_loss, a.id, b.id)
def mse_loss_backward(g, a, b): return _call(lib.applegpu_eager_mse_loss_backward, g.id, a.id, b.id)


def linear(x, w, b=None, act=0):
    """act(x @ w^T + b); act 0 none, 1 relu, 2 gelu-tanh, 3 gelu-erf."""
    return _call(lib.applegpu_eager_linear, x.id, w.id, b.id if b is not None else 0, act)


def matmul_masked(a, b, ta, tb, mask):
    """(op(a) @ op(b)) where mask > 0, else 0 (matmul + relu backward in one kernel)."""
    return _call(lib.applegpu_eager_matmul_masked, a.id, b.id, ta, tb, mask.id)


def create_view(base, shape, strides, offset=0):
    n = len(shape)
    sh = (c_uint64 * n)(*shape)
    st = (c_uint64 * n)(*strides)
    return _call(lib.applegpu_eager_create_view, base.id, sh, st, n, offset)


def add_(self, other, alpha=1.0):
    if lib.applegpu_eager_add_scaled_inplace(self.id, other.id, alpha) != 0:
        raise RuntimeError(eager_error())


def fill_(t, value):
    if lib.applegpu_eager_fill(t.id, float(value)) != 0:
        raise RuntimeError(eager_error())


def op(name: str, tensors, f=(), i=(), nout=1):
    """Any op of the Python surface, run eagerly (applegpu_eager_op)."""
    n = len(tensors)
    ins = (c_uint64 * n)(*[t.id for t in tensors])
    fa = (c_double * len(f))(*f) if f else None
    ia = (c_int64 * len(i))(*i) if i else None
    out = (c_uint64 * nout)()
    r = lib.applegpu_eager_op(name.encode(), ins, n, fa, len(f), ia, len(i), out, nout)
    if r < 0:
        raise RuntimeError(eager_error())
    res = [EagerTensor(out[k], None) for k in range(r)]
    return res[0] if nout == 1 else tuple(res)


def sgd_matmul_(w, a, b, ta=False, tb=False, alpha=1.0, bias=None):
    """w += alpha * op(a) @ op(b) in place: an SGD weight step fused with its
    gradient GEMM (the update runs in the GEMM's epilogue).  With `bias`
    (fp32, [rows of op(a)]) also bias += alpha * op(a).sum(1): for a Linear
    layer's step, op(a) = g^T and this is the bias step bias += alpha *
    g.sum(0); the outer-product plan computes it while packing g."""
    ins = [w, a, b] if bias is None else [w, a, b, bias]
    op("sgd_matmul_", ins, f=(float(alpha),), i=(int(ta), int(tb)))


def linear_backward_sgd_(w, b, g, a, mask=None, alpha=1.0):
    """A Linear layer's backward and SGD step, in place (y = a @ w^T + b,
    upstream gradient g): w += alpha * g^T @ a, b += alpha * g.sum(0).  With
    `mask` also returns (g @ w) where mask > 0, else 0 -- the gradient of the
    layer input through the previous ReLU, from w before the update; without
    it returns None.  A one-output layer (w [1, N], mask the input a itself)
    is one launch."""
    ins = [w, b, g, a] if mask is None else [w, b, g, a, mask]
    r = op("linear_backward_sgd_", ins, f=(float(alpha),))
    return r if mask is not None else None


def linear_mse_backward_sgd_(h, w, b, y, alpha=1.0, grad_in=True):
    """The last Linear layer of an MSE regression through its SGD step, in
    place: z = h @ w^T + b, loss = mean((z - y)^2), then w += alpha * g^T @ h
    and b += alpha * g.sum(0) for g = dloss/dz.  Returns (loss, g_in), g_in
    the gradient of h through the previous ReLU (from w before the update),
    or (loss, None) with grad_in=False.  A one-output layer is two launches."""
    loss, gi = op("linear_mse_backward_sgd_", [h, w, b, y], f=(float(alpha),), i=(int(bool(grad_in)),), nout=2)
    return loss, (gi if grad_in else None)


def linear_relu_mse_backward_sgd_(a, wh, bh, w, b, y, alpha=1.0, grad_in=True):
    """The last hidden layer h = relu(a @ wh^T + bh) and a one-output MSE
    regression layer (w [1, N], b [1]) through the output layer's SGD step,
    as linear(a, wh, bh, act=1) then linear_mse_backward_sgd_(h, w, b, y):
    returns (loss, g_in or None, h).  The hidden GEMM's split-K partial sums
    are reduced by the output layer's forward (three launches instead of
    four)."""
    loss, gi, h = op("linear_relu_mse_backward_sgd_", [a, wh, bh, w, b, y], f=(float(alpha),),
                     i=(int(bool(grad_in)),), nout=3)
    return loss, (gi if grad_in else None), h


def linear_backward_sgd_pair_(w1, b1, g, h, w0, b0, x, alpha=1.0):
    """The backward and SGD steps of the first two Linear layers of a net,
    in place: h = relu(x @ w0^T + b0) feeds the layer (w1, b1), whose output
    gradient is g.  g0 = (g @ w1) * (h > 0) from w1 before its step; then
    w1 += alpha * g^T @ h, b1 += alpha * g.sum(0), w0 += alpha * g0^T @ x and
    b0 += alpha * g0.sum(0).  Large fp32 layers update both weights in one
    pack launch and one GEMM launch."""
    op("linear_backward_sgd_pair_", [w1, b1, g, h, w0, b0, x], f=(float(alpha),))


def mlp2_sgd_step_(x, y, w1, b1, w2, b2, alpha=1.0):
    """One SGD step of Linear(w1, b1) -> ReLU -> Linear(w2, b2) with MSE
    loss against y, in place (w += alpha * grad, every gradient from the
    step's starting parameters); returns the loss [1].  Small fp32 shapes
    (activations within 64 KB) run as one launch."""
    return op("mlp2_sgd_step_", [x, y, w1, b1, w2, b2], f=(float(alpha),))


def sgd_sum_rows_(bias, g, alpha=1.0):
    """bias += alpha * g.sum(0) in place: an SGD bias step fused with its
    gradient reduction."""
    op("sgd_sum_rows_", [bias, g], f=(float(alpha),))


def mse_loss_grad(out, y):
    """(mean((out - y)^2), d loss / d out) in one launch."""
    return op("mse_loss_grad", [out, y], nout=2)


def synchronize():
    lib.applegpu_eager_flush_and_wait()
