"""numpy restatement of the reference's hot-path ops (test infrastructure only).

Arithmetic is float32 like the reference kernels (fp32 accumulate); where a
reduction order is unspecified, float64 accumulation is used so the oracle is
at least as accurate as any fp32 order.  Reference paths are relative to the
reference checkout.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


# ── elementwise ────────────────────────────────────────────────────────────
def broadcast_binary(op: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """crates/core/src/eager.rs:246-342 (numpy broadcasting, tensor.rs:148-168)."""
    if op == "add": return a + b
    if op == "sub": return a - b
    if op == "mul": return a * b
    if op == "div": return a / b
    raise ValueError(op)


def relu(x):
    """max(x, 0) — crates/core/src/kernel_templates.rs:119-168."""
    return np.maximum(x, 0).astype(x.dtype)


def gelu_tanh(x):
    """0.5 x (1 + tanh(clamp(0.7978845608 (x + 0.044715 x^3), -10, 10)))
    — crates/core/src/kernel_templates.rs:272-307 (clamp :300-301)."""
    xd = x.astype(np.float64)
    inner = np.clip(0.7978845608 * (xd + 0.044715 * xd ** 3), -10.0, 10.0)
    return (0.5 * xd * (1.0 + np.tanh(inner))).astype(F32)


def gelu_erf(x):
    """x/2 (1 + erf(x/sqrt 2)) — exact GELU; the reference's MSL uses the
    Abramowitz-Stegun erf approximation (kernel_templates.rs:311-360, max err
    1.5e-7), this oracle uses the exact erf."""
    v = np.vectorize(math.erf)
    xd = x.astype(np.float64)
    return (0.5 * xd * (1.0 + v(xd / math.sqrt(2.0)))).astype(F32)


def threshold_backward(grad, x, thr=0.0):
    """grad where x > thr else 0 — crates/core/src/kernel_templates.rs:1996-2020."""
    return np.where(x > thr, grad, np.zeros_like(grad)).astype(grad.dtype)


def add_bias(x, bias):
    """out[i] = x[i] + bias[(i / channel_stride) % C], channel = dim 1
    — crates/core/src/kernel_templates.rs:747-762, ops.rs:1322-1365."""
    shape = [1] * x.ndim
    shape[1] = bias.shape[0]
    return (x + bias.reshape(shape)).astype(x.dtype)


# ── rows ───────────────────────────────────────────────────────────────────
def softmax(x):
    """m = max, e = exp(x - m), e / sum(e) over the last dim
    — crates/core/src/kernel_templates.rs:398-430."""
    xd = x.astype(np.float64)
    m = xd.max(axis=-1, keepdims=True)
    e = np.exp(xd - m)
    return (e / e.sum(axis=-1, keepdims=True)).astype(x.dtype)


def log_softmax(x):
    """x - m - log(sum(exp(x - m))) — crates/core/src/kernel_templates.rs:434-465."""
    xd = x.astype(np.float64)
    m = xd.max(axis=-1, keepdims=True)
    return (xd - m - np.log(np.exp(xd - m).sum(axis=-1, keepdims=True))).astype(x.dtype)


def softmax_causal(x):
    """Per matrix of the last two dims: row i sees columns j <= i (diagonal at
    (0,0)), zeros above — crates/core/src/kernel_templates.rs:468-497."""
    rows, cols = x.shape[-2], x.shape[-1]
    mask = np.arange(cols)[None, :] <= np.arange(rows)[:, None]
    xd = np.where(mask, x.astype(np.float64), -np.inf)
    m = xd.max(axis=-1, keepdims=True)
    e = np.where(mask, np.exp(xd - m), 0.0)
    return (e / e.sum(axis=-1, keepdims=True)).astype(x.dtype)


def layer_norm(x, gamma, beta, eps=1e-5):
    """Two-pass mean, population variance, y = gamma (x - mean) / sqrt(var + eps) + beta
    — crates/core/src/kernel_templates.rs:1075-1116 (eps default 1e-5, crates/python/src/lib.rs:911)."""
    xd = x.astype(np.float64)
    mean = xd.mean(axis=-1, keepdims=True)
    var = ((xd - mean) ** 2).mean(axis=-1, keepdims=True)
    return (gamma.astype(np.float64) * (xd - mean) / np.sqrt(var + eps) + beta.astype(np.float64)).astype(x.dtype)


def argmax(x):
    """Last-dim argmax, first maximum wins, int32 — crates/core/src/kernel_templates.rs:500-520.
    NaN: counted as the maximum (first NaN wins), as torch.argmax does on the CPU."""
    x = np.asarray(x)
    flat = x.reshape(-1, x.shape[-1])
    out = np.empty(flat.shape[0], np.int32)
    for r, row in enumerate(flat):
        nan = np.isnan(row) if np.issubdtype(row.dtype, np.floating) else np.zeros(row.shape, bool)
        out[r] = int(np.argmax(nan)) if nan.any() else int(np.argmax(row))
    shp = x.shape[:-1] if x.ndim > 1 else (1,)
    return out.reshape(shp)


# ── reductions / loss ──────────────────────────────────────────────────────
def sum_dim(x, dim, keepdim=False):
    """crates/core/src/eager.rs:827-855 (output shape; a 0-D result becomes [1])."""
    out = x.astype(np.float64).sum(axis=dim, keepdims=keepdim).astype(x.dtype)
    return out.reshape(1) if out.ndim == 0 else out


def mean_all(x):
    """crates/core/src/eager.rs:710-769 -> one element [1]."""
    return np.array([x.astype(np.float64).mean()], dtype=x.dtype)


def mse_loss(a, b):
    """mean((a - b)^2) — backend_cpp/applegpu_backend.cpp:801-832."""
    d = a.astype(np.float64) - b.astype(np.float64)
    return np.array([(d * d).mean()], dtype=a.dtype)


def mse_loss_backward(g, a, b):
    """(a - b) * 2/n * g — backend_cpp/applegpu_backend.cpp:835-867."""
    n = a.size
    return ((a.astype(np.float64) - b.astype(np.float64)) * (2.0 / n) * float(g.reshape(-1)[0])).astype(a.dtype)


# ── backward ops of the transformer blocks ────────────────────────────────
def softmax_backward(dy, y):
    """y * (dy - sum(dy * y)) per row — crates/core/src/kernel_templates.rs:1562-1597."""
    dy64, y64 = dy.astype(np.float64), y.astype(np.float64)
    return (y64 * (dy64 - (dy64 * y64).sum(-1, keepdims=True))).astype(dy.dtype)


def layer_norm_backward(dy, x, gamma, eps=1e-5, params=False):
    """dx = inv (dy g - mean(dy g) - xhat mean(dy g xhat)), statistics from x
    (two-pass mean, population variance) — kernel_templates.rs:1601-1659;
    with params also dgamma = sum_rows(dy xhat), dbeta = sum_rows(dy)
    (python/applegpu_runtime/torch_backend.py:1652-1692 computes those)."""
    x64, dy64, g64 = x.astype(np.float64), dy.astype(np.float64), gamma.astype(np.float64)
    mean = x64.mean(-1, keepdims=True)
    inv = 1.0 / np.sqrt(((x64 - mean) ** 2).mean(-1, keepdims=True) + eps)
    xh = (x64 - mean) * inv
    dg = dy64 * g64
    dx = inv * (dg - dg.mean(-1, keepdims=True) - xh * (dg * xh).mean(-1, keepdims=True))
    if not params:
        return dx.astype(x.dtype)
    flat = (-1, x.shape[-1])
    return (dx.astype(x.dtype), (dy64 * xh).reshape(flat).sum(0).astype(x.dtype),
            dy64.reshape(flat).sum(0).astype(x.dtype))


def gelu_tanh_backward(dy, x):
    """dy * d/dx gelu_tanh(x), inner term clamped to +-10 — kernel_templates.rs:2074-2122."""
    x64 = x.astype(np.float64)
    k = math.sqrt(2.0 / math.pi)
    t = np.tanh(np.clip(k * (x64 + 0.044715 * x64 ** 3), -10.0, 10.0))
    d = 0.5 * (1.0 + t) + 0.5 * x64 * (1.0 - t * t) * k * (1.0 + 3.0 * 0.044715 * x64 * x64)
    return (dy.astype(np.float64) * d).astype(dy.dtype)


def gelu_erf_backward(dy, x):
    """dy * (Phi(x) + x phi(x)) — kernel_templates.rs:2126-2152 (erf from math.erf)."""
    x64 = x.astype(np.float64)
    cdf = 0.5 * (1.0 + np.vectorize(math.erf)(x64 / math.sqrt(2.0)))
    pdf = np.exp(-0.5 * x64 * x64) / math.sqrt(2.0 * math.pi)
    return (dy.astype(np.float64) * (cdf + x64 * pdf)).astype(dy.dtype)


def embedding_backward(dy, idx, num_weights):
    """Row w = sum of dy rows whose index is w — ops.rs:915-960,
    kernel_templates.rs:1867-1913.  Added in token order in float32, the
    order the device kernel uses, so results compare bit for bit; indices
    outside [0, num_weights) add nothing."""
    idx = np.asarray(idx).reshape(-1)
    rows = dy.reshape(idx.size, -1).astype(np.float32)
    out = np.zeros((num_weights, rows.shape[1]), np.float32)
    for i, w in enumerate(idx):
        if 0 <= w < num_weights:
            out[w] = out[w] + rows[i]
    return out.astype(dy.dtype)


# ── GEMM / attention ───────────────────────────────────────────────────────
def matmul(a, b):
    """Batched row-major C = A @ B with fp32 results; batch dims broadcast and a
    2-D B is shared by every batch (lazy path, crates/core/src/lazy.rs:2389-2409;
    ops.rs:390-462).  Accumulates in float64."""
    return np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.result_type(a.dtype, np.float32))


def matmul_ex(a, b, ta=False, tb=False):
    """GEMM reading transposed operands in place — crates/core/src/eager.rs:485-560."""
    if ta: a = np.swapaxes(a, -1, -2)
    if tb: b = np.swapaxes(b, -1, -2)
    return matmul(a, b)


def linear(x, w, b=None):
    """x W^T + b (torch Linear) — backend_cpp/applegpu_backend.cpp:584-620."""
    y = np.matmul(x.astype(np.float64), w.astype(np.float64).T)
    if b is not None:
        y = y + b.astype(np.float64)
    return y.astype(F32)


def attention(q, k, v, causal=False):
    """softmax[_causal](Q K^T * (1/sqrt(d_k))) V — crates/core/src/ops.rs:1531-1620
    (scale applied after the product, :1556-1557)."""
    dk = q.shape[-1]
    s = np.matmul(q.astype(np.float64), np.swapaxes(k.astype(np.float64), -1, -2))
    s = s * (1.0 / math.sqrt(dk))
    if causal:
        rows, cols = s.shape[-2], s.shape[-1]
        mask = np.arange(cols)[None, :] <= np.arange(rows)[:, None]
        s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    p = e / e.sum(axis=-1, keepdims=True)
    return np.matmul(p, v.astype(np.float64)).astype(q.dtype)


# ── indexing ───────────────────────────────────────────────────────────────
def embedding(w, idx):
    """out[i, :] = W[idx[i], :] — crates/core/src/kernel_templates.rs:1119-1143."""
    return w[np.asarray(idx, dtype=np.int64)]


def gather(x, dim, idx):
    """out = x gathered along dim by idx (idx shaped like out) — kernel_templates.rs:870-975."""
    return np.take_along_axis(x, np.asarray(idx, dtype=np.int64), axis=dim)


def index_select(x, dim, idx):
    """kernel_templates.rs:870-975."""
    return np.take(x, np.asarray(idx, dtype=np.int64), axis=dim)


# ── quantization ───────────────────────────────────────────────────────────
def quantize_per_tensor(x, scale, zero_point=0, dtype="int8"):
    """clamp(round_half_away(x / scale) + zp, lo, hi) with a per-tensor scale
    — crates/core/src/kernel_templates.rs:2193-2218 (MSL round() rounds half
    away from zero)."""
    q = np.asarray(x, dtype=F32) / F32(scale)
    t = np.trunc(q)
    r = t + np.where(np.abs(q - t) >= F32(0.5), np.sign(q), F32(0))  # exact: q - trunc(q) is representable
    r = r + F32(zero_point)
    lo, hi = (-128, 127) if dtype == "int8" else (0, 255)
    return np.clip(r, lo, hi).astype(np.int8 if dtype == "int8" else np.uint8)


def dequantize_per_tensor(q, scale, zero_point=0):
    """(q - zp) * scale — crates/core/src/kernel_templates.rs:2222-2240."""
    return ((q.astype(np.int32) - zero_point).astype(F32) * F32(scale)).astype(F32)


def quantize_per_row(w):
    """Symmetric per-row int8 of the benchmark config: scale = absmax(row)/127
    in fp32, codes = clamp(round_half_even(w / scale), -128, 127); a row of
    zeros has scale 0 and codes 0 (convention of this backend; the fp32
    expression would divide 0 by 0)."""
    w = w.astype(F32)
    scale = (np.abs(w).max(axis=-1) / F32(127)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(w / scale[..., None])
    r = np.where(scale[..., None] == 0, F32(0), r)
    return np.clip(r, -128, 127).astype(np.int8), scale


def dequantize_per_row(q, scale):
    """q * scale[row] in fp32."""
    return (q.astype(F32) * scale[..., None].astype(F32)).astype(F32)
