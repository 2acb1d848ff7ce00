"""Fused attention on the MFMA kernels (16-bit, and fp32 on native fp32
MFMA): parity with the oracle's
softmax(Q K^T / sqrt(d)) V (crates/core/src/ops.rs:1531-1620, causal mask with
the diagonal at (0,0), kernel_templates.rs:468-497) on the fp16/bf16-rounded
inputs, over the shapes that exercise its tiling: 64- and 128-row query
blocks, ragged query and key counts, tiles that are fully visible, cut by the
diagonal or by Tk, Tq != Tk with and without the causal mask, d = 64 and 128,
strided head views of a fused QKV projection, and the scalar kernel that
takes misaligned rows."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(1234)
TOL = 1e-2  # fp16 / bf16 bar, normwise (max |err| / max |ref|)


def _inputs(gpu, dt, shapes, scale=1.0):
    dev = [gpu.cast(gpu.from_numpy((RNG.standard_normal(s) * scale).astype(np.float32)), dt) for s in shapes]
    host = [t.to_numpy().astype(np.float32) for t in dev]  # the rounded values the kernel sees
    return dev, host


def _row_err(got, ref):
    """Largest error of any query row relative to that row's largest value."""
    num = np.abs(got - ref).max(axis=-1)
    den = np.maximum(np.abs(ref).max(axis=-1), 1e-6)
    return float((num / den).max())


@pytest.mark.parametrize("dt", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("b,h,tq,tk,d,causal", [
    (8, 20, 512, 512, 64, True),    # C4 prefill: 128-row blocks (fp32: 64-row blocks)
    (1, 12, 128, 128, 64, True),    # 64-row blocks
    (2, 3, 65, 65, 64, True),       # ragged, partial last tile
    (1, 2, 200, 200, 128, True),    # d = 128
    (2, 4, 5, 300, 64, False),      # Tq < Tk, no mask: last key tile cut by Tk
    (1, 2, 1, 37, 64, False),       # one query, Tk below one tile
    (1, 2, 130, 70, 64, True),      # causal, Tq > Tk: late queries see every key
    (1, 2, 70, 130, 64, True),      # causal, Tq < Tk: keys past the last query unseen
    (1, 3, 64, 64, 64, False),      # exact tiles
    (3, 5, 257, 257, 128, False),   # d = 128, full attention, ragged
])
def test_attention_mfma_matches_oracle(gpu, dt, b, h, tq, tk, d, causal):
    """fp32 runs the fp32 MFMA kernel: 64-query blocks when they fill the GPU,
    else 16-query blocks with the keys split across wavefronts (GPT-2 at 128
    tokens); fp32 bar 1e-3, checked at 1e-4."""
    (q, k, v), (qn, kn, vn) = _inputs(gpu, dt, [(b, h, tq, d), (b, h, tk, d), (b, h, tk, d)])
    fn = gpu.attention_causal if causal else gpu.attention
    got = fn(q, k, v).to_numpy().astype(np.float32)
    ref = O.attention(qn, kn, vn, causal)
    tol = 1e-4 if dt == "float32" else TOL
    assert rel_err(got, ref) < tol
    assert _row_err(got, ref) < 2 * tol


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_attention_mfma_peaked_scores(gpu, dt):
    """Large score ranges (one key dominating each row) exercise the running
    max: a wrong rescale shows up as a wrong weighted value."""
    (q, k, v), (qn, kn, vn) = _inputs(gpu, dt, [(2, 2, 160, 64), (2, 2, 160, 64), (2, 2, 160, 64)], scale=3.0)
    got = gpu.attention_causal(q, k, v).to_numpy().astype(np.float32)
    ref = O.attention(qn, kn, vn, True)
    assert rel_err(got, ref) < TOL


def test_attention_mfma_onehot_values_return_probabilities(gpu):
    """V = identity (key j -> unit vector j): the output row is the probability
    row itself, so a key permuted inside the transposed V tile, or a query
    row paired with the wrong probabilities, cannot cancel out."""
    T = 64
    (q, k), (qn, kn) = _inputs(gpu, "float16", [(1, 1, T, 64), (1, 1, T, 64)])
    eye = np.eye(T, 64, dtype=np.float32)[None, None]
    v = gpu.cast(gpu.from_numpy(eye), "float16")
    got = gpu.attention_causal(q, k, v).to_numpy().astype(np.float32)[0, 0]
    s = (qn[0, 0].astype(np.float64) @ kn[0, 0].astype(np.float64).T) / 8.0
    s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(got, p, atol=2e-3)
    assert (got[np.triu_indices(T, 1)] == 0).all()  # masked keys carry exactly zero weight


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_attention_mfma_fused_qkv_heads(gpu, dt):
    """GPT-2 layout: Q/K/V are head views of one [B*T, 3*d] projection
    (row stride 3*d), as the model feeds them."""
    B, T, H, hd = 2, 100, 12, 64
    d = H * hd
    (t,), (qkv,) = _inputs(gpu, dt, [(B, T, 3 * d)])

    def heads(lo):
        return gpu.transpose_dims(gpu.reshape(gpu.slice(t, 2, lo, lo + d), [B, T, H, hd]), 1, 2)

    got = gpu.attention_causal(heads(0), heads(d), heads(2 * d)).to_numpy().astype(np.float32)
    qn, kn, vn = (qkv[:, :, j * d:(j + 1) * d].reshape(B, T, H, hd).transpose(0, 2, 1, 3) for j in range(3))
    assert rel_err(got, O.attention(qn, kn, vn, True)) < TOL


def test_attention_misaligned_rows_take_scalar_kernel(gpu):
    """A row stride that is not a multiple of 8 elements cannot use 16-byte
    loads: the scalar kernel runs and gives the same answer."""
    T, hd = 40, 64
    (t,), (x,) = _inputs(gpu, "float16", [(T, 3 * hd + 1)])
    q, k, v = (gpu.slice(t, 1, j * hd, (j + 1) * hd) for j in range(3))  # [T, hd], row stride 3*hd+1
    got = gpu.attention_causal(q, k, v).to_numpy().astype(np.float32)
    qn, kn, vn = (x[:, j * hd:(j + 1) * hd] for j in range(3))
    assert rel_err(got, O.attention(qn, kn, vn, True)) < TOL


def test_attention_mfma_deterministic(gpu):
    (q, k, v), _ = _inputs(gpu, "float16", [(2, 4, 300, 64)] * 3)
    a = gpu.attention_causal(q, k, v).to_numpy()
    b = gpu.attention_causal(q, k, v).to_numpy()
    np.testing.assert_array_equal(a, b)
