"""GEMM (MFMA) and fused attention parity against the oracle: every operand
layout, batching, split-K, the fused epilogues, fp16/bf16, ragged and
degenerate shapes."""
import math

import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(77)


def f32(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def test_mfma_exact_small_integers(gpu):
    """Small integers are exact in fp32: any lane/row mapping error in the MFMA
    tiles shows up as a wrong integer."""
    a = RNG.integers(-3, 4, (131, 70)).astype(np.float32)
    b = RNG.integers(-3, 4, (70, 133)).astype(np.float32)
    got = (gpu.from_numpy(a) @ gpu.from_numpy(b)).to_numpy()
    np.testing.assert_array_equal(got, a @ b)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (2, 3, 4), (37, 45, 29), (64, 64, 64), (128, 768, 2304),
                                   (256, 4096, 128), (200, 300, 500), (7, 2000, 9), (128, 768, 50257)])
def test_matmul_shapes(gpu, m, k, n):
    a, b = f32(m, k), f32(k, n)
    got = (gpu.from_numpy(a) @ gpu.from_numpy(b)).to_numpy()
    assert rel_err(got, O.matmul(a, b)) < 1e-3


def test_matmul_golden(gpu, fixtures):
    got = (gpu.from_numpy(fixtures["matmul_a"]) @ gpu.from_numpy(fixtures["matmul_b"])).to_numpy()
    np.testing.assert_allclose(got, fixtures["matmul_y"], rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_transposed_operands_in_place(gpu, ta, tb):
    m, k, n = 96, 130, 72
    a = f32(k, m) if ta else f32(m, k)
    b = f32(n, k) if tb else f32(k, n)
    A, B = gpu.from_numpy(a), gpu.from_numpy(b)
    if ta:
        A = gpu.transpose(A)
    if tb:
        B = gpu.transpose(B)
    got = (A @ B).to_numpy()
    assert rel_err(got, O.matmul_ex(a, b, ta, tb)) < 1e-3


def test_batched_and_broadcast(gpu):
    a, b = f32(3, 4, 33, 20), f32(3, 4, 20, 17)
    assert rel_err((gpu.from_numpy(a) @ gpu.from_numpy(b)).to_numpy(), O.matmul(a, b)) < 1e-3
    b2 = f32(20, 17)  # 2-D B shared by every batch
    assert rel_err((gpu.from_numpy(a) @ gpu.from_numpy(b2)).to_numpy(), O.matmul(a, b2)) < 1e-3
    b3 = f32(4, 20, 17)  # batch broadcast [3,4] x [4]
    assert rel_err((gpu.from_numpy(a) @ gpu.from_numpy(b3)).to_numpy(), O.matmul(a, b3)) < 1e-3


@pytest.mark.parametrize("k", [4096, 8192])
def test_split_k_skinny(gpu, k):
    a, b = f32(64, k), f32(k, 192)
    got = (gpu.from_numpy(a) @ gpu.from_numpy(b)).to_numpy()
    assert rel_err(got, O.matmul(a, b)) < 1e-3


def test_fused_epilogues_through_graph(gpu):
    """matmul -> add_bias -> gelu and matmul -> add_bias -> + residual are fused
    into one GEMM launch each; results equal the unfused oracle."""
    x, w, b, r = f32(70, 96), f32(96, 130), f32(130), f32(70, 130)
    before = gpu.graph_stats()["fused_gemm_epilogues"]
    y = gpu.gelu(gpu.add_bias(gpu.from_numpy(x) @ gpu.from_numpy(w), gpu.from_numpy(b)))
    z = gpu.from_numpy(r) + gpu.add_bias(gpu.from_numpy(x) @ gpu.from_numpy(w), gpu.from_numpy(b))
    y_np, z_np = y.to_numpy(), z.to_numpy()
    after = gpu.graph_stats()["fused_gemm_epilogues"]
    assert after - before == 2
    ref = O.add_bias(O.matmul(x, w), b)
    assert rel_err(y_np, O.gelu_tanh(ref)) < 1e-3
    assert rel_err(z_np, r + ref) < 1e-3


@pytest.mark.parametrize("xshape,rshape", [((1, 96), (70, 130)), ((70, 96), (3, 70, 130))])
def test_broadcasting_residual_stays_unfused(gpu, xshape, rshape):
    """An add that broadcasts the GEMM output ([1,N] + [M,N], or a 2-D
    product + a 3-D residual) is evaluated as its own node, with the same
    numbers as op by op."""
    x, w, b, r = f32(*xshape), f32(96, 130), f32(130), f32(*rshape)
    z = gpu.from_numpy(r) + gpu.add_bias(gpu.from_numpy(x) @ gpu.from_numpy(w), gpu.from_numpy(b))
    got = z.to_numpy()
    assert got.shape == np.broadcast_shapes(rshape, (xshape[0], 130))
    assert rel_err(got, r + O.add_bias(O.matmul(x, w), b)) < 1e-3
    # the residual on the other side of the add
    z2 = gpu.add_bias(gpu.from_numpy(x) @ gpu.from_numpy(w), gpu.from_numpy(b)) + gpu.from_numpy(r)
    assert rel_err(z2.to_numpy(), r + O.add_bias(O.matmul(x, w), b)) < 1e-3


def test_linear_relu(gpu):
    x, w, b = f32(33, 64), f32(48, 64), f32(48)
    got = gpu.linear(gpu.from_numpy(x), gpu.from_numpy(w), gpu.from_numpy(b), "relu").to_numpy()
    assert rel_err(got, O.relu(O.linear(x, w, b))) < 1e-3


@pytest.mark.parametrize("dt,tol", [("float16", 1e-2), ("bfloat16", 2e-2)])
@pytest.mark.parametrize("m,k,n", [(64, 64, 64), (130, 200, 70), (512, 1280, 1280)])
def test_matmul_half(gpu, dt, tol, m, k, n):
    a, b = f32(m, k), f32(k, n)
    A, B = gpu.cast(gpu.from_numpy(a), dt), gpu.cast(gpu.from_numpy(b), dt)
    got = (A @ B).to_numpy().astype(np.float32)
    ar = A.to_numpy().astype(np.float32)
    br = B.to_numpy().astype(np.float32)
    assert rel_err(got, O.matmul(ar, br)) < tol
    got_t = (A @ gpu.transpose(gpu.cast(gpu.from_numpy(b.T.copy()), dt))).to_numpy().astype(np.float32)
    assert rel_err(got_t, O.matmul(ar, br)) < tol


# ── attention ──────────────────────────────────────────────────────────────
def test_attention_golden(gpu, fixtures):
    q, k, v = (gpu.from_numpy(fixtures[f"attn_{n}"]) for n in "qkv")
    np.testing.assert_allclose(gpu.attention_causal(q, k, v).to_numpy(), fixtures["attn_causal_y"], rtol=1e-3,
                               atol=1e-4)
    np.testing.assert_allclose(gpu.attention(q, k, v).to_numpy(), fixtures["attn_full_y"], rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("h,tq,tk,d,causal", [(12, 128, 128, 64, True), (2, 1, 37, 64, False),
                                              (3, 65, 65, 64, True), (1, 200, 200, 128, True),
                                              (4, 5, 300, 64, False), (2, 64, 64, 32, True),
                                              (2, 10, 10, 16, True)])
def test_attention_shapes(gpu, h, tq, tk, d, causal):
    q, k, v = f32(h, tq, d), f32(h, tk, d), f32(h, tk, d)
    fn = gpu.attention_causal if causal else gpu.attention
    got = fn(gpu.from_numpy(q), gpu.from_numpy(k), gpu.from_numpy(v)).to_numpy()
    assert rel_err(got, O.attention(q, k, v, causal)) < 1e-3


def test_attention_strided_heads_from_fused_qkv(gpu):
    """Q/K/V as head views of one [T, 3*d] projection (the GPT-2 layout) and
    the head-merge transpose; no copies needed, same numbers."""
    T, H, hd = 100, 12, 64
    d = H * hd
    qkv = f32(T, 3 * d)
    t = gpu.from_numpy(qkv)

    def heads(lo):
        return gpu.transpose_dims(gpu.reshape(gpu.slice(t, 1, lo, lo + d), [T, H, hd]), 0, 1)

    out = gpu.attention_causal(heads(0), heads(d), heads(2 * d))
    merged = gpu.reshape(gpu.transpose_dims(out, 0, 1), [T, d]).to_numpy()
    qn, kn, vn = (qkv[:, j * d:(j + 1) * d].reshape(T, H, hd).transpose(1, 0, 2) for j in range(3))
    ref = O.attention(qn, kn, vn, True).transpose(1, 0, 2).reshape(T, d)
    assert rel_err(merged, ref) < 1e-3


@pytest.mark.parametrize("dt,tol", [("float16", 1e-2), ("bfloat16", 2e-2)])
def test_attention_half(gpu, dt, tol):
    q, k, v = f32(4, 96, 64), f32(4, 96, 64), f32(4, 96, 64)
    tq, tk, tv = (gpu.cast(gpu.from_numpy(a), dt) for a in (q, k, v))
    got = gpu.attention_causal(tq, tk, tv).to_numpy().astype(np.float32)
    ref = O.attention(*(t.to_numpy().astype(np.float32) for t in (tq, tk, tv)), causal=True)
    assert rel_err(got, ref) < tol


def test_attention_unsupported_head_dim_uses_composition(gpu):
    q, k, v = f32(2, 9, 24), f32(2, 9, 24), f32(2, 9, 24)
    got = gpu.attention_causal(gpu.from_numpy(q), gpu.from_numpy(k), gpu.from_numpy(v)).to_numpy()
    assert rel_err(got, O.attention(q, k, v, True)) < 1e-3
