"""qkv_attention: GPT-2's QKV projection, head split and causal attention as
one op (models/gpt2.py:84-178's c_attn -> split -> attention_causal).  With
read_partials the fp32 attention kernel reads the projection's split-K
partial sums plus the bias; either way the values must equal the composed
ops' bit for bit (same partial-sum order, same bias add) and the float64
oracle within the fp32 bar."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(6262)


def f32(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def _composed(gpu, x, w, b, H, batch, causal):
    R, d = x.shape[0], w.shape[1] // 3
    T, hd = R // batch, d // H
    qkv = gpu.add_bias(x @ w, b)

    def heads(lo):
        return gpu.transpose_dims(gpu.reshape(gpu.slice(qkv, 1, lo, lo + d), [batch, T, H, hd]), 1, 2)

    fn = gpu.attention_causal if causal else gpu.attention
    a = fn(heads(0), heads(d), heads(2 * d))
    return gpu.reshape(gpu.transpose_dims(a, 1, 2), [R, d])


def _oracle(x, w, b, H, batch, causal):
    R, d = x.shape[0], w.shape[1] // 3
    T, hd = R // batch, d // H
    qkv = x.astype(np.float64) @ w.astype(np.float64) + b
    q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(batch, T, H, hd).transpose(0, 2, 1, 3) for j in range(3))
    a = O.attention(q, k, v, causal)
    return a.transpose(0, 2, 1, 3).reshape(R, d)


@pytest.mark.parametrize("batch,T,K,d,H,causal", [
    (1, 128, 768, 768, 12, True),    # GPT-2 small layer (4 K splits)
    (1, 100, 768, 768, 12, True),    # ragged sequence
    (2, 64, 512, 256, 4, True),      # two sequences
    (1, 96, 3072, 256, 2, True),     # head dim 128, 8 K splits
    (1, 80, 768, 768, 12, False),    # full attention
])
def test_qkv_attention_matches_composed_and_oracle(gpu, batch, T, K, d, H, causal):
    x, w, b = f32(batch * T, K), f32(K, 3 * d, scale=0.05), f32(3 * d, scale=0.1)
    tx, tw, tb = gpu.from_numpy(x), gpu.from_numpy(w), gpu.from_numpy(b)
    ref = _composed(gpu, tx, tw, tb, H, batch, causal).to_numpy()
    for partials in (False, True):
        got = gpu.qkv_attention(tx, tw, tb, H, causal=causal, batch=batch, read_partials=partials).to_numpy()
        np.testing.assert_array_equal(got, ref)
        assert rel_err(got, _oracle(x, w, b, H, batch, causal)) < 1e-4  # fp32 bar 1e-3


def test_qkv_attention_unsplit_shape_falls_back(gpu):
    """A projection without a K split (K of one slice) runs as separate ops."""
    x, w, b = f32(128, 64), f32(64, 3 * 128, scale=0.1), f32(3 * 128, scale=0.1)
    got = gpu.qkv_attention(gpu.from_numpy(x), gpu.from_numpy(w), gpu.from_numpy(b), 2, read_partials=True).to_numpy()
    assert rel_err(got, _oracle(x, w, b, 2, 1, True)) < 1e-4


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_qkv_attention_16bit_composes(gpu, dt):
    x, w, b = f32(64, 256), f32(256, 3 * 128, scale=0.05), f32(3 * 128, scale=0.1)
    tx, tw, tb = (gpu.cast(gpu.from_numpy(v), dt) for v in (x, w, b))
    got = gpu.qkv_attention(tx, tw, tb, 2).to_numpy().astype(np.float32)
    rnd = [t.to_numpy().astype(np.float32) for t in (tx, tw, tb)]
    assert rel_err(got, _oracle(*rnd, 2, 1, True)) < 2e-2


def test_qkv_attention_rejects_bad_shapes(gpu):
    x, w, b = gpu.from_numpy(f32(8, 16)), gpu.from_numpy(f32(16, 48)), gpu.from_numpy(f32(48))
    with pytest.raises(ValueError):
        gpu.qkv_attention(x, w, b, 5).eval()           # 16 columns in 5 heads
    with pytest.raises(ValueError):
        gpu.qkv_attention(x, w, b, 2, batch=3).eval()  # 8 rows in 3 sequences
    with pytest.raises(ValueError):
        gpu.qkv_attention(x, gpu.from_numpy(f32(16, 47)), b, 2).eval()


def test_gpt2_forward_without_cache_is_identical(gpu):
    """need_cache=False (qkv_attention per layer) gives the same logits as the
    composed forward, and both match the oracle."""
    from applegpu_runtime.models import gpt2 as G
    from oracle import models as M
    cfg = {"vocab_size": 500, "n_positions": 128, "n_embd": 128, "n_layer": 2, "n_head": 2}
    w = G.random_weights(cfg, seed=5)
    model = G.load_model(w, cfg, x3=False)   # qkv_attention serves unpacked fp32 weights
    ids = RNG.integers(0, cfg["vocab_size"], 40).astype(np.int32)
    a, cache_a = G.gpt2_forward(model, ids)
    b, cache_b = G.gpt2_forward(model, ids, need_cache=False)
    assert cache_b is None and len(cache_a) == cfg["n_layer"]
    np.testing.assert_array_equal(a.to_numpy(), b.to_numpy())
    ref, _ = M.gpt2_forward_np(w, cfg, ids)
    assert rel_err(b.to_numpy(), ref) < 1e-3
