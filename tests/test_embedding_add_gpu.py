"""Token + position embedding and the layer_norm that reads the sum, run as
one kernel by the graph executor (GPT-2's wte[ids] + wpe[pos] -> ln_1,
python/applegpu_runtime/models/gpt2.py:84-178).  The fused launch must give
the four-launch result bit for bit: the sum is rounded once to the table
dtype and layer_norm reads the rounded sum.  Indices outside a table give a
zero row from that table, as the embedding kernel does; widths past 2048
columns run unfused."""
import numpy as np
import pytest

from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4242)


def _case(gpu, dt, rows, cols, vocab, fuse_ln, idx_dt=np.int32, bad=False):
    w1 = RNG.standard_normal((vocab, cols)).astype(np.float32) * 0.1
    w2 = RNG.standard_normal((64, cols)).astype(np.float32) * 0.1
    i1 = RNG.integers(0, vocab, rows).astype(idx_dt)
    i2 = (np.arange(rows) % 64).astype(idx_dt)
    if bad:
        i1[0], i2[1] = vocab + 3, -1
    g = (RNG.standard_normal(cols) * 0.2 + 1).astype(np.float32)
    b = (RNG.standard_normal(cols) * 0.1).astype(np.float32)
    cast = (lambda t: t) if dt == "float32" else (lambda t: gpu.cast(t, dt))
    tw1, tw2, tg, tb = (cast(gpu.from_numpy(a)) for a in (w1, w2, g, b))
    for t in (tw1, tw2, tg, tb):  # parameters are materialised, as a model's are
        t.eval()
    ti1, ti2 = gpu.from_numpy(i1), gpu.from_numpy(i2)

    def build(split):
        e1, e2 = gpu.embedding(tw1, ti1), gpu.embedding(tw2, ti2)
        if split:
            e1.eval()
            e2.eval()
        x = e1 + e2
        if split:
            x.eval()
        y = gpu.layer_norm(x, tg, tb, 1e-5) if fuse_ln else None
        return x, y

    before = gpu.graph_stats()["launches_saved"]
    x, y = build(False)
    # y first: its evaluation reaches the sum too, so both run in one launch
    ys = y.to_numpy() if fuse_ln else None
    xs = x.to_numpy()
    saved = gpu.graph_stats()["launches_saved"] - before
    x2, y2 = build(True)
    np.testing.assert_array_equal(xs, x2.to_numpy())
    if fuse_ln:
        np.testing.assert_array_equal(ys, y2.to_numpy())
    ref = O.embedding(w1, np.clip(i1, 0, vocab - 1)) + O.embedding(w2, np.clip(i2, 0, 63))
    if bad:
        ref[0] = w2[i2[0]]
        ref[1] = w1[i1[1]]
    tol = 1e-6 if dt == "float32" else 1e-2
    np.testing.assert_allclose(np.asarray(xs, np.float32), ref, rtol=tol, atol=tol)
    return saved


@pytest.mark.parametrize("dt", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("rows,cols", [(128, 768), (8, 1280), (37, 100), (4096, 1280)])
def test_embedding_add_layer_norm_is_bitwise_the_unfused_result(gpu, dt, rows, cols):
    assert _case(gpu, dt, rows, cols, 500, True) >= 3


def test_embedding_add_without_layer_norm_and_edges(gpu):
    assert _case(gpu, "float32", 64, 768, 300, False) >= 2
    _case(gpu, "float32", 16, 256, 50, True, idx_dt=np.int64, bad=True)
    assert _case(gpu, "float32", 16, 2500, 50, True) == 0   # wider than a wavefront's row: unfused


def test_gpt2_forward_unchanged(gpu):
    """The forward (whose first op pair fuses) against the float64 oracle."""
    from applegpu_runtime.models import gpt2 as G
    from oracle import models as M
    from conftest import rel_err
    cfg = {"vocab_size": 400, "n_positions": 64, "n_embd": 128, "n_layer": 2, "n_head": 2}
    w = G.random_weights(cfg, seed=12)
    ids = RNG.integers(0, cfg["vocab_size"], 33).astype(np.int32)
    got, _ = G.gpt2_forward(G.load_model(w, cfg), ids, need_cache=False)
    ref, _ = M.gpt2_forward_np(w, cfg, ids)
    assert rel_err(got.to_numpy(), ref) < 1e-3
