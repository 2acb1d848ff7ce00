"""Backward kernels of the transformer blocks against the oracle
(ops.rs:655-728, 915-960, 1090-1158 of the reference; its tests at
ops.rs:4573-4811, 4973-5035 and python/tests/test_backward_ops.py):
layer_norm (dx, and dgamma/dbeta), softmax, gelu (tanh and erf forms) and
embedding.  fp32 bars: 1e-5 relative for the row and elementwise kernels;
embedding_backward is bit-exact (the device adds rows in token order, as
the oracle does); 16-bit within 1e-2.  Then the same ops under torch
autograd on the `applegpu` device: a GPT-2-style block trains with no CPU
fallback."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(8181)


def f32(*shape, scale=1.0, shift=0.0):
    return (RNG.standard_normal(shape) * scale + shift).astype(np.float32)


def _dev(gpu, a, dt="float32"):
    t = gpu.from_numpy(np.ascontiguousarray(a, np.float32))
    return t if dt == "float32" else gpu.cast(t, dt)


def _host(t):
    return np.asarray(t.to_numpy(), np.float32)


def _rnd(gpu, a, dt):
    return a if dt == "float32" else _host(_dev(gpu, a, dt))


# ── layer_norm ──────────────────────────────────────────────────────────────
@pytest.mark.parametrize("shape", [(3, 7), (128, 768), (37, 1280), (16, 2048), (4, 2500), (2, 5, 768), (1000, 64)])
def test_layer_norm_backward(gpu, shape):
    cols = shape[-1]
    x, dy = f32(*shape, scale=2.0, shift=0.5), f32(*shape)
    g = f32(cols, scale=0.5, shift=1.0)
    got = _host(gpu.layer_norm_backward(_dev(gpu, dy), _dev(gpu, x), _dev(gpu, g), 1e-5))
    ref = O.layer_norm_backward(dy, x, g, 1e-5)
    assert got.shape == shape
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("rows,cols", [(4096, 768), (300, 1280), (7, 33), (513, 2500)])
def test_layer_norm_grads(gpu, rows, cols):
    """(dx, dgamma, dbeta) in one op: dx equals layer_norm_backward's bit for
    bit; the parameter gradients (column sums over 1-16 row chunks) match
    the oracle."""
    x, dy = f32(rows, cols, scale=2.0), f32(rows, cols)
    g = f32(cols, shift=1.0)
    tdy, tx, tg = _dev(gpu, dy), _dev(gpu, x), _dev(gpu, g)
    dx, dg, db = gpu.layer_norm_grads(tdy, tx, tg, 1e-5)
    rdx, rdg, rdb = O.layer_norm_backward(dy, x, g, 1e-5, params=True)
    np.testing.assert_array_equal(_host(dx), _host(gpu.layer_norm_backward(tdy, tx, tg, 1e-5)))
    assert rel_err(_host(dx), rdx) < 1e-5
    assert rel_err(_host(dg), rdg) < 1e-5
    assert rel_err(_host(db), rdb) < 1e-5


def test_layer_norm_backward_known_answers(gpu):
    """ops.rs:4699-4730: uniform dy and gamma = 1 give rows summing to 0;
    ops.rs:4733-4781's 1x3 case against the oracle."""
    x = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    got = _host(gpu.layer_norm_backward(_dev(gpu, np.ones_like(x)), _dev(gpu, x), _dev(gpu, np.ones(4, np.float32))))
    np.testing.assert_allclose(got.sum(-1), 0.0, atol=1e-4)
    x1, g1, d1 = (np.array([[1, 3, 5]], np.float32), np.array([2, 1, 0.5], np.float32),
                  np.ones((1, 3), np.float32))
    got = _host(gpu.layer_norm_backward(_dev(gpu, d1), _dev(gpu, x1), _dev(gpu, g1)))
    np.testing.assert_allclose(got, O.layer_norm_backward(d1, x1, g1), atol=1e-6)


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_layer_norm_grads_16bit(gpu, dt):
    x, dy, g = f32(64, 1280), f32(64, 1280), f32(1280, shift=1.0)
    dx, dg, db = gpu.layer_norm_grads(_dev(gpu, dy, dt), _dev(gpu, x, dt), _dev(gpu, g, dt))
    ref = O.layer_norm_backward(_rnd(gpu, dy, dt), _rnd(gpu, x, dt), _rnd(gpu, g, dt), params=True)
    for a, b in zip((dx, dg, db), ref):
        assert rel_err(_host(a), b) < 1e-2


def test_layer_norm_backward_rejects_bad_shapes(gpu):
    a, b = _dev(gpu, f32(2, 4)), _dev(gpu, f32(3, 4))
    with pytest.raises(ValueError):
        gpu.layer_norm_backward(a, b, _dev(gpu, f32(4))).eval()
    with pytest.raises(ValueError):
        gpu.layer_norm_backward(a, a, _dev(gpu, f32(3))).eval()


# ── softmax and gelu ────────────────────────────────────────────────────────
@pytest.mark.parametrize("shape", [(2, 3), (12, 128, 128), (5, 2500)])
def test_softmax_backward(gpu, shape):
    y = O.softmax(f32(*shape))
    dy = f32(*shape)
    got = _host(gpu.softmax_backward(_dev(gpu, dy), _dev(gpu, y)))
    assert rel_err(got, O.softmax_backward(dy, y)) < 1e-5
    np.testing.assert_allclose(got.sum(-1), 0.0, atol=1e-5)


@pytest.mark.parametrize("n", [5, 4096, 128 * 3072 + 3])
def test_gelu_backward(gpu, n):
    x, dy = f32(n, scale=3.0), f32(n)
    tx, tdy = _dev(gpu, x), _dev(gpu, dy)
    tanh_ref, erf_ref = O.gelu_tanh_backward(dy, x), O.gelu_erf_backward(dy, x)
    assert rel_err(_host(gpu.gelu_backward(tdy, tx)), tanh_ref) < 1e-5
    assert rel_err(_host(gpu.gelu_tanh_backward(tdy, tx)), tanh_ref) < 1e-5
    assert rel_err(_host(gpu.gelu_exact_backward(tdy, tx)), erf_ref) < 1e-5


def test_gelu_backward_far_tails_and_16bit(gpu):
    """|x| up to 30: the clamped tanh term saturates (gradient 0 or 1).  In
    fp32 tanh(+-10) rounds to +-1, so the clamped formula's x (1 - t^2) term
    vanishes there, as in the reference's fp32 kernel; the float64 oracle
    keeps it (up to 1.2e-5 at |x| = 30), hence 2e-5 absolute in the tails."""
    x = np.array([-30, -12, -6, -1e-3, 0, 1e-3, 6, 12, 30], np.float32)
    dy = np.ones_like(x)
    got = _host(gpu.gelu_backward(_dev(gpu, dy), _dev(gpu, x)))
    np.testing.assert_allclose(got, O.gelu_tanh_backward(dy, x), atol=2e-5)
    np.testing.assert_allclose(got[3:6], O.gelu_tanh_backward(dy, x)[3:6], atol=1e-6)
    got = _host(gpu.gelu_exact_backward(_dev(gpu, dy), _dev(gpu, x)))
    np.testing.assert_allclose(got, O.gelu_erf_backward(dy, x), atol=1e-6)
    for dt in ("float16", "bfloat16"):
        x2, d2 = f32(3000, scale=3.0), f32(3000)
        got = _host(gpu.gelu_exact_backward(_dev(gpu, d2, dt), _dev(gpu, x2, dt)))
        assert rel_err(got, O.gelu_erf_backward(_rnd(gpu, d2, dt), _rnd(gpu, x2, dt))) < 1e-2


# ── embedding ───────────────────────────────────────────────────────────────
def test_embedding_backward_known_answers(gpu):
    """ops.rs:4973-5021."""
    dy = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    got = _host(gpu.embedding_backward(_dev(gpu, dy), gpu.from_numpy(np.array([0, 1, 0], np.int32)), 3))
    np.testing.assert_array_equal(got, [[6, 8], [3, 4], [0, 0]])
    dy = np.array([[10, 20], [30, 40], [50, 60]], np.float32)
    got = _host(gpu.embedding_backward(_dev(gpu, dy), gpu.from_numpy(np.array([0, 1, 2], np.int32)), 3))
    np.testing.assert_array_equal(got, dy)


@pytest.mark.parametrize("n,vocab,dim,idx_dt", [
    (128, 50257, 768, np.int32),     # GPT-2 small, one sequence
    (3000, 500, 768, np.int32),      # many repeats
    (2500, 10, 1300, np.int64),      # > 1024 tokens per row (several rounds), two column passes
    (700, 1000, 5, np.int32),        # narrow rows
])
def test_embedding_backward_bit_exact(gpu, n, vocab, dim, idx_dt):
    idx = RNG.integers(0, vocab, n).astype(idx_dt)
    if n >= 2000:
        idx[::3] = 3                 # one index named by > 1024 tokens
    dy = f32(n, dim)
    got = _host(gpu.embedding_backward(_dev(gpu, dy), gpu.from_numpy(idx), vocab))
    np.testing.assert_array_equal(got, O.embedding_backward(dy, idx, vocab))


def test_embedding_backward_edges(gpu):
    """Out-of-range indices add nothing; no tokens gives zeros; 3-D grads;
    16-bit grads are summed in fp32 and rounded once."""
    idx = np.array([2, -1, 9, 2, 40], np.int32)
    dy = f32(5, 16)
    got = _host(gpu.embedding_backward(_dev(gpu, dy), gpu.from_numpy(idx), 10))
    np.testing.assert_array_equal(got, O.embedding_backward(dy, idx, 10))
    assert (got[[0, 1, 3, 4, 5, 6, 7, 8]] == 0).all()
    dy3 = f32(2, 6, 8)
    idx3 = RNG.integers(0, 4, (2, 6)).astype(np.int32)
    got = _host(gpu.embedding_backward(_dev(gpu, dy3), gpu.from_numpy(idx3), 4))
    np.testing.assert_array_equal(got, O.embedding_backward(dy3, idx3, 4))
    for dt in ("float16", "bfloat16"):
        d2 = f32(900, 64)
        i2 = RNG.integers(0, 50, 900).astype(np.int32)
        got = _host(gpu.embedding_backward(_dev(gpu, d2, dt), gpu.from_numpy(i2), 50))
        ref = O.embedding_backward(_rnd(gpu, d2, dt), i2, 50)
        np.testing.assert_array_equal(got, _rnd(gpu, ref, dt))
    got = _host(gpu.embedding_backward(_dev(gpu, np.zeros((0, 4), np.float32)),
                                       gpu.from_numpy(np.zeros(0, np.int32)), 3))
    np.testing.assert_array_equal(got, np.zeros((3, 4), np.float32))
    with pytest.raises(ValueError):
        gpu.embedding_backward(_dev(gpu, f32(3, 2)), gpu.from_numpy(np.zeros(3, np.float32)), 3).eval()


# ── under torch autograd ────────────────────────────────────────────────────
def test_gpt2_style_block_trains_without_fallback(gpu):
    """Embedding -> layer_norm -> Linear -> gelu(tanh) -> Linear -> softmax
    cross terms, backward through the shim's kernels; gradients match torch
    CPU and no op of the step falls back to the CPU."""
    import torch
    import torch.nn.functional as F
    from applegpu_runtime.cpp_backend import fallback_count, load_cpp_backend
    load_cpp_backend()
    torch.manual_seed(3)

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.wte = torch.nn.Embedding(100, 64)
            self.ln = torch.nn.LayerNorm(64)
            self.fc = torch.nn.Linear(64, 256)
            self.proj = torch.nn.Linear(256, 64)

        def forward(self, ids):
            h = self.wte(ids)
            a = self.proj(F.gelu(self.fc(self.ln(h)), approximate="tanh"))
            p = torch.softmax(a, -1)
            return (p * a).sum() + F.gelu(h, approximate="none").sum()

    cpu = Block()
    dev = Block()
    dev.load_state_dict(cpu.state_dict())
    dev = dev.to("applegpu")
    ids = torch.randint(0, 100, (4, 16))
    cpu(ids).backward()
    before = fallback_count()
    out = dev(ids.to(torch.int32).to("applegpu"))
    out.backward()
    for (name, p), q in zip(dev.named_parameters(), cpu.parameters()):
        assert p.grad is not None, name
        err = (p.grad.cpu() - q.grad).abs().max().item() / max(q.grad.abs().max().item(), 1e-12)
        assert err < 1e-4, (name, err)
    assert fallback_count() == before
