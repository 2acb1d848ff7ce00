"""layer_norm of a GEMM's output computed by the GEMM's split-K reduction
(the GPT-2 residual stream: x = x + proj(..) or fc2(..), then ln_2 / ln_1,
models/gpt2.py:84-178): values against the float64 oracle, bitwise against
the same graph with the layer_norm run as its own kernel, the residual
output itself, fp16/bf16, ragged widths, and the shapes that do not fuse."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(5151)


def f32(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def _block(gpu, a, w, b, res, g, beta, dt="float32", split_ln=False):
    """x = a @ w + b + res; y = layer_norm(x).  split_ln: evaluate x first so
    the layer_norm runs as its own kernel."""
    cast = (lambda t: t) if dt == "float32" else (lambda t: gpu.cast(t, dt))
    ta, tw, tb, tr, tg, tbeta = (cast(gpu.from_numpy(v)) for v in (a, w, b, res, g, beta))
    x = gpu.add_bias(ta @ tw, tb) + tr
    if split_ln:
        x.eval()
    y = gpu.layer_norm(x, tg, tbeta, 1e-5)
    return x, y


def _ref(a, w, b, res, g, beta):
    x = a.astype(np.float64) @ w.astype(np.float64) + b + res
    return x, O.layer_norm(x, g.astype(np.float64), beta.astype(np.float64), 1e-5)


@pytest.mark.parametrize("m,k,n", [(128, 768, 768), (128, 3072, 768), (64, 2048, 100), (32, 512, 2048)])
def test_post_ln_matches_oracle_and_unfused(gpu, m, k, n):
    a, w, b, res = f32(m, k), f32(k, n, scale=0.05), f32(n), f32(m, n)
    g, beta = f32(n, scale=0.5) + 1, f32(n, scale=0.1)
    before = gpu.graph_stats()["launches_saved"]
    x, y = _block(gpu, a, w, b, res, g, beta)
    yn = y.to_numpy()
    saved = gpu.graph_stats()["launches_saved"] - before
    xn = x.to_numpy()
    xr, yr = _ref(a, w, b, res, g, beta)
    assert rel_err(xn, xr) < 1e-4
    assert rel_err(yn, yr) < 1e-4
    # layer_norm of the stored x, as the separate kernel computes it (bitwise)
    x2, y2 = _block(gpu, a, w, b, res, g, beta, split_ln=True)
    np.testing.assert_array_equal(x2.to_numpy(), xn)
    np.testing.assert_array_equal(y2.to_numpy(), yn)
    assert saved >= 3  # bias + residual + the layer_norm launch


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_post_ln_16bit(gpu, dt):
    m, k, n = 64, 2048, 1280
    a, w, b, res = f32(m, k), f32(k, n, scale=0.05), f32(n), f32(m, n)
    g, beta = f32(n, scale=0.5) + 1, f32(n, scale=0.1)
    x, y = _block(gpu, a, w, b, res, g, beta, dt)
    x2, y2 = _block(gpu, a, w, b, res, g, beta, dt, split_ln=True)
    np.testing.assert_array_equal(x.to_numpy(), x2.to_numpy())
    np.testing.assert_array_equal(y.to_numpy(), y2.to_numpy())
    rnd = lambda v: gpu.cast(gpu.from_numpy(v), dt).to_numpy().astype(np.float32)
    _, yr = _ref(rnd(a), rnd(w), rnd(b), rnd(res), rnd(g), rnd(beta))
    assert rel_err(y.to_numpy().astype(np.float32), yr) < 2e-2


@pytest.mark.parametrize("m,k,n", [(4096, 256, 512), (128, 768, 2050), (128, 768, 766)])
def test_post_ln_unfusable_shapes_still_correct(gpu, m, k, n):
    """No K split (a full grid of tiles), N > 2048, or N % 4 != 0: the
    layer_norm runs as its own kernel."""
    a, w, b, res = f32(m, k), f32(k, n, scale=0.05), f32(n), f32(m, n)
    g, beta = f32(n, scale=0.5) + 1, f32(n, scale=0.1)
    x, y = _block(gpu, a, w, b, res, g, beta)
    xr, yr = _ref(a, w, b, res, g, beta)
    assert rel_err(x.to_numpy(), xr) < 1e-4
    assert rel_err(y.to_numpy(), yr) < 1e-4
