"""Per-op parity of the gfx950 kernels against the oracle and the golden
vectors, through the lazy graph API (applegpu_graph_op).  Tolerances are the
north star's: bit-exact for integer/index work, 1e-5 relative for fp32
elementwise and norms, 1e-3 for fp32 matmul/attention, 1e-2 for fp16/bf16."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(1234)


def f32(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def test_known_answers(gpu, known):
    for k in known:
        op = k["op"]
        if op == "matmul":
            got = (gpu.from_numpy(np.array(k["a"], np.float32)) @ gpu.from_numpy(np.array(k["b"], np.float32)))
            np.testing.assert_array_equal(got.to_numpy(), np.array(k["expect"], np.float32), err_msg=k["src"])
        elif op == "relu":
            np.testing.assert_array_equal(gpu.relu(gpu.from_numpy(np.array(k["x"], np.float32))).to_numpy(),
                                          k["expect"])
        elif op == "softmax":
            np.testing.assert_allclose(gpu.softmax(gpu.from_numpy(np.array(k["x"], np.float32))).to_numpy(),
                                       k["expect"], atol=k["atol"])
        elif op == "softmax_causal":
            np.testing.assert_allclose(
                gpu.softmax_causal(gpu.from_numpy(np.array(k["x"], np.float32))).to_numpy(), k["expect"],
                atol=k["atol"])
        elif op == "attention_causal_row0":
            q, kk, v = (gpu.from_numpy(np.array(k[n], np.float32)) for n in "qkv")
            out = gpu.attention_causal(q, kk, v)
            assert out.shape == [2, 2]
            np.testing.assert_allclose(out.to_numpy()[0], k["expect_row0"], atol=k["atol"])
        elif op == "softmax_rows_sum":
            r = gpu.softmax(gpu.from_numpy(np.array(k["x"], np.float32))).to_numpy()
            np.testing.assert_allclose(r.sum(-1), k["expect_row_sums"], atol=k["atol"])
        elif op == "transpose":
            t = gpu.transpose(gpu.from_numpy(np.array(k["x"], np.float32)))
            assert t.shape == [3, 2]
            np.testing.assert_array_equal(t.to_numpy(), k["expect"])
        elif op == "layer_norm":
            got = gpu.layer_norm(*(gpu.from_numpy(np.array(k[n], np.float32)) for n in ("x", "gamma", "beta")))
            np.testing.assert_allclose(got.to_numpy(), k["expect"], rtol=k["rtol"], atol=1e-6)
        elif op == "gelu":
            got = gpu.gelu(gpu.from_numpy(np.array(k["x"], np.float32))).to_numpy()
            np.testing.assert_allclose(got, k["expect"], rtol=k["rtol"], atol=1e-7)
        elif op == "embedding":
            got = gpu.embedding(gpu.from_numpy(np.array(k["w"], np.float32)),
                                gpu.from_numpy(np.array(k["idx"], np.int32))).to_numpy()
            np.testing.assert_array_equal(got, np.array(k["expect"], np.float32))


@pytest.mark.parametrize("name", ["r7", "r768", "r2500"])
def test_rows_vs_golden(gpu, fixtures, name):
    x = fixtures[f"softmax_{name}_x"]
    tx = gpu.from_numpy(x)
    assert rel_err(gpu.softmax(tx).to_numpy(), fixtures[f"softmax_{name}_y"]) < 1e-5
    np.testing.assert_allclose(gpu.log_softmax(tx).to_numpy(), fixtures[f"log_softmax_{name}_y"], rtol=1e-5,
                               atol=1e-5)
    g, b = gpu.from_numpy(fixtures[f"layer_norm_{name}_g"]), gpu.from_numpy(fixtures[f"layer_norm_{name}_b"])
    _check_norm(gpu.layer_norm(tx, g, b).to_numpy(), fixtures[f"layer_norm_{name}_y"])


def _check_norm(got, ref):
    """The 1e-5 relative bar for norms: normwise, and per element with an
    absolute floor of 1e-6 of the output scale for values that cancel to
    near zero (gamma * x_hat + beta)."""
    assert rel_err(got, ref) < 1e-5
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6 * max(1.0, float(np.abs(ref).max())))


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (17, 255), (4, 256), (5, 1024), (2, 2047), (2, 2049),
                                   (3, 50257), (2, 3, 64)])
def test_softmax_family_shapes(gpu, shape):
    x = f32(*shape, scale=4.0)
    t = gpu.from_numpy(x)
    np.testing.assert_allclose(gpu.softmax(t).to_numpy(), O.softmax(x), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(gpu.log_softmax(t).to_numpy(), O.log_softmax(x), rtol=1e-5, atol=1e-5)
    if len(shape) >= 2:
        np.testing.assert_allclose(gpu.softmax_causal(t).to_numpy(), O.softmax_causal(x), rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("shape", [(1, 3), (7, 13), (128, 768), (33, 1280), (3, 3000)])
def test_layer_norm_shapes(gpu, shape):
    x = f32(*shape, scale=2.0) + 1.5
    g, b = f32(shape[-1]), f32(shape[-1])
    got = gpu.layer_norm(gpu.from_numpy(x), gpu.from_numpy(g), gpu.from_numpy(b)).to_numpy()
    _check_norm(got, O.layer_norm(x, g, b))


@pytest.mark.parametrize("dt,tol", [("float16", 1e-2), ("bfloat16", 2e-2)])
def test_rows_half_precision(gpu, dt, tol):
    x = f32(9, 300, scale=2.0)
    g, b = f32(300), f32(300)
    t = gpu.cast(gpu.from_numpy(x), dt)
    sm = gpu.softmax(t).to_numpy().astype(np.float32)
    assert rel_err(sm, O.softmax(x)) < tol
    ln = gpu.layer_norm(t, gpu.cast(gpu.from_numpy(g), dt), gpu.cast(gpu.from_numpy(b), dt)).to_numpy()
    assert rel_err(ln.astype(np.float32), O.layer_norm(x, g, b)) < 4 * tol


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
@pytest.mark.parametrize("cols", [256, 300, 768, 772, 1024, 1280, 1800, 2048])
def test_rows_16bit_each_column_once(gpu, dt, cols):
    """The register-resident 16-bit row kernels (a lane reads 8 consecutive
    values per 16-byte load; an odd group count ends in a 4-value group;
    772 columns are not 16-byte aligned rows and take the guarded path):
    softmax, log_softmax, causal softmax, layer_norm and its backward against
    the oracle in float64 on the input as stored, within one rounding of the
    output dtype (rtol 2^-10 fp16, 2^-7 bf16), so a column read, reduced or
    written in the wrong place fails."""
    rtol = 2.0 ** -10 if dt == "float16" else 2.0 ** -7
    rows = 9
    cast = lambda a: gpu.cast(gpu.from_numpy(a), dt)
    back = lambda t: t.to_numpy().astype(np.float64)
    x, g, b, dy = cast(f32(rows, cols, scale=2.0)), cast(f32(cols)), cast(f32(cols)), cast(f32(rows, cols))
    xs, gs, bs, dys = back(x), back(g), back(b), back(dy)

    def close(got, ref, what):
        np.testing.assert_allclose(back(got), ref, rtol=rtol, atol=1e-5 * np.abs(ref).max(), err_msg=what)

    close(gpu.softmax(x), O.softmax(xs), "softmax")
    close(gpu.log_softmax(x), O.log_softmax(xs), "log_softmax")
    close(gpu.softmax_causal(x), O.softmax_causal(xs), "softmax_causal")
    close(gpu.layer_norm(x, g, b), O.layer_norm(xs, gs, bs), "layer_norm")
    close(gpu.layer_norm_backward(dy, x, g), O.layer_norm_backward(dys, xs, gs), "layer_norm_backward")


def test_gelu_vs_golden(gpu, fixtures):
    t = gpu.from_numpy(fixtures["gelu_x"])
    np.testing.assert_allclose(gpu.gelu(t).to_numpy(), fixtures["gelu_tanh_y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gpu.gelu_exact(t).to_numpy(), fixtures["gelu_erf_y"], rtol=1e-5, atol=1e-6)


def test_binary_broadcast_and_views(gpu):
    a = f32(4, 5, 6)
    b = f32(5, 1)
    ta, tb = gpu.from_numpy(a), gpu.from_numpy(b)
    for name, fn in [("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", np.divide)]:
        got = getattr(gpu, name)(ta, tb).to_numpy()
        np.testing.assert_allclose(got, fn(a, b).astype(np.float32), rtol=1e-6)
    # strided operand (a transposed view) goes through the N-D kernel
    v = gpu.transpose_dims(ta, 0, 2)
    np.testing.assert_array_equal((v + v).to_numpy(), (a.transpose(2, 1, 0) * 2))
    # sliced operand (byte offset)
    s = gpu.slice(ta, 2, 1, 4)
    np.testing.assert_array_equal(gpu.relu(s).to_numpy(), np.maximum(a[:, :, 1:4], 0))


def test_unary_ops(gpu):
    x = f32(3, 7, scale=2.0)
    t = gpu.from_numpy(x)
    checks = {"neg": -x, "relu": np.maximum(x, 0), "exp": np.exp(x), "tanh": np.tanh(x), "sin": np.sin(x),
              "cos": np.cos(x), "abs": np.abs(x), "sign": np.sign(x), "sigmoid": 1 / (1 + np.exp(-x))}
    for name, ref in checks.items():
        np.testing.assert_allclose(getattr(gpu, name)(t).to_numpy(), ref.astype(np.float32), rtol=2e-6, atol=2e-7,
                                   err_msg=name)
    p = np.abs(x) + 0.5
    tp = gpu.from_numpy(p)
    np.testing.assert_allclose(gpu.log(tp).to_numpy(), np.log(p), rtol=2e-6)
    np.testing.assert_allclose(gpu.sqrt(tp).to_numpy(), np.sqrt(p), rtol=2e-6)
    np.testing.assert_allclose(gpu.scalar_mul(t, 0.125).to_numpy(), x * np.float32(0.125), rtol=0)
    np.testing.assert_allclose(gpu.clamp(t, -0.5, 0.5).to_numpy(), np.clip(x, -0.5, 0.5))
    np.testing.assert_allclose(gpu.pow(tp, 2.0).to_numpy(), p ** 2, rtol=2e-6)


def test_integer_and_bitwise_ops_bit_exact(gpu):
    a = RNG.integers(-1000, 1000, (6, 9)).astype(np.int32)
    b = RNG.integers(1, 50, (6, 9)).astype(np.int32)
    ta, tb = gpu.from_numpy(a), gpu.from_numpy(b)
    np.testing.assert_array_equal(gpu.add(ta, tb).to_numpy(), a + b)
    np.testing.assert_array_equal(gpu.mul(ta, tb).to_numpy(), a * b)
    np.testing.assert_array_equal(gpu.bitwise_and(ta, tb).to_numpy(), a & b)
    np.testing.assert_array_equal(gpu.bitwise_or(ta, tb).to_numpy(), a | b)
    np.testing.assert_array_equal(gpu.bitwise_xor(ta, tb).to_numpy(), a ^ b)
    np.testing.assert_array_equal(gpu.bitwise_not(ta).to_numpy(), ~a)
    np.testing.assert_array_equal(gpu.shl(tb, 3).to_numpy(), b << 3)
    np.testing.assert_array_equal(gpu.shr(ta, 2).to_numpy(), a >> 2)
    np.testing.assert_array_equal(gpu.mod_(ta, tb).to_numpy(), np.fmod(a, b))
    np.testing.assert_array_equal(gpu.elem_min(ta, tb).to_numpy(), np.minimum(a, b))
    for name, fn in [("lt", np.less), ("gt", np.greater), ("le", np.less_equal), ("ge", np.greater_equal),
                     ("eq_", np.equal), ("ne_", np.not_equal)]:
        r = getattr(gpu, name)(ta, tb)
        assert r.dtype == "bool"
        np.testing.assert_array_equal(r.to_numpy(), fn(a, b))
    u = RNG.integers(0, 256, 37).astype(np.uint8)
    np.testing.assert_array_equal(gpu.bitwise_not(gpu.from_numpy(u)).to_numpy(), ~u)
    bo = RNG.integers(0, 2, 11).astype(bool)
    np.testing.assert_array_equal(gpu.bitwise_not(gpu.from_numpy(bo)).to_numpy(), ~bo)
    np.testing.assert_array_equal(gpu.logical_not(gpu.from_numpy(bo)).to_numpy(), ~bo)


def test_argmax_bit_exact(gpu, fixtures):
    np.testing.assert_array_equal(gpu.argmax(gpu.from_numpy(fixtures["argmax_x"])).to_numpy(),
                                  fixtures["argmax_y"])
    x = np.array([[1, 3, 3, 2], [np.nan, 5, 1, np.nan], [0, 0, 0, 0], [2, np.nan, 9, 9]], np.float32)
    np.testing.assert_array_equal(gpu.argmax(gpu.from_numpy(x)).to_numpy(), O.argmax(x))
    big = f32(8, 50257)
    big[3, 777] = 99.0
    big[3, 40000] = 99.0
    got = gpu.argmax(gpu.from_numpy(big)).to_numpy()
    np.testing.assert_array_equal(got, O.argmax(big))
    assert got[3] == 777
    one = gpu.argmax(gpu.from_numpy(np.array([4.0, 7.0, 7.0], np.float32)))
    assert one.shape == [1] and one.to_list() == [1]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "int32", "int8", "uint8"])
def test_argmax_long_rows_unaligned(gpu, dtype):
    """Long rows take the block-per-row kernel; rows of odd length start
    unaligned, so ties and NaNs sit in the scalar head, the 16-byte body and
    the scalar tail of different rows."""
    rows, cols = 7, 50257
    if dtype in ("int8", "uint8"):
        lo, hi = (-100, 100) if dtype == "int8" else (0, 200)
        x = RNG.integers(lo, hi, (rows, cols)).astype(dtype)
        top = np.array(120 if dtype == "int8" else 250, dtype)
    elif dtype == "int32":
        x = RNG.integers(-10**6, 10**6, (rows, cols)).astype(np.int32)
        top = np.int32(2 * 10**6)
    else:
        x = f32(rows, cols)
        top = np.float32(50.0)
    # ties: first occurrence must win, wherever the copies fall
    for r, (a, b) in enumerate([(0, 5), (3, cols - 1), (cols - 2, cols - 1), (1000, 1001), (7, 40000)]):
        x[r, a] = top
        x[r, b] = top
    if dtype in ("float32", "float16", "bfloat16"):
        x[5, 9] = np.nan         # NaN beats a larger value later on
        x[5, 30000] = 99.0
        x[6, cols - 1] = np.nan  # NaN in the tail
        x[6, 2] = np.nan         # ... but the first NaN wins
    t = gpu.from_numpy(x) if dtype not in ("float16", "bfloat16") else gpu.cast(gpu.from_numpy(x), dtype)
    ref_in = x if dtype != "bfloat16" else gpu.cast(t, "float32").to_numpy()
    if dtype == "float16":
        ref_in = x.astype(np.float16)
    got = gpu.argmax(t).to_numpy()
    np.testing.assert_array_equal(got, O.argmax(ref_in))
    # a row starting at an unaligned offset inside a wider tensor
    sub = gpu.slice(t, 1, 3, cols)
    np.testing.assert_array_equal(gpu.argmax(sub).to_numpy(), O.argmax(np.asarray(ref_in)[:, 3:]))


def test_embedding_gather_index_select_bit_exact(gpu, fixtures):
    got = gpu.embedding(gpu.from_numpy(fixtures["emb_w"]), gpu.from_numpy(fixtures["emb_idx"])).to_numpy()
    np.testing.assert_array_equal(got, fixtures["emb_y"])
    x = np.arange(60, dtype=np.float32).reshape(3, 4, 5)
    idx = RNG.integers(0, 4, (3, 6, 5)).astype(np.int32)
    np.testing.assert_array_equal(gpu.gather(gpu.from_numpy(x), 1, gpu.from_numpy(idx)).to_numpy(),
                                  O.gather(x, 1, idx))
    sel = np.array([3, 0, 2], np.int32)
    np.testing.assert_array_equal(gpu.index_select(gpu.from_numpy(x), 1, gpu.from_numpy(sel)).to_numpy(),
                                  O.index_select(x, 1, sel))
    # out-of-range ids give zero rows, not a fault
    w = gpu.from_numpy(np.ones((4, 3), np.float32))
    bad = gpu.embedding(w, gpu.from_numpy(np.array([1, 7, -1], np.int32))).to_numpy()
    np.testing.assert_array_equal(bad, [[1, 1, 1], [0, 0, 0], [0, 0, 0]])


def test_reductions(gpu):
    x = f32(3, 4, 37)
    t = gpu.from_numpy(x)
    np.testing.assert_allclose(gpu.sum(t).to_numpy(), x.sum(-1), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gpu.mean(t).to_numpy(), x.mean(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(gpu.amax(t).to_numpy(), x.max(-1))
    np.testing.assert_allclose(gpu.var(t).to_numpy(), x.var(-1, ddof=1), rtol=1e-4)
    np.testing.assert_allclose(gpu.std_dev(t, 0).to_numpy(), x.std(-1), rtol=1e-4)
    for d in (0, 1, 2, -1):
        np.testing.assert_allclose(gpu.sum_dim(t, d).to_numpy(), O.sum_dim(x, d), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gpu.sum_dim(t, 1, True).to_numpy(), O.sum_dim(x, 1, True), rtol=1e-5, atol=1e-5)
    big = f32(1000, 1000)
    np.testing.assert_allclose(gpu.mean_all(gpu.from_numpy(big)).to_numpy(), O.mean_all(big), rtol=1e-4, atol=1e-7)
    ints = RNG.integers(-5, 5, (7, 300)).astype(np.int32)
    np.testing.assert_array_equal(gpu.sum(gpu.from_numpy(ints)).to_numpy(), ints.sum(-1))


@pytest.mark.parametrize("shape", [(1 << 21,), (3, (1 << 20) + 5)])
@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_sum_mean_of_few_long_rows(gpu, shape, dt):
    """At most 16 rows of >= 2^20 values reduce over many blocks (two-stage
    fp32 partials): sum and mean of each row against a float64 sum of the
    values as stored; a plain positive offset keeps the sums well away from
    zero so that a relative bar applies (fp16: small values, so that the
    sums of 2^21 of them stay inside the fp16 range)."""
    x = (RNG.standard_normal(shape) + 2.0).astype(np.float32)
    if dt == "float16":
        x *= np.float32(0.005)
    t = gpu.from_numpy(x)
    if dt != "float32":
        t = gpu.cast(t, dt)
    xs = t.to_numpy().astype(np.float64)
    tol = 1e-5 if dt == "float32" else 2e-3
    np.testing.assert_allclose(gpu.sum(t).to_numpy().astype(np.float64), xs.sum(-1), rtol=tol)
    np.testing.assert_allclose(gpu.mean(t).to_numpy().astype(np.float64), xs.mean(-1), rtol=tol)


def test_mse_vs_golden(gpu, fixtures):
    a, b = gpu.from_numpy(fixtures["mse_a"]), gpu.from_numpy(fixtures["mse_b"])
    np.testing.assert_allclose(gpu.mse_loss(a, b).to_numpy(), fixtures["mse_loss"], rtol=1e-5)
    one = gpu.from_numpy(np.ones(1, np.float32))
    np.testing.assert_allclose(gpu.mse_loss_backward(one, a, b).to_numpy(), fixtures["mse_grad"], rtol=1e-5,
                               atol=1e-8)


def test_add_bias_where_tri_threshold(gpu):
    x = f32(4, 6, 5)
    bias = f32(6)
    np.testing.assert_allclose(gpu.add_bias(gpu.from_numpy(x), gpu.from_numpy(bias)).to_numpy(),
                               O.add_bias(x, bias), rtol=1e-6)
    m = f32(5, 5)
    np.testing.assert_array_equal(gpu.triu(gpu.from_numpy(m), 1).to_numpy(), np.triu(m, 1))
    np.testing.assert_array_equal(gpu.tril(gpu.from_numpy(m)).to_numpy(), np.tril(m))
    mask = gpu.from_numpy(m > 0)
    np.testing.assert_array_equal(gpu.masked_fill(gpu.from_numpy(m), mask, -1e9).to_numpy(),
                                  np.where(m > 0, np.float32(-1e9), m))
    g, inp = f32(3, 8), f32(3, 8)
    np.testing.assert_array_equal(gpu.threshold_backward(gpu.from_numpy(g), gpu.from_numpy(inp), 0.0).to_numpy(),
                                  O.threshold_backward(g, inp))


def test_shape_ops(gpu):
    x = f32(4, 6)
    t = gpu.from_numpy(x)
    np.testing.assert_array_equal(gpu.reshape(t, [2, 12]).to_numpy(), x.reshape(2, 12))
    np.testing.assert_array_equal(gpu.reshape(gpu.transpose(t), [24]).to_numpy(), x.T.reshape(24))
    y = f32(4, 3)
    np.testing.assert_array_equal(gpu.concat(t, gpu.from_numpy(y), 1).to_numpy(), np.concatenate([x, y], 1))
    np.testing.assert_array_equal(gpu.concat(t, t, 0).to_numpy(), np.concatenate([x, x], 0))
    np.testing.assert_array_equal(gpu.slice(t, 1, 2, 5).to_numpy(), x[:, 2:5])
    np.testing.assert_array_equal(gpu.contiguous(gpu.transpose(t)).to_numpy(), x.T)


def test_casts(gpu):
    x = f32(5, 7, scale=3)
    t = gpu.from_numpy(x)
    np.testing.assert_array_equal(gpu.cast(t, "float16").to_numpy(), x.astype(np.float16))
    np.testing.assert_array_equal(gpu.cast(t, "int32").to_numpy(), x.astype(np.int32))
    bf = gpu.cast(t, "bfloat16").to_numpy()
    assert rel_err(bf, x) < 1e-2
    np.testing.assert_array_equal(gpu.cast(gpu.cast(t, "bfloat16"), "float32").to_numpy(), bf)


def test_errors_raise_value_error(gpu):
    a = gpu.from_numpy(f32(2, 3))
    b = gpu.from_numpy(f32(4, 5))
    with pytest.raises(ValueError, match="inner dimensions"):
        gpu.matmul(a, b)
    with pytest.raises(ValueError, match="broadcast"):
        gpu.add(a, b)
    with pytest.raises(ValueError, match="Int32"):
        gpu.embedding(a, a)
    with pytest.raises(ValueError, match="float"):
        gpu.softmax(gpu.from_numpy(np.ones((2, 2), np.int32)))
    with pytest.raises(ValueError, match="gamma"):
        gpu.layer_norm(a, gpu.from_numpy(f32(4)), gpu.from_numpy(f32(3)))
    with pytest.raises(ValueError, match="reshape"):
        gpu.reshape(a, [5])
    with pytest.raises(ValueError):
        gpu.quantize(a, "int8", 0.0)
