"""Elementwise-chain fusion in the lazy executor.

The reference replaces every chain of two or more single-consumer
elementwise nodes by one generated kernel on each eval
(crates/core/src/fusion.rs:60-141 finds the chains, :145-240 generates the
kernel, :243-282 rewrites the graph; lazy.rs:237 runs it).  Here a chain runs
as one `fused_chain` launch that interprets the chain's op list per element.
Results must equal the op-by-op launches bit for bit (every step computes in
fp32 and rounds to the chain's dtype as the unfused node stores it), and the
chain must cost one kernel launch.
"""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4242)


def _stats(gpu):
    return gpu.graph_stats()


def _launches_for(gpu, t):
    """Kernel launcher calls made while `t` (whose inputs are materialised)
    evaluates."""
    before = _stats(gpu)
    t.eval()
    after = _stats(gpu)
    return {k: after[k] - before[k] for k in after}


def _host(t):
    return np.asarray(t.to_numpy(), np.float32)


def test_reference_known_answers(gpu):
    """crates/core/tests/fusion_integration.rs fused_add_relu,
    fused_chain_of_three and fused_add_gelu, each as one launch."""
    a = gpu.from_numpy(np.array([1.0, -2.0, 3.0, -4.0], np.float32))
    b = gpu.from_numpy(np.array([10.0, 20.0, 30.0, 40.0], np.float32))
    r = gpu.relu(a + b)
    d = _launches_for(gpu, r)
    assert d["fused_chains"] == 1 and d["chain_nodes"] == 2 and d["launcher_calls"] == 1
    np.testing.assert_array_equal(r.to_numpy(), [11.0, 18.0, 33.0, 36.0])

    a = gpu.from_numpy(np.array([1.0, 4.0, 9.0, 16.0], np.float32))
    r = gpu.relu(gpu.neg(gpu.sqrt(a)))
    d = _launches_for(gpu, r)
    assert d["fused_chains"] == 1 and d["chain_nodes"] == 3 and d["launcher_calls"] == 1
    np.testing.assert_array_equal(r.to_numpy(), [0.0, 0.0, 0.0, 0.0])

    a = gpu.from_numpy(np.array([0.0, 1.0, -1.0, 2.0], np.float32))
    z = gpu.from_numpy(np.zeros(4, np.float32))
    r = gpu.gelu(a + z)
    d = _launches_for(gpu, r)
    assert d["fused_chains"] == 1 and d["launcher_calls"] == 1
    np.testing.assert_allclose(r.to_numpy(), [0.0, 0.8412, -0.1588, 1.9545], atol=2e-4)


def _build_chain(a, b, c, ev=lambda t: t):
    """relu((a + b) * c) - c, then exp(-x), then * 0.5 (scalar_mul), clamp."""
    import applegpu_runtime as g
    x = ev(a + b)
    x = ev(x * c)
    x = ev(g.relu(x))
    x = ev(x - c)
    x = ev(g.neg(x))
    x = ev(g.exp(x))
    x = ev(g.scalar_mul(x, 0.5))
    return ev(g.clamp(x, 0.0, 3.0))


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_chain_one_launch_bitwise_equal_to_op_by_op(gpu, dtype):
    shape = (37, 129)
    an, bn, cn = (RNG.standard_normal(shape).astype(np.float32) for _ in range(3))
    a, b, c = (gpu.cast(gpu.from_numpy(v), dtype) for v in (an, bn, cn))
    for t in (a, b, c):
        t.eval()
    fused = _build_chain(a, b, c)
    d = _launches_for(gpu, fused)
    assert d["fused_chains"] == 1 and d["chain_nodes"] == 8, d
    assert d["launcher_calls"] == 1, d
    unfused = _build_chain(a, b, c, ev=lambda t: (t.eval(), t)[1])
    np.testing.assert_array_equal(_host(fused), _host(unfused))
    # and the oracle (fp32 at the elementwise bar; 16-bit at theirs)
    ar, br, cr = (_host(t) for t in (a, b, c))
    ref = np.clip(0.5 * np.exp(-(O.relu((ar + br) * cr) - cr)), 0.0, 3.0)
    tol = 1e-5 if dtype == "float32" else (1e-2 if dtype == "float16" else 2e-2)
    assert rel_err(_host(fused), ref) < tol


def test_chain_accumulator_on_the_right(gpu):
    """Binary steps whose chain operand is the right one: c - x, c / x."""
    an = RNG.uniform(0.5, 2.0, (300,)).astype(np.float32)
    cn = RNG.standard_normal(300).astype(np.float32)
    a, c = gpu.from_numpy(an), gpu.from_numpy(cn)
    r = gpu.div(c, gpu.sub(c, gpu.exp(a)))
    d = _launches_for(gpu, r)
    assert d["fused_chains"] == 1 and d["chain_nodes"] == 3 and d["launcher_calls"] == 1
    x = gpu.exp(a)
    x.eval()
    y = gpu.sub(c, x)
    y.eval()
    np.testing.assert_array_equal(r.to_numpy(), gpu.div(c, y).to_numpy())


@pytest.mark.parametrize("case", ["row_bias", "scalar", "column", "transposed_view", "offset_view", "3d_batch"])
def test_chain_broadcast_and_strided_leaves(gpu, case):
    """Leaves broadcast onto the chain's output (suffix vectors, scalars,
    columns) or read through view strides and offsets: one launch, equal to
    op by op."""
    M, N = 48, 64
    xn = RNG.standard_normal((M, N)).astype(np.float32)
    x = gpu.from_numpy(xn)
    if case == "row_bias":
        other = gpu.from_numpy(RNG.standard_normal(N).astype(np.float32))
    elif case == "scalar":
        other = gpu.from_numpy(np.array([0.75], np.float32))
    elif case == "column":
        other = gpu.from_numpy(RNG.standard_normal((M, 1)).astype(np.float32))
    elif case == "transposed_view":
        other = gpu.transpose(gpu.from_numpy(RNG.standard_normal((N, M)).astype(np.float32)))
    elif case == "offset_view":
        other = gpu.slice(gpu.from_numpy(RNG.standard_normal((M, N + 7)).astype(np.float32)), 1, 5, 5 + N)
    else:
        x = gpu.from_numpy(RNG.standard_normal((3, M, N)).astype(np.float32))
        other = gpu.from_numpy(RNG.standard_normal((M, N)).astype(np.float32))
    other.eval()
    x.eval()
    r = gpu.tanh(gpu.mul(gpu.add(x, other), other))
    d = _launches_for(gpu, r)
    assert d["fused_chains"] == 1 and d["launcher_calls"] == 1, d
    s = gpu.add(x, other)
    s.eval()
    m = gpu.mul(s, other)
    m.eval()
    np.testing.assert_array_equal(r.to_numpy(), gpu.tanh(m).to_numpy())


def test_shared_intermediate_ends_the_chain(gpu):
    """A node with a second consumer is materialised: the chains around it
    are fused separately and both results are right."""
    an = RNG.standard_normal(1000).astype(np.float32)
    a = gpu.from_numpy(an)
    a.eval()
    s = gpu.exp(gpu.neg(a))          # chain 1 ends at s (two users)
    u = gpu.relu(gpu.scalar_mul(s, 2.0))
    v = gpu.sqrt(gpu.add(s, s))
    before = _stats(gpu)
    u.eval()
    v.eval()
    after = _stats(gpu)
    assert after["fused_chains"] - before["fused_chains"] >= 2
    ref_s = np.exp(-an.astype(np.float32))
    np.testing.assert_allclose(u.to_numpy(), np.maximum(2 * ref_s, 0), rtol=1e-6)
    np.testing.assert_allclose(v.to_numpy(), np.sqrt(ref_s + ref_s), rtol=1e-6)


def test_kept_intermediate_is_materialised(gpu):
    """An intermediate the caller still holds is not absorbed."""
    a = gpu.from_numpy(RNG.standard_normal(256).astype(np.float32))
    b = gpu.from_numpy(RNG.standard_normal(256).astype(np.float32))
    s = a + b
    r = gpu.relu(gpu.neg(s))
    r.eval()
    np.testing.assert_array_equal(s.to_numpy(), a.to_numpy() + b.to_numpy())
    np.testing.assert_array_equal(r.to_numpy(), np.maximum(-(a.to_numpy() + b.to_numpy()), 0))


def test_long_chains_and_many_leaves_split(gpu):
    """Chains beyond the program limits (16 steps, 8 leaves) split into
    several launches with the same result."""
    an = RNG.uniform(-1, 1, 512).astype(np.float32)
    a = gpu.from_numpy(an)
    leaves_np = [RNG.uniform(-1, 1, 512).astype(np.float32) for _ in range(12)]
    leaves = [gpu.from_numpy(v) for v in leaves_np]
    x = a
    ref = an.copy()
    for i in range(40):
        if i % 3 == 0:
            x = x + leaves[i % 12]
            ref = (ref + leaves_np[i % 12]).astype(np.float32)
        elif i % 3 == 1:
            x = gpu.scalar_mul(x, 0.9)
            ref = (ref * np.float32(0.9)).astype(np.float32)
        else:
            x = gpu.tanh(x)
            ref = np.tanh(ref).astype(np.float32)
    before = _stats(gpu)
    got = x.to_numpy()
    after = _stats(gpu)
    assert after["fused_chains"] - before["fused_chains"] >= 3
    assert after["launcher_calls"] - before["launcher_calls"] <= 5
    assert rel_err(got, ref) < 1e-5


def test_relu_add_loop_runs_as_one_launch(gpu):
    """relu(y + x) twenty times (40 nodes) over one leaf pair: three chains
    at most, not 40 launches."""
    xn = np.ones((64, 64), np.float32)
    x = gpu.from_numpy(xn)
    x.eval()
    y = x
    for _ in range(20):
        y = gpu.relu(y + x)
    before = _stats(gpu)
    got = y.to_numpy()
    after = _stats(gpu)
    assert after["launcher_calls"] - before["launcher_calls"] <= 4
    np.testing.assert_array_equal(got, np.full((64, 64), 21.0, np.float32))


def test_gemm_epilogue_keeps_priority(gpu):
    """matmul + bias -> gelu stays a fused GEMM epilogue; the elementwise
    tail after it forms a chain of its own."""
    xn = RNG.standard_normal((32, 48)).astype(np.float32)
    wn = RNG.standard_normal((48, 40)).astype(np.float32)
    bn = RNG.standard_normal(40).astype(np.float32)
    x, w, b = gpu.from_numpy(xn), gpu.from_numpy(wn), gpu.from_numpy(bn)
    y = gpu.exp(gpu.neg(gpu.gelu(gpu.add_bias(x @ w, b))))
    before = _stats(gpu)
    got = y.to_numpy()
    after = _stats(gpu)
    assert after["fused_gemm_epilogues"] - before["fused_gemm_epilogues"] == 1
    assert after["fused_chains"] - before["fused_chains"] == 1
    ref = np.exp(-O.gelu_tanh(O.add_bias(O.matmul(xn, wn), bn)))
    assert rel_err(got, ref) < 1e-3


def test_empty_chain_output(gpu):
    a = gpu.from_numpy(np.zeros((0, 5), np.float32))
    r = gpu.relu(gpu.neg(a))
    assert r.to_numpy().shape == (0, 5)
