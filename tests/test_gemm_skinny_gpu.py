"""GEMMs with at most 16 rows of A (decode steps) against the oracle: the
skinny MFMA kernel (16-bit, weights contiguous along k) and, for the other
layouts and fp32, the MFMA tile path; both paths on the same inputs; fused
epilogues; determinism; graph replay."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4242)


def _lib():
    from applegpu_runtime._native import lib
    return lib


def _plan(M, N, K, dt, b_kcontig):
    codes = {"float32": 0, "float16": 1, "bfloat16": 10}
    buf = ctypes.create_string_buffer(128)
    assert _lib().applegpu_ffi_gemm_plan(M, N, K, 1, codes[dt], True, b_kcontig, buf, 128) == 0
    return buf.value.decode()


def _dev(gpu, a, dt):
    t = gpu.from_numpy(np.ascontiguousarray(a, np.float32))
    return t if dt == "float32" else gpu.cast(t, dt)


def _round(a, dt):
    if dt == "float16":
        return a.astype(np.float16).astype(np.float32)
    if dt == "bfloat16":
        u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        return u.astype(np.uint32).view(np.float32)
    return a.astype(np.float32)


def _np(t):
    return np.asarray(t.to_numpy(), np.float32)


TOL = {"float32": 1e-3, "float16": 1e-2, "bfloat16": 2e-2}


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
@pytest.mark.parametrize("M", [1, 3, 8, 16])
@pytest.mark.parametrize("K,N", [(1280, 3840), (5120, 1280), (1280, 50257), (8, 5), (776, 1001), (96, 17),
                                 (2056, 33), (6144, 48), (6152, 40)])
def test_skinny_mfma_vs_oracle(gpu, dt, M, K, N):
    """x [M, K] @ W^T with W [N, K] (torch Linear layout, tied LM head, the
    k-major GPT-2 weights): ragged N, K not a multiple of 32, K = 8; rows
    staged in LDS (K <= 2048, or the wide staging up to K = 6144 for M <= 8)
    or read from global memory (K = 6152: more steps than a wave keeps in
    flight, so the k loop turns)."""
    assert _plan(M, N, K, dt, True).startswith("skinny")
    x = _round(RNG.standard_normal((M, K)).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K)) * 0.05).astype(np.float32), dt)
    got = _np(_dev(gpu, x, dt) @ gpu.transpose(_dev(gpu, w, dt)))
    assert rel_err(got, O.matmul(x.astype(np.float64), w.T.astype(np.float64))) < TOL[dt]


def test_skinny_mfma_exact_small_integers(gpu):
    """Small integers are exact in fp16 and fp32 accumulation: any error in
    the 16x16x32 operand or output lane layout shows up as a wrong integer."""
    M, K, N = 13, 200, 45
    x = RNG.integers(-3, 4, (M, K)).astype(np.float32)
    w = RNG.integers(-3, 4, (N, K)).astype(np.float32)
    got = _np(gpu.cast(gpu.cast(gpu.from_numpy(x), "float16") @
                       gpu.transpose(gpu.cast(gpu.from_numpy(w), "float16")), "float32"))
    np.testing.assert_array_equal(got, x @ w.T)


@pytest.mark.parametrize("dt", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("K,N,bk", [(1280, 3840, False), (5120, 1280, False), (33, 70, True), (100, 7, False),
                                    (1280, 640, True)])
def test_small_m_other_layouts_vs_oracle(gpu, dt, M, K, N, bk):
    """The layouts the skinny kernel does not take (W n-contiguous, fp32,
    K % 8 != 0) run the MFMA tiles at small M."""
    x = _round(RNG.standard_normal((M, K)).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K) if bk else (K, N)) * 0.05).astype(np.float32), dt)
    wd = _dev(gpu, w, dt)
    got = _np(_dev(gpu, x, dt) @ (gpu.transpose(wd) if bk else wd))
    ref = O.matmul(x.astype(np.float64), (w.T if bk else w).astype(np.float64))
    assert rel_err(got, ref) < TOL[dt]


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_skinny_matches_mfma_tiles(gpu, dt):
    """Same inputs through both kernels (switching the skinny path off)."""
    M, K, N = 8, 1280, 5120
    x = _round(RNG.standard_normal((M, K)).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K)) * 0.05).astype(np.float32), dt)
    xd, wt = _dev(gpu, x, dt), gpu.transpose(_dev(gpu, w, dt))
    a = _np(xd @ wt)
    prev = _lib().applegpu_ffi_gemm_skinny(0)
    try:
        assert not _plan(M, N, K, dt, True).startswith("skinny")
        b = _np(xd @ wt)
    finally:
        _lib().applegpu_ffi_gemm_skinny(prev)
    assert rel_err(a, b) < TOL[dt]


def test_skinny_is_deterministic(gpu):
    """The 16 waves' partial tiles are summed in wave order: repeated launches
    agree bit for bit."""
    M, K, N = 8, 5120, 1280
    x = RNG.standard_normal((M, K)).astype(np.float16)
    w = RNG.standard_normal((N, K)).astype(np.float16)
    xd, wt = gpu.from_numpy(x), gpu.transpose(gpu.from_numpy(w))
    first = _np(xd @ wt)
    for _ in range(5):
        np.testing.assert_array_equal(_np(xd @ wt), first)


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_skinny_fused_epilogues_through_graph(gpu, dt):
    """bias + gelu and bias + residual fuse into the skinny kernel's epilogue
    (the GPT-2 decode block)."""
    M, K, N = 8, 1280, 5120
    x = _round(RNG.standard_normal((M, K)).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K)) * 0.03).astype(np.float32), dt)
    b = _round(RNG.standard_normal(N).astype(np.float32), dt)
    r = _round(RNG.standard_normal((M, N)).astype(np.float32), dt)
    xd, wd, bd, rd = (_dev(gpu, a, dt) for a in (x, w, b, r))
    wt = gpu.transpose(wd)
    before = gpu.graph_stats()["fused_gemm_epilogues"]
    y1 = _np(gpu.gelu(gpu.add_bias(xd @ wt, bd)))
    y2 = _np(rd + gpu.add_bias(xd @ wt, bd))
    assert gpu.graph_stats()["fused_gemm_epilogues"] >= before + 2
    h = O.matmul(x.astype(np.float64), w.T.astype(np.float64)) + b
    assert rel_err(y1, O.gelu_tanh(h)) < TOL[dt]
    assert rel_err(y2, h + r) < TOL[dt]


def test_skinny_strided_activation_rows(gpu):
    """A rows from a view of a wider activation (16-byte aligned offset)."""
    M, K, N = 4, 320, 96
    base = RNG.standard_normal((M, K + 56)).astype(np.float16)
    w = RNG.standard_normal((N, K)).astype(np.float16)
    xd = gpu.slice(gpu.from_numpy(base), 1, 16, 16 + K)
    got = _np(xd @ gpu.transpose(gpu.from_numpy(w)))
    ref = O.matmul(base[:, 16:16 + K].astype(np.float64), w.T.astype(np.float64))
    assert rel_err(got, ref) < 1e-2


def test_skinny_graph_replay(gpu):
    """A captured skinny GEMM replayed many times keeps giving the eager
    result, with eager work in between."""
    M, K, N = 8, 5120, 1280
    x = RNG.standard_normal((M, K)).astype(np.float16)
    w = RNG.standard_normal((N, K)).astype(np.float16)
    xd, wt = gpu.from_numpy(x), gpu.transpose(gpu.from_numpy(w))
    want = _np(xd @ wt)
    g = gpu.capture(lambda: xd @ wt)
    try:
        for _ in range(6):
            g.replay()
            np.testing.assert_array_equal(_np(g.outputs), want)
            _np(xd @ wt)
    finally:
        g.destroy()


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
@pytest.mark.parametrize("M,K,N", [(8, 1280, 3840), (1, 1280, 5120), (16, 4096, 64), (5, 8, 24), (12, 1360, 100),
                                   (8, 2048, 50)])
def test_layer_norm_folded_into_skinny_gemm(gpu, dt, M, K, N):
    """add_bias(layer_norm(x) @ W^T) with the layer_norm output used once:
    the graph folds the normalisation into the skinny kernel's A loads."""
    x = _round((RNG.standard_normal((M, K)) * 3 + 1).astype(np.float32), dt)
    gam = _round((RNG.standard_normal(K) * 0.5 + 1).astype(np.float32), dt)
    bet = _round((RNG.standard_normal(K) * 0.1).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K)) * 0.03).astype(np.float32), dt)
    bias = _round(RNG.standard_normal(N).astype(np.float32), dt)
    xd, gd, bd, wd, biasd = (_dev(gpu, a, dt) for a in (x, gam, bet, w, bias))
    wt = gpu.transpose(wd)
    before = gpu.graph_stats()["fused_gemm_epilogues"]
    fused = _np(gpu.add_bias(gpu.layer_norm(xd, gd, bd) @ wt, biasd))
    assert gpu.graph_stats()["fused_gemm_epilogues"] == before + 1
    h = gpu.layer_norm(xd, gd, bd)           # a live handle: no folding
    plain = _np(gpu.add_bias(h @ wt, biasd))
    ln = _round(O.layer_norm(x, gam, bet), dt)   # the layer_norm output as the device stores it
    ref = O.matmul(ln.astype(np.float64), w.T.astype(np.float64)) + bias
    assert rel_err(fused, ref) < TOL[dt]
    assert rel_err(fused, plain) < TOL[dt]


@pytest.mark.parametrize("dt,M,bk", [("float32", 8, True), ("float16", 32, True), ("float16", 8, False)])
def test_layer_norm_fold_falls_back(gpu, dt, M, bk):
    """Where the skinny kernel does not run (fp32, M > 16, W n-contiguous) the
    folded layer_norm is computed explicitly first: same result."""
    K, N = 256, 96
    x = _round(RNG.standard_normal((M, K)).astype(np.float32), dt)
    gam = _round((RNG.standard_normal(K) * 0.5 + 1).astype(np.float32), dt)
    bet = _round((RNG.standard_normal(K) * 0.1).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K) if bk else (K, N)) * 0.05).astype(np.float32), dt)
    bias = _round(RNG.standard_normal(N).astype(np.float32), dt)
    xd, gd, bd, wd, biasd = (_dev(gpu, a, dt) for a in (x, gam, bet, w, bias))
    got = _np(gpu.add_bias(gpu.layer_norm(xd, gd, bd) @ (gpu.transpose(wd) if bk else wd), biasd))
    ln = _round(O.layer_norm(x, gam, bet), dt)
    ref = O.matmul(ln.astype(np.float64), (w.T if bk else w).astype(np.float64)) + bias
    assert rel_err(got, ref) < TOL[dt]


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
@pytest.mark.parametrize("M,K,N", [(8, 1280, 3840), (8, 5120, 1280), (1, 1280, 50257), (16, 4096, 64), (3, 40, 21),
                                   (13, 776, 1001)])
def test_packed_weights_vs_oracle_and_unpacked(gpu, dt, M, K, N):
    """pack_weight + matmul_packed: zero-padded tiles for ragged N and K; the
    same MFMA sequence as the unpacked skinny kernel, so the same bits."""
    x = _round(RNG.standard_normal((M, K)).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K)) * 0.05).astype(np.float32), dt)
    xd, wd = _dev(gpu, x, dt), _dev(gpu, w, dt)
    pk = gpu.pack_weight(wd)
    assert pk.shape == [(N + 15) // 16, (K + 31) // 32, 64, 8]
    got = _np(gpu.matmul_packed(xd, pk, N))
    assert rel_err(got, O.matmul(x.astype(np.float64), w.T.astype(np.float64))) < TOL[dt]
    np.testing.assert_array_equal(got, _np(xd @ gpu.transpose(wd)))


def test_packed_layout_matches_definition(gpu):
    """packed[t][s][l][e] = W^T[16t + l%16][32s + 8(l/16) + e], zero outside."""
    N, K = 37, 72
    w = RNG.standard_normal((N, K)).astype(np.float16)
    pk = gpu.pack_weight(gpu.from_numpy(w)).to_numpy()
    want = np.zeros(pk.shape, np.float16)
    for t in range(pk.shape[0]):
        for s in range(pk.shape[1]):
            for l in range(64):
                n, k0 = 16 * t + l % 16, 32 * s + 8 * (l // 16)
                for e in range(8):
                    if n < N and k0 + e < K:
                        want[t, s, l, e] = w[n, k0 + e]
    np.testing.assert_array_equal(pk, want)


def test_packed_fused_epilogue_and_layer_norm(gpu):
    """layer_norm -> matmul_packed -> add_bias -> gelu: one fused kernel."""
    M, K, N, dt = 8, 1280, 5120, "float16"
    x = _round((RNG.standard_normal((M, K)) * 2 + 0.5).astype(np.float32), dt)
    gam = _round((RNG.standard_normal(K) * 0.5 + 1).astype(np.float32), dt)
    bet = _round((RNG.standard_normal(K) * 0.1).astype(np.float32), dt)
    w = _round((RNG.standard_normal((N, K)) * 0.03).astype(np.float32), dt)
    bias = _round(RNG.standard_normal(N).astype(np.float32), dt)
    xd, gd, bd, wd, biasd = (_dev(gpu, a, dt) for a in (x, gam, bet, w, bias))
    pk = gpu.pack_weight(wd)
    before = gpu.graph_stats()["fused_gemm_epilogues"]
    got = _np(gpu.gelu(gpu.add_bias(gpu.matmul_packed(gpu.layer_norm(xd, gd, bd), pk, N), biasd)))
    assert gpu.graph_stats()["fused_gemm_epilogues"] == before + 1
    ln = _round(O.layer_norm(x, gam, bet), dt)
    ref = O.gelu_tanh(O.matmul(ln.astype(np.float64), w.T.astype(np.float64)) + bias)
    assert rel_err(got, ref) < 1e-2


def test_packed_rejects_bad_use(gpu):
    w = gpu.cast(gpu.from_numpy(RNG.standard_normal((64, 128)).astype(np.float32)), "float16")
    pk = gpu.pack_weight(w)
    with pytest.raises(ValueError):  # 17 rows: the packed layout is for decode steps
        gpu.matmul_packed(gpu.zeros([17, 128], "float16"), pk, 64).eval()
    with pytest.raises(ValueError):  # wrong output width for these tiles
        gpu.matmul_packed(gpu.zeros([4, 128], "float16"), pk, 100).eval()
    with pytest.raises(ValueError):
        gpu.pack_weight(gpu.zeros([4, 8], "float32")).eval()
