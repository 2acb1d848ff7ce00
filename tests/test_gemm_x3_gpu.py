"""fp32 GEMM against weights packed once into bf16 hi/lo MFMA fragments
(pack_weight_x3 + matmul_packed): the packed bits against a numpy
restatement of the layout, products against the float64 oracle at the fp32
matmul bar (1e-3, checked at 1e-4), and the graph's epilogue and layer_norm
fusions on the packed path.  The reference computes these products with
MPSMatrixMultiplication (swift/Sources/AppleGPUBridge/compute.swift:1544-1630)
and its GPT-2 recipe multiplies x @ W for HF Conv1D weights
(python/applegpu_runtime/models/gpt2.py:106-107)."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(31337)


def f32(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def _check_norm(got, ref):
    """The 1e-5 relative bar for norms: normwise, and per element with an
    absolute floor of 1e-6 of the output scale."""
    assert rel_err(got, ref) < 1e-5
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6 * max(1.0, float(np.abs(ref).max())))


def _bf16_rne_bits(x):
    """bf16 bits of x rounded to nearest even (finite inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def _bits_to_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def _bits_of(t):
    """bf16 bits of a BF16 device tensor (read back as float32, exactly)."""
    return (np.asarray(t.to_numpy(), np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _valid_rows(bits, M):
    """The elements of packed rows [S, T, 2, 64, 8] that belong to rows < M
    (rows past M up to the next multiple of 32 are never written by a fused
    producer)."""
    S = bits.shape[0]
    row = 32 * np.arange(S)[:, None, None, None, None] + (np.arange(64) % 32)[None, None, None, :, None]
    return bits[np.broadcast_to(row < M, bits.shape)]


def _packed_ref(b):
    """Element ((s T + t) 2 + h) 512 + 8 l + j = part h of B(16 t + 8 (l // 32) + j, 32 s + l % 32)."""
    K, N = b.shape
    S, T = (N + 31) // 32, K // 16
    hi = _bf16_rne_bits(b)
    lo = _bf16_rne_bits(b - _bits_to_f32(hi))
    out = np.zeros((S, T, 2, 64, 8), np.uint16)
    for s in range(S):
        for t in range(T):
            for lane in range(64):
                n = 32 * s + lane % 32
                if n >= N:
                    continue
                k0 = 16 * t + 8 * (lane // 32)
                out[s, t, 0, lane] = hi[k0:k0 + 8, n]
                out[s, t, 1, lane] = lo[k0:k0 + 8, n]
    return out


def test_packed_layout_bit_exact(gpu):
    b = f32(48, 70)
    pk = gpu.pack_weight_x3(gpu.from_numpy(b))
    assert pk.shape == [3, 3, 2, 64, 8]
    np.testing.assert_array_equal(_bits_of(pk), _packed_ref(b))
    # hi + lo reconstructs b to within the dropped lo rounding (2^-16 relative)
    hl = _bits_to_f32(_packed_ref(b)[:, :, 0]) + _bits_to_f32(_packed_ref(b)[:, :, 1])
    assert np.isfinite(hl).all()


def test_packed_layout_of_a_transposed_view(gpu):
    """torch Linear weights [out, in]: B = W^T read through strides."""
    w = f32(40, 32)
    pk = gpu.pack_weight_x3(gpu.transpose(gpu.from_numpy(w)))
    np.testing.assert_array_equal(_bits_of(pk), _packed_ref(np.ascontiguousarray(w.T)))


@pytest.mark.parametrize("M,K,N", [(1, 16, 32), (5, 64, 70), (33, 48, 1536), (128, 768, 2304), (128, 768, 768),
                                   (128, 3072, 768), (128, 768, 3072), (200, 256, 100), (256, 768, 2304)])
def test_matmul_matches_oracle(gpu, M, K, N):
    a, b = f32(M, K), f32(K, N, scale=0.05)
    pk = gpu.pack_weight_x3(gpu.from_numpy(b))
    got = gpu.matmul_packed(gpu.from_numpy(a), pk, N).to_numpy()
    assert got.shape == (M, N)
    assert rel_err(got, O.matmul(a, b)) < 1e-4


def test_exact_small_integers(gpu):
    """Integers of a few bits are exact in bf16 hi alone: any fragment
    mapping error shows as a wrong integer."""
    a = RNG.integers(-3, 4, (130, 64)).astype(np.float32)
    b = RNG.integers(-3, 4, (64, 96)).astype(np.float32)
    got = gpu.matmul_packed(gpu.from_numpy(a), gpu.pack_weight_x3(gpu.from_numpy(b)), 96).to_numpy()
    np.testing.assert_array_equal(got, a @ b)


def test_strided_activations(gpu):
    """A view with a row pitch that is not 16-byte aligned is copied first."""
    base = f32(64, 70)
    a = gpu.slice(gpu.from_numpy(base), 1, 3, 67)   # [64, 64], row pitch 70
    b = f32(64, 96, scale=0.1)
    got = gpu.matmul_packed(a, gpu.pack_weight_x3(gpu.from_numpy(b)), 96).to_numpy()
    assert rel_err(got, O.matmul(base[:, 3:67], b)) < 1e-4


def test_epilogues_and_layer_norm_through_the_graph(gpu):
    """bias + gelu and bias + residual fuse into the packed GEMM's launch (or
    its split-K reduction), and a layer_norm reading the residual sum is
    computed by the reduction; results at the fp32 bars."""
    M, K, N = 128, 768, 768
    x, b, bias, r = f32(M, K), f32(K, N, scale=0.05), f32(N, scale=0.1), f32(M, N)
    g, be = f32(N, scale=0.5) + 1.0, f32(N, scale=0.1)
    pk = gpu.pack_weight_x3(gpu.from_numpy(b))
    before = gpu.graph_stats()
    y = gpu.gelu(gpu.add_bias(gpu.matmul_packed(gpu.from_numpy(x), pk, N), gpu.from_numpy(bias)))
    z = gpu.from_numpy(r) + gpu.add_bias(gpu.matmul_packed(gpu.from_numpy(x), pk, N), gpu.from_numpy(bias))
    ln = gpu.layer_norm(z, gpu.from_numpy(g), gpu.from_numpy(be))
    y_np, z_np, ln_np = y.to_numpy(), z.to_numpy(), ln.to_numpy()
    after = gpu.graph_stats()
    assert after["fused_gemm_epilogues"] - before["fused_gemm_epilogues"] == 2
    ref = O.add_bias(O.matmul(x, b), bias)
    assert rel_err(y_np, O.gelu_tanh(ref)) < 1e-4
    assert rel_err(z_np, r + ref) < 1e-4
    # the reduction's layer_norm equals layer_norm of the stored sum
    _check_norm(ln_np, O.layer_norm(z_np, g, be))


def test_rejects_unsupported_operands(gpu):
    with pytest.raises(ValueError, match="pack_weight_x3"):
        gpu.pack_weight_x3(gpu.from_numpy(f32(40, 8))).eval()        # K not a multiple of 16
    with pytest.raises(ValueError, match="pack_weight_x3"):
        gpu.pack_weight_x3(gpu.cast(gpu.from_numpy(f32(32, 8)), "float16")).eval()
    pk = gpu.pack_weight_x3(gpu.from_numpy(f32(32, 40)))
    with pytest.raises(ValueError, match="matmul_packed"):
        gpu.matmul_packed(gpu.from_numpy(f32(4, 48)), pk, 40).eval()  # K mismatch
    with pytest.raises(ValueError, match="matmul_packed"):
        gpu.matmul_packed(gpu.cast(gpu.from_numpy(f32(4, 32)), "float16"), pk, 40).eval()


@pytest.mark.parametrize("M,K,N", [(128, 768, 2304), (128, 768, 3072), (100, 256, 96), (33, 512, 64),
                                   (128, 1024, 160), (1, 768, 768)])
def test_layer_norm_folds_into_the_row_panel_prologue(gpu, M, K, N):
    """layer_norm(x) @ W + b (+ gelu) for K of 256..1024: the row-panel
    kernel normalises its rows itself, so the layer_norm costs no launch; the
    result matches the oracle's layer_norm then product at the fp32 bar."""
    x, b, bias = f32(M, K, scale=2.0) + 0.5, f32(K, N, scale=0.05), f32(N, scale=0.1)
    g, be = f32(K, scale=0.5) + 1.0, f32(K, scale=0.1)
    pk = gpu.pack_weight_x3(gpu.from_numpy(b))
    pk.eval()
    xd, gd, bd, biasd = (gpu.from_numpy(a) for a in (x, g, be, bias))
    for t in (xd, gd, bd, biasd):
        t.eval()
    y = gpu.gelu(gpu.add_bias(gpu.matmul_packed(gpu.layer_norm(xd, gd, bd), pk, N), biasd))
    before = gpu.graph_stats()
    got = y.to_numpy()
    after = gpu.graph_stats()
    assert after["launcher_calls"] - before["launcher_calls"] == 1
    ref = O.gelu_tanh(O.add_bias(O.matmul(O.layer_norm(x, g, be), b), bias))
    assert rel_err(got, ref) < 1e-4


def test_row_panel_residual_epilogue_bitwise_stable(gpu):
    """x + (a @ W + b) on the row-panel plan: at the fp32 bar, and identical
    bits on a second evaluation (fixed summation order)."""
    M, K, N = 128, 768, 768
    a, b, bias, r = f32(M, K), f32(K, N, scale=0.05), f32(N), f32(M, N)
    pk = gpu.pack_weight_x3(gpu.from_numpy(b))
    outs = []
    for _ in range(2):
        z = gpu.from_numpy(r) + gpu.add_bias(gpu.matmul_packed(gpu.from_numpy(a), pk, N), gpu.from_numpy(bias))
        outs.append(z.to_numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    assert rel_err(outs[0], r + O.add_bias(O.matmul(a, b), bias)) < 1e-4


# ── packed activation rows (pack_rows_x3 + matmul_pp) ─────────────────────
def test_pack_rows_layout_bit_exact(gpu):
    """Rows are packed in the weights' layout with rows in place of columns:
    pack_rows_x3(x) == pack_weight_x3(x^T), zero past the last row."""
    x = f32(45, 64)
    pk = gpu.pack_rows_x3(gpu.from_numpy(x))
    assert pk.shape == [2, 4, 2, 64, 8]
    np.testing.assert_array_equal(_bits_of(pk), _packed_ref(np.ascontiguousarray(x.T)))
    # a strided view packs the values it shows
    base = f32(40, 80)
    v = gpu.slice(gpu.from_numpy(base), 1, 8, 40)
    np.testing.assert_array_equal(_bits_of(gpu.pack_rows_x3(v)), _packed_ref(np.ascontiguousarray(base[:, 8:40].T)))


@pytest.mark.parametrize("M,K,N", [(128, 768, 2304), (128, 768, 3072), (128, 3072, 768), (33, 256, 96),
                                   (1, 768, 768), (100, 1280, 160), (64, 1536, 64), (40, 2048, 48), (7, 16, 40)])
def test_matmul_pp_matches_oracle(gpu, M, K, N):
    """Both operands packed: row-panel plans for K = 256..1536 (K % 256 ==
    0), split-K plans otherwise; at the fp32 bar."""
    a, b = f32(M, K), f32(K, N, scale=0.05)
    apk = gpu.pack_rows_x3(gpu.from_numpy(a))
    got = gpu.matmul_pp(apk, M, gpu.pack_weight_x3(gpu.from_numpy(b)), N).to_numpy()
    assert got.shape == (M, N)
    assert rel_err(got, O.matmul(a, b)) < 1e-4


def test_matmul_pp_exact_small_integers(gpu):
    a = RNG.integers(-3, 4, (70, 256)).astype(np.float32)
    b = RNG.integers(-3, 4, (256, 96)).astype(np.float32)
    got = gpu.matmul_pp(gpu.pack_rows_x3(gpu.from_numpy(a)), 70, gpu.pack_weight_x3(gpu.from_numpy(b)), 96)
    np.testing.assert_array_equal(got.to_numpy(), a @ b)


def test_matmul_pp_rejects_mismatches(gpu):
    apk = gpu.pack_rows_x3(gpu.from_numpy(f32(40, 64)))
    pk = gpu.pack_weight_x3(gpu.from_numpy(f32(64, 32)))
    with pytest.raises(ValueError, match="matmul_pp"):
        gpu.matmul_pp(apk, 70, pk, 32).eval()           # 70 rows need 3 strips, not 2
    with pytest.raises(ValueError, match="matmul_pp"):
        gpu.matmul_pp(apk, 40, gpu.pack_weight_x3(gpu.from_numpy(f32(48, 32))), 32).eval()  # K 64 vs 48
    with pytest.raises(ValueError, match="pack_rows_x3"):
        gpu.pack_rows_x3(gpu.from_numpy(f32(8, 40))).eval()


@pytest.mark.parametrize("M,K,N,N2", [(128, 768, 768, 3072), (128, 3072, 768, 2304), (50, 512, 256, 96)])
def test_reduction_writes_packed_layer_norm_rows(gpu, M, K, N, N2):
    """The split-K reduction that computes layer_norm(r + x W + b) writes it
    straight as packed rows for the next product: the same bits as the
    layer_norm stored in fp32 and packed by its own launch (forced by holding
    the layer_norm tensor), one launch fewer, and at the fp32 bar against the
    oracle."""
    x, w, bias, r = f32(M, K), f32(K, N, scale=0.05), f32(N, scale=0.1), f32(M, N)
    g, be = f32(N, scale=0.5) + 1.0, f32(N, scale=0.1)
    w2, b2 = f32(N, N2, scale=0.05), f32(N2, scale=0.1)
    dev = [gpu.from_numpy(a) for a in (x, bias, r, g, be, b2)]
    pk_w, pk_w2 = gpu.pack_weight_x3(gpu.from_numpy(w)), gpu.pack_weight_x3(gpu.from_numpy(w2))
    for t in dev + [pk_w, pk_w2]:
        t.eval()
    xd, bd, rd, gd, bed, bd2 = dev
    outs, ln_np = [], None
    for keep in (False, True):
        z = rd + gpu.add_bias(gpu.matmul_packed(xd, pk_w, N), bd)
        ln = gpu.layer_norm(z, gd, bed)
        y = gpu.add_bias(gpu.matmul_pp(gpu.pack_rows_x3(ln), M, pk_w2, N2), bd2)
        if not keep:
            del ln
        before = gpu.graph_stats()
        y.eval()
        after = gpu.graph_stats()
        outs.append((z.to_numpy(), y.to_numpy(), after["launcher_calls"] - before["launcher_calls"]))
        if keep:
            ln_np = ln.to_numpy()
            del ln
    (z0, y0, n0), (z1, y1, n1) = outs
    np.testing.assert_array_equal(z0, z1)
    np.testing.assert_array_equal(y0, y1)
    assert n0 == n1 - 1, (n0, n1)
    _check_norm(ln_np, O.layer_norm(z1, g, be))
    ref = O.add_bias(O.matmul(O.layer_norm(r + O.add_bias(O.matmul(x, w), bias), g, be), w2), b2)
    assert rel_err(y0, ref) < 1e-4


@pytest.mark.parametrize("M,K,N,N2", [(128, 768, 3072, 768), (70, 256, 512, 64)])
def test_gemm_epilogue_writes_packed_gelu_rows(gpu, M, K, N, N2):
    """gelu(pack_rows(x) W + b) feeding another packed product: the row-panel
    epilogue writes the packed rows itself, with no pack launch, whether or
    not the fp32 output is also kept (held outside the graph: then the same
    launch stores it too); both results are bitwise equal and at the fp32
    bar."""
    x, w, bias = f32(M, K), f32(K, N, scale=0.05), f32(N, scale=0.1)
    w2, b2 = f32(N, N2, scale=0.05), f32(N2, scale=0.1)
    pk_w, pk_w2 = gpu.pack_weight_x3(gpu.from_numpy(w)), gpu.pack_weight_x3(gpu.from_numpy(w2))
    bd, bd2 = gpu.from_numpy(bias), gpu.from_numpy(b2)
    apk = gpu.pack_rows_x3(gpu.from_numpy(x))
    for t in (pk_w, pk_w2, bd, bd2, apk):
        t.eval()
    res, f_np, apk_f = [], None, None
    for keep in (False, True):
        f = gpu.gelu(gpu.add_bias(gpu.matmul_pp(apk, M, pk_w, N), bd))
        fp = gpu.pack_rows_x3(f)
        y = gpu.add_bias(gpu.matmul_pp(fp, M, pk_w2, N2), bd2)
        if not keep:
            del f
        before = gpu.graph_stats()
        y.eval()
        after = gpu.graph_stats()
        res.append((y.to_numpy(), after["launcher_calls"] - before["launcher_calls"]))
        if keep:
            f_np = f.to_numpy()
            apk_f = fp
            del f
    (y0, n0), (y1, n1) = res
    np.testing.assert_array_equal(y0, y1)
    assert n0 == n1, (n0, n1)
    np.testing.assert_array_equal(_valid_rows(_bits_of(gpu.pack_rows_x3(gpu.from_numpy(f_np))), M),
                                  _valid_rows(_bits_of(apk_f), M))
    f_ref = O.gelu_tanh(O.add_bias(O.matmul(x, w), bias))
    assert rel_err(f_np, f_ref) < 1e-4
    assert rel_err(y0, O.add_bias(O.matmul(f_ref, w2), b2)) < 1e-4


def test_embedding_writes_packed_layer_norm_rows(gpu):
    """token + position embedding -> layer_norm -> packed rows: one fused
    embedding launch writes the packed rows; same bits as packing the stored
    layer_norm, and the product at the fp32 bar."""
    V, P, T, D, N = 97, 64, 50, 128, 96
    wte, wpe = f32(V, D), f32(P, D, scale=0.3)
    g, be = f32(D, scale=0.5) + 1.0, f32(D, scale=0.1)
    w = f32(D, N, scale=0.05)
    ids = RNG.integers(0, V, T).astype(np.int32)
    pos = np.arange(T, dtype=np.int32)
    dev = [gpu.from_numpy(a) for a in (wte, wpe, g, be, ids, pos)]
    pk_w = gpu.pack_weight_x3(gpu.from_numpy(w))
    for t in dev + [pk_w]:
        t.eval()
    wte_d, wpe_d, g_d, be_d, ids_d, pos_d = dev
    res = []
    for keep in (False, True):
        e = gpu.embedding(wte_d, ids_d) + gpu.embedding(wpe_d, pos_d)
        ln = gpu.layer_norm(e, g_d, be_d)
        y = gpu.matmul_pp(gpu.pack_rows_x3(ln), T, pk_w, N)
        if not keep:
            del ln
        before = gpu.graph_stats()
        y.eval()
        after = gpu.graph_stats()
        res.append((y.to_numpy(), after["launcher_calls"] - before["launcher_calls"]))
        if keep:
            del ln
    (y0, n0), (y1, n1) = res
    np.testing.assert_array_equal(y0, y1)
    assert n0 == n1 - 1, (n0, n1)
    ref = O.matmul(O.layer_norm(wte[ids] + wpe[pos], g, be), w)
    assert rel_err(y0, ref) < 1e-4


# ── layer_norm folded into the next packed product (row_stats_x3 + matmul_pp_norm)
def _tile_stats_ref(x):
    """(sum, sum of squared deviations from the tile mean) per 32-column tile, float64."""
    M, N = x.shape
    t = x.astype(np.float64).reshape(M, N // 32, 32)
    s = t.sum(-1)
    return np.stack([s, ((t - (s / 32)[..., None]) ** 2).sum(-1)], -1)


def test_row_stats_vs_float64(gpu):
    x = f32(37, 160, scale=3.0) + 2.0
    got = gpu.row_stats_x3(gpu.from_numpy(x)).to_numpy()
    assert got.shape == (37, 5, 2)
    np.testing.assert_allclose(got, _tile_stats_ref(x), rtol=1e-5, atol=1e-4)
    with pytest.raises(ValueError, match="row_stats_x3"):
        gpu.row_stats_x3(gpu.from_numpy(f32(4, 48))).eval()


def _fold(g, be, W, c):
    gw = (g.astype(np.float64)[:, None] * W).astype(np.float32)
    return gw, gw.astype(np.float64).sum(0).astype(np.float32), (be.astype(np.float64) @ W + c).astype(np.float32)


@pytest.mark.parametrize("M,K,N", [(128, 768, 3072), (50, 256, 96), (1, 512, 64), (33, 1024, 160)])
def test_matmul_pp_norm_vs_oracle(gpu, M, K, N):
    """layer_norm(x) @ W + c as inv * (x @ (g W) - mean * colsum(g W)) +
    (b @ W + c), with x's statistics from row_stats_x3: at the fp32 bar
    against the oracle's layer_norm then product, for rows whose mean is
    far from zero."""
    x = f32(M, K, scale=1.5) + 3.0
    g, be = f32(K, scale=0.5) + 1.0, f32(K, scale=0.1)
    W, c = f32(K, N, scale=0.05), f32(N, scale=0.1)
    gw, cs, bb = _fold(g, be, W, c)
    xd = gpu.from_numpy(x)
    y = gpu.gelu(gpu.add_bias(gpu.matmul_pp_norm(gpu.pack_rows_x3(xd), gpu.row_stats_x3(xd), M,
                                                 gpu.pack_weight_x3(gpu.from_numpy(gw)), gpu.from_numpy(cs), N),
                              gpu.from_numpy(bb)))
    ref = O.gelu_tanh(O.add_bias(O.matmul(O.layer_norm(x, g, be), W), c))
    assert rel_err(y.to_numpy(), ref) < 1e-4


def test_matmul_pp_norm_rejects_split_plans(gpu):
    x = f32(16, 2048)
    xd = gpu.from_numpy(x)
    pk = gpu.pack_weight_x3(gpu.from_numpy(f32(2048, 64)))
    with pytest.raises(ValueError, match="matmul_pp"):
        gpu.matmul_pp_norm(gpu.pack_rows_x3(xd), gpu.row_stats_x3(xd), 16, pk, gpu.from_numpy(f32(64)), 64).eval()


@pytest.mark.parametrize("M,K,N,N2", [(128, 768, 768, 3072), (70, 512, 256, 512)])
def test_producer_writes_rows_and_statistics(gpu, M, K, N, N2):
    """x1 = r + (a @ W + b) on the fp32-A row panel writes x1, its packed rows
    and its row statistics in one launch (the same bits as row_stats_x3 and
    pack_rows_x3 of the stored x1), and the folded layer_norm product reading
    them is one more launch, at the fp32 bar against the oracle."""
    a, W, b, r = f32(M, K), f32(K, N, scale=0.05), f32(N, scale=0.1), f32(M, N)
    g, be = f32(N, scale=0.5) + 1.0, f32(N, scale=0.1)
    W2, c2 = f32(N, N2, scale=0.05), f32(N2, scale=0.1)
    gw, cs, bb = _fold(g, be, W2, c2)
    dev = [gpu.from_numpy(v) for v in (a, b, r, cs, bb)]
    pk_w, pk_g = gpu.pack_weight_x3(gpu.from_numpy(W)), gpu.pack_weight_x3(gpu.from_numpy(gw))
    for t in dev + [pk_w, pk_g]:
        t.eval()
    ad, bd, rd, csd, bbd = dev
    x1 = rd + gpu.add_bias(gpu.matmul_packed(ad, pk_w, N), bd)
    st, xp = gpu.row_stats_x3(x1), gpu.pack_rows_x3(x1)
    y = gpu.gelu(gpu.add_bias(gpu.matmul_pp_norm(xp, st, M, pk_g, csd, N2), bbd))
    before = gpu.graph_stats()
    y.eval()
    after = gpu.graph_stats()
    assert after["launcher_calls"] - before["launcher_calls"] == 2
    x1_np, st_np = x1.to_numpy(), st.to_numpy()
    np.testing.assert_array_equal(st_np, gpu.row_stats_x3(gpu.from_numpy(x1_np)).to_numpy())
    np.testing.assert_array_equal(_valid_rows(_bits_of(xp), M),
                                  _valid_rows(_bits_of(gpu.pack_rows_x3(gpu.from_numpy(x1_np))), M))
    x1_ref = r + O.add_bias(O.matmul(a, W), b)
    assert rel_err(x1_np, x1_ref) < 1e-4
    ref = O.gelu_tanh(O.add_bias(O.matmul(O.layer_norm(x1_ref, g, be), W2), c2))
    assert rel_err(y.to_numpy(), ref) < 1e-4


@pytest.mark.parametrize("H,T,D,causal", [(12, 128, 64, True), (4, 50, 64, False), (2, 33, 128, True)])
def test_attention_writes_packed_rows(gpu, H, T, D, causal):
    """attention -> heads merged ([H, T, D] -> [T, H*D]) -> packed rows: the
    attention kernel writes the packed rows itself (one launch for the three
    ops); the same bits as packing the merged fp32 output, and the product
    reading them at the fp32 bar."""
    q, k, v = f32(H, T, D), f32(H, T, D), f32(H, T, D)
    N = 96
    w = f32(H * D, N, scale=0.05)
    pk = gpu.pack_weight_x3(gpu.from_numpy(w))
    dq, dk, dv = (gpu.from_numpy(a) for a in (q, k, v))
    for t in (pk, dq, dk, dv):
        t.eval()
    att = gpu.attention_causal if causal else gpu.attention
    merged = gpu.reshape(gpu.transpose_dims(att(dq, dk, dv), 0, 1), [T, H * D])
    rows = gpu.pack_rows_x3(merged)
    del merged
    before = gpu.graph_stats()
    rows.eval()
    after = gpu.graph_stats()
    assert after["launcher_calls"] - before["launcher_calls"] == 1
    ref_merged = gpu.reshape(gpu.transpose_dims(att(dq, dk, dv), 0, 1), [T, H * D]).to_numpy()
    np.testing.assert_array_equal(_valid_rows(_bits_of(rows), T),
                                  _valid_rows(_bits_of(gpu.pack_rows_x3(gpu.from_numpy(ref_merged))), T))
    o = O.attention(q, k, v, causal=causal)
    assert rel_err(ref_merged, o.transpose(1, 0, 2).reshape(T, H * D)) < 1e-4
    y = gpu.matmul_pp(rows, T, pk, N).to_numpy()
    assert rel_err(y, O.matmul(o.transpose(1, 0, 2).reshape(T, H * D), w)) < 1e-4


@pytest.mark.parametrize("M,K,N,forced", [(128, 768, 16448, False), (200, 256, 300, True), (1, 64, 130, True),
                                          (33, 512, 1000, True), (130, 96, 260, True)])
def test_weight_streaming_panel_matches_oracle(gpu, M, K, N, forced):
    """Packed rows times many columns (a vocabulary head) runs the
    vocabulary-head panel (one weight strip per wavefront, every weight byte
    read once; K = 96 leaves a partial phase of k steps); forced
    through gemm_tune's cfg 3 for small and ragged shapes and more than 128
    rows; at the fp32 bar, and exact on small integers."""
    from applegpu_runtime._native import lib
    a, b = f32(M, K), f32(K, N, scale=0.05)
    if forced:
        assert lib.applegpu_ffi_gemm_tune(0, 3, 0) == 0
    try:
        got = gpu.matmul_pp(gpu.pack_rows_x3(gpu.from_numpy(a)), M, gpu.pack_weight_x3(gpu.from_numpy(b)), N)
        got = got.to_numpy()
        ai = RNG.integers(-3, 4, (M, K)).astype(np.float32)
        bi = RNG.integers(-3, 4, (K, N)).astype(np.float32)
        exact = gpu.matmul_pp(gpu.pack_rows_x3(gpu.from_numpy(ai)), M, gpu.pack_weight_x3(gpu.from_numpy(bi)), N)
        exact = exact.to_numpy()
    finally:
        lib.applegpu_ffi_gemm_tune(0, -1, 0)
    assert rel_err(got, O.matmul(a, b)) < 1e-4
    np.testing.assert_array_equal(exact, ai @ bi)


@pytest.mark.parametrize("M,K,N,N2", [(128, 3072, 768, 2304), (70, 2048, 256, 512), (33, 4096, 256, 96)])
def test_split_panel_finishes_tiles_in_the_launch(gpu, M, K, N, N2):
    """A split packed-A row panel (2, 8 and 16 K splits at these shapes)
    whose tiles are finished in the GEMM launch by their last-arriving split:
    one launch writes x1 = r + (a @ W + b), its packed rows and its row
    statistics, and the folded layer_norm product reading them is one more;
    x1, the statistics, the packed rows and the product have the same bits
    as with the split-K reduction launch (switched back on for comparison),
    are identical over repeated launches and graph replays (the arrival
    counters return to zero), and meet the fp32 bar against the oracle."""
    from applegpu_runtime._native import lib
    a, W, b, r = f32(M, K), f32(K, N, scale=0.05), f32(N, scale=0.1), f32(M, N)
    g, be = f32(N, scale=0.5) + 1.0, f32(N, scale=0.1)
    W2, c2 = f32(N, N2, scale=0.05), f32(N2, scale=0.1)
    gw, cs, bb = _fold(g, be, W2, c2)
    ad, bd, rd, csd, bbd = (gpu.from_numpy(v) for v in (a, b, r, cs, bb))
    apk, pk_w, pk_g = gpu.pack_rows_x3(ad), gpu.pack_weight_x3(gpu.from_numpy(W)), gpu.pack_weight_x3(gpu.from_numpy(gw))
    for t in (ad, bd, rd, csd, bbd, apk, pk_w, pk_g):
        t.eval()

    def forward():
        x1 = rd + gpu.add_bias(gpu.matmul_pp(apk, M, pk_w, N), bd)
        st, xp = gpu.row_stats_x3(x1), gpu.pack_rows_x3(x1)
        return x1, st, xp, gpu.add_bias(gpu.matmul_pp_norm(xp, st, M, pk_g, csd, N2), bbd)

    def run():
        x1, st, xp, y = forward()
        before = gpu.graph_stats()["launcher_calls"]
        y.eval()
        calls = gpu.graph_stats()["launcher_calls"] - before
        return x1.to_numpy(), st.to_numpy(), _valid_rows(_bits_of(xp), M), y.to_numpy(), calls

    prev = lib.applegpu_ffi_split_inkernel(1)
    try:
        got = [run() for _ in range(2)]
        graph = gpu.capture(lambda: forward()[3])
        try:
            reps = []
            for _ in range(3):
                graph.replay()
                reps.append(graph.outputs.to_numpy())
                t = gpu.from_numpy(np.ones(64, np.float32))
                (t + t).to_numpy()
        finally:
            graph.destroy()
        lib.applegpu_ffi_split_inkernel(0)
        want = run()
    finally:
        lib.applegpu_ffi_split_inkernel(prev)
    x1, st, xp, y, calls = got[0]
    assert calls == 2, calls
    assert want[4] > 2, want[4]
    for u, v in zip(got[1][:4], got[0][:4]):
        np.testing.assert_array_equal(u, v)
    for u, v in zip(got[0][:4], want[:4]):
        np.testing.assert_array_equal(u, v)
    for rep in reps:
        np.testing.assert_array_equal(rep, y)
    np.testing.assert_array_equal(st, gpu.row_stats_x3(gpu.from_numpy(x1)).to_numpy())
    x1_ref = r + O.add_bias(O.matmul(a, W), b)
    assert rel_err(x1, x1_ref) < 1e-4
    assert rel_err(y, O.add_bias(O.matmul(O.layer_norm(x1_ref, g, be), W2), c2)) < 1e-4


def test_eval_many_runs_a_shared_producer_once(gpu):
    """eval_many over a GEMM's output, its packed rows and its row statistics:
    one launch (the row panel writes all three), the same bits as evaluating
    them one after another (three launches)."""
    M, K, N = 128, 768, 768
    a, W, b, r = f32(M, K), f32(K, N, scale=0.05), f32(N, scale=0.1), f32(M, N)
    ad, bd, rd = gpu.from_numpy(a), gpu.from_numpy(b), gpu.from_numpy(r)
    apk, pk_w = gpu.pack_rows_x3(ad), gpu.pack_weight_x3(gpu.from_numpy(W))
    for t in (ad, bd, rd, apk, pk_w):
        t.eval()

    def build():
        y = rd + gpu.add_bias(gpu.matmul_pp(apk, M, pk_w, N), bd)
        return y, gpu.pack_rows_x3(y), gpu.row_stats_x3(y)

    y, pk, st = build()
    before = gpu.graph_stats()["launcher_calls"]
    gpu.eval_many([y, pk, st])
    assert gpu.graph_stats()["launcher_calls"] - before == 1
    y2, pk2, st2 = build()
    for t in (y2, pk2, st2):
        t.eval()
    np.testing.assert_array_equal(y.to_numpy(), y2.to_numpy())
    np.testing.assert_array_equal(st.to_numpy(), st2.to_numpy())
    np.testing.assert_array_equal(_valid_rows(_bits_of(pk), M), _valid_rows(_bits_of(pk2), M))
    assert rel_err(y.to_numpy(), r + O.add_bias(O.matmul(a, W), b)) < 1e-4
    with pytest.raises(ValueError):
        gpu.eval_many([y, 123456789])
