"""KV-cache decode: the in-place cache append, split-KV decode attention over
device-resident lengths, strided copies into views, and batched greedy
generation (prefill + decode steps, eager and graph-replayed) against the
oracle, teacher-forced."""
import numpy as np
import pytest

from conftest import rel_err
from oracle import models as M
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(2024)


def _dev(gpu, a, dtype):
    t = gpu.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t if dtype == "float32" else gpu.cast(t, dtype)


def _host(t):
    return np.asarray(t.to_numpy(), dtype=np.float32)


def _round(a, dtype):
    """a rounded to the device dtype (the oracle's inputs are the device's)."""
    if dtype == "float16":
        return a.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        return u.astype(np.uint32).view(np.float32)
    return a.astype(np.float32)


# ── strided copy into views ────────────────────────────────────────────────
def test_blit_copy_into_slice_and_transpose(gpu):
    base = RNG.standard_normal((6, 10)).astype(np.float32)
    dst = gpu.from_numpy(base)
    src = RNG.standard_normal((6, 3)).astype(np.float32)
    gpu.blit_copy(gpu.from_numpy(src), gpu.slice(dst, 1, 4, 7))
    want = base.copy()
    want[:, 4:7] = src
    np.testing.assert_array_equal(dst.to_numpy(), want)
    # transposed destination, with a dtype cast from int32
    src2 = RNG.integers(-50, 50, (10, 6)).astype(np.int32)
    gpu.blit_copy(gpu.from_numpy(src2), gpu.transpose(dst))
    np.testing.assert_array_equal(dst.to_numpy(), src2.T.astype(np.float32))


def test_blit_copy_rejects_mismatched_count(gpu):
    t = gpu.from_numpy(np.zeros((1, 4), np.float32))
    with pytest.raises(ValueError):
        gpu.blit_copy(gpu.from_numpy(np.ones((3, 4), np.float32)), t)
    gpu.blit_copy(gpu.from_numpy(np.ones(4, np.float32)), t)   # same count, other shape
    np.testing.assert_array_equal(t.to_numpy(), np.ones((1, 4), np.float32))


# ── kv_write ───────────────────────────────────────────────────────────────
@pytest.mark.parametrize("dtype", ["float16", "float32", "bfloat16"])
def test_kv_write_ragged_positions_bit_exact(gpu, dtype):
    B, H, Tmax, D, T = 4, 3, 11, 64, 3
    cache0 = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    rows = _round(RNG.standard_normal((B, T, H, D)).astype(np.float32), dtype)
    pos = np.array([0, 5, 9, 11], np.int32)   # last two spill past the end
    cache = _dev(gpu, cache0, dtype)
    # rows arrive as a [B, H, T, D] view of a [B, T, H, D] tensor (the head
    # split of a fused projection)
    r = gpu.transpose_dims(_dev(gpu, rows, dtype), 1, 2)
    gpu.kv_write(cache, r, gpu.from_numpy(pos))
    want = cache0.copy()
    for b in range(B):
        for t in range(T):
            if pos[b] + t < Tmax:
                want[b, :, pos[b] + t, :] = rows[b, t]
    np.testing.assert_array_equal(_host(cache), want)


def test_kv_write_pair_bit_exact(gpu):
    """K and V rows of a fused QKV projection into two caches in one launch."""
    B, H, Tmax, D, T = 3, 4, 9, 64, 2
    kc0 = RNG.standard_normal((B, H, Tmax, D)).astype(np.float16)
    vc0 = RNG.standard_normal((B, H, Tmax, D)).astype(np.float16)
    qkv = RNG.standard_normal((B, T, 3, H, D)).astype(np.float16)
    pos = np.array([0, 4, 8], np.int32)
    kc, vc = gpu.from_numpy(kc0), gpu.from_numpy(vc0)
    qd = gpu.reshape(gpu.from_numpy(qkv), [B, T, 3 * H * D])
    rows = [gpu.transpose_dims(gpu.reshape(gpu.slice(qd, 2, j * H * D, (j + 1) * H * D), [B, T, H, D]), 1, 2)
            for j in (1, 2)]
    gpu.kv_write_pair(kc, vc, rows[0], rows[1], gpu.from_numpy(pos))
    wk, wv = kc0.copy(), vc0.copy()
    for b in range(B):
        for t in range(T):
            if pos[b] + t < Tmax:
                wk[b, :, pos[b] + t] = qkv[b, t, 1]
                wv[b, :, pos[b] + t] = qkv[b, t, 2]
    np.testing.assert_array_equal(kc.to_numpy(), wk)
    np.testing.assert_array_equal(vc.to_numpy(), wv)
    with pytest.raises(ValueError, match="kv_write"):
        gpu.kv_write_pair(kc, gpu.zeros([B, H, Tmax + 1, D], "float16"), rows[0], rows[1], gpu.from_numpy(pos))


def test_kv_write_rejects_bad_operands(gpu):
    cache = gpu.zeros([2, 2, 8, 32], "float16")
    rows = gpu.zeros([2, 2, 1, 32], "float32")
    with pytest.raises(ValueError, match="kv_write"):
        gpu.kv_write(cache, rows, gpu.from_numpy(np.zeros(2, np.int32)))
    rows = gpu.zeros([2, 2, 1, 32], "float16")
    with pytest.raises(ValueError, match="kv_write"):
        gpu.kv_write(cache, rows, gpu.from_numpy(np.zeros(3, np.int32)))
    with pytest.raises(ValueError, match="kv_write"):
        gpu.kv_write(cache, rows, gpu.from_numpy(np.zeros(2, np.int64)))
    with pytest.raises(ValueError, match="kv_write"):
        gpu.kv_write(cache, gpu.zeros([2, 2, 9, 32], "float16"), gpu.from_numpy(np.zeros(2, np.int32)))


# ── decode attention ───────────────────────────────────────────────────────
def _decode_ref(q, kc, vc, lens):
    """Query row i of sequence b attends to cache rows j <= lens[b] - Tq + i
    (with Tq = 1: the reference's non-causal attention of the new token over
    the whole cache, python/applegpu_runtime/models/gpt2.py:132-135)."""
    B, H, Tq, D = q.shape
    Tmax = kc.shape[2]
    out = np.zeros((B, H, Tq, D), np.float64)
    for b in range(B):
        n = int(min(max(lens[b], 0), Tmax))
        for i in range(Tq):
            vis = max(0, min(n, n - Tq + i + 1))
            if vis == 0:
                continue
            out[b, :, i] = O.attention(q[b, :, i:i + 1].astype(np.float64), kc[b, :, :vis].astype(np.float64),
                                       vc[b, :, :vis].astype(np.float64))[:, 0]
    return out


@pytest.mark.parametrize("dtype,tol", [("float32", 1e-3), ("float16", 1e-2), ("bfloat16", 2e-2)])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("Tmax,Tq", [(1, 1), (7, 1), (129, 1), (640, 1), (1000, 3)])
def test_decode_attention_vs_oracle(gpu, dtype, tol, D, Tmax, Tq):
    B, H = 3, 2
    q = _round(RNG.standard_normal((B, H, Tq, D)).astype(np.float32), dtype)
    kc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    vc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    lens = np.array([Tmax, max(Tq, Tmax // 2 + 1), min(Tq, Tmax)], np.int32)
    got = gpu.decode_attention(_dev(gpu, q, dtype), _dev(gpu, kc, dtype), _dev(gpu, vc, dtype),
                               gpu.from_numpy(lens))
    assert got.shape == [B, H, Tq, D]
    ref = _decode_ref(q, kc, vc, lens)
    assert rel_err(_host(got), ref) < tol


@pytest.mark.parametrize("dtype,tol", [("float32", 1e-3), ("float16", 1e-2)])
@pytest.mark.parametrize("B,H,Tq,Tmax,D", [(8, 20, 1, 640, 64), (4, 16, 2, 300, 128), (2, 64, 1, 97, 32)])
def test_decode_attention_whole_row_blocks_vs_oracle(gpu, dtype, tol, B, H, Tq, Tmax, D):
    """At least 128 (batch, head, query) rows: one 16-wave block per row over
    the whole context (the C4 decode shape is the first case)."""
    q = _round(RNG.standard_normal((B, H, Tq, D)).astype(np.float32), dtype)
    kc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    vc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    lens = np.linspace(Tq, Tmax, B).astype(np.int32)
    lens[0] = 0 if Tq == 1 else Tq   # an empty row (zeros) when allowed
    lens[-1] = Tmax
    got = gpu.decode_attention(_dev(gpu, q, dtype), _dev(gpu, kc, dtype), _dev(gpu, vc, dtype),
                               gpu.from_numpy(lens))
    assert rel_err(_host(got), _decode_ref(q, kc, vc, lens)) < tol


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("B,H,Tmax,D", [(8, 20, 640, 64), (2, 3, 300, 64), (4, 2, 97, 128), (8, 20, 97, 32)])
def test_decode_attention_appending_new_rows(gpu, dtype, B, H, Tmax, D):
    """k_new/v_new: the launch appends the step's K/V rows (as cache row
    lens - 1) and attends over them.  Both caches equal kv_write_pair's bit
    for bit; the output equals kv_write_pair followed by decode_attention up
    to summation order (the new key is the last online-softmax term of its
    block) and the float64 oracle within the attention bar, in whole-row
    (B*H >= 128) and split-KV blocks, for lengths that put the new row in
    the first key block, the middle and the last cache row."""
    q = _round(RNG.standard_normal((B, H, 1, D)).astype(np.float32), dtype)
    kc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    vc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    kn = _round(RNG.standard_normal((B, H, 1, D)).astype(np.float32), dtype)
    vn = _round(RNG.standard_normal((B, H, 1, D)).astype(np.float32), dtype)
    lens = np.linspace(1, Tmax, B).astype(np.int32)
    lens[-1] = Tmax
    pos = (lens - 1).astype(np.int32)
    # fused
    k1, v1 = _dev(gpu, kc, dtype), _dev(gpu, vc, dtype)
    got = gpu.decode_attention(_dev(gpu, q, dtype), k1, v1, gpu.from_numpy(lens),
                               k_new=_dev(gpu, kn, dtype), v_new=_dev(gpu, vn, dtype))
    got_h = _host(got)
    # two launches
    k2, v2 = _dev(gpu, kc, dtype), _dev(gpu, vc, dtype)
    gpu.kv_write_pair(k2, v2, _dev(gpu, kn, dtype), _dev(gpu, vn, dtype), gpu.from_numpy(pos))
    want = _host(gpu.decode_attention(_dev(gpu, q, dtype), k2, v2, gpu.from_numpy(lens)))
    if dtype == "float32":
        np.testing.assert_allclose(got_h, want, rtol=1e-5, atol=1e-6)
    else:  # one rounding of the 16-bit output apart
        np.testing.assert_allclose(got_h, want, rtol=1e-2, atol=1e-3)
    np.testing.assert_array_equal(_host(k1), _host(k2))
    np.testing.assert_array_equal(_host(v1), _host(v2))
    kref, vref = kc.copy(), vc.copy()
    for bi in range(B):
        kref[bi, :, pos[bi]] = kn[bi, :, 0]
        vref[bi, :, pos[bi]] = vn[bi, :, 0]
    tol = 1e-3 if dtype == "float32" else 2e-2
    assert rel_err(got_h, _decode_ref(q, kref, vref, lens)) < tol


def test_decode_attention_new_rows_past_the_cache_are_dropped(gpu):
    """A length past Tmax: the cache keeps its rows (kv_write drops such rows
    too) and attention covers the whole cache."""
    B, H, Tmax, D = 2, 2, 40, 64
    q = RNG.standard_normal((B, H, 1, D)).astype(np.float32)
    kc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    vc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    kn = RNG.standard_normal((B, H, 1, D)).astype(np.float32)
    kd, vd = gpu.from_numpy(kc), gpu.from_numpy(vc)
    lens = np.array([Tmax + 1, 5], np.int32)
    gpu.decode_attention(gpu.from_numpy(q), kd, vd, gpu.from_numpy(lens), k_new=gpu.from_numpy(kn),
                         v_new=gpu.from_numpy(kn)).eval()
    np.testing.assert_array_equal(_host(kd)[0], kc[0])      # nothing stored for sequence 0
    np.testing.assert_array_equal(_host(kd)[1, :, 4], kn[1, :, 0])


def test_decode_attention_new_rows_reject_bad_shapes(gpu):
    q = gpu.from_numpy(RNG.standard_normal((1, 2, 2, 64)).astype(np.float32))
    kc = gpu.from_numpy(RNG.standard_normal((1, 2, 8, 64)).astype(np.float32))
    kn = gpu.from_numpy(RNG.standard_normal((1, 2, 1, 64)).astype(np.float32))
    lens = gpu.from_numpy(np.array([4], np.int32))
    with pytest.raises(ValueError):   # two query rows
        gpu.decode_attention(q, kc, kc, lens, k_new=kn, v_new=kn).eval()
    with pytest.raises(ValueError):   # V row missing
        gpu.decode_attention(gpu.slice(q, 2, 0, 1), kc, kc, lens, k_new=kn).eval()


def test_decode_step_folds_every_layer_norm(gpu):
    """One decode step is one lazy graph (the K/V append rides in the
    attention launch), in which every ln_1/ln_2 feeds a skinny GEMM that
    normalises its rows itself, even where the same layer_norm also reads
    the previous GEMM group's output: per layer 2 folded layer_norms plus
    the bias/residual/gelu epilogues: 9 launches saved per layer."""
    from applegpu_runtime.models import gpt2 as G
    cfg = {"vocab_size": 300, "n_positions": 64, "n_embd": 128, "n_layer": 3, "n_head": 2}
    model = G.load_model(G.random_weights(cfg, seed=9), cfg, dtype="float16")
    cache = G.KVCache(cfg, batch=4, max_len=32, dtype="float16")
    prompt = RNG.integers(0, cfg["vocab_size"], (4, 8)).astype(np.int32)
    _, tok = G.gpt2_prefill(model, gpu.from_numpy(prompt), cache)
    gpu.blit_copy(gpu.from_numpy(np.full(4, 8, np.int32)), cache.pos)
    before = gpu.graph_stats()["launches_saved"]
    logits, nxt, lens = G.gpt2_decode_step(model, tok, cache)
    nxt.eval()
    saved = gpu.graph_stats()["launches_saved"] - before
    assert saved >= 9 * cfg["n_layer"], saved


def test_decode_attention_empty_and_clamped_lengths(gpu):
    """len 0 gives zeros; lengths past the cache are clamped to it."""
    B, H, Tmax, D = 3, 2, 70, 64
    q = RNG.standard_normal((B, H, 1, D)).astype(np.float32)
    kc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    vc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    lens = np.array([0, 10_000, -3], np.int32)
    got = gpu.decode_attention(gpu.from_numpy(q), gpu.from_numpy(kc), gpu.from_numpy(vc), gpu.from_numpy(lens))
    ref = _decode_ref(q, kc, vc, np.array([0, Tmax, 0]))
    np.testing.assert_array_equal(_host(got)[0], 0)
    np.testing.assert_array_equal(_host(got)[2], 0)
    assert rel_err(_host(got), ref) < 1e-3


@pytest.mark.parametrize("dtype", ["float16", "float32"])
@pytest.mark.parametrize("B,H", [(8, 20), (2, 2)])
def test_decode_attention_ignores_nan_in_unused_cache_rows(gpu, dtype, B, H):
    """Rows past each sequence's length hold NaN and Inf: masked keys add
    nothing, so the output equals attention over the valid rows alone, in
    whole-row and split-KV blocks, with and without the appended new row."""
    Tmax, D = 200, 64
    q = _round(RNG.standard_normal((B, H, 1, D)).astype(np.float32), dtype)
    kc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    vc = _round(RNG.standard_normal((B, H, Tmax, D)).astype(np.float32), dtype)
    lens = np.linspace(3, Tmax - 5, B).astype(np.int32)
    kbad, vbad = kc.copy(), vc.copy()
    for b in range(B):
        kbad[b, :, lens[b]:] = np.nan
        vbad[b, :, lens[b]:] = np.inf
        vbad[b, :, lens[b]::2] = np.nan
    got = gpu.decode_attention(_dev(gpu, q, dtype), _dev(gpu, kbad, dtype), _dev(gpu, vbad, dtype),
                               gpu.from_numpy(lens))
    got_h = _host(got)
    assert np.isfinite(got_h).all()
    tol = 1e-3 if dtype == "float32" else 1e-2
    assert rel_err(got_h, _decode_ref(q, kc, vc, lens)) < tol
    # the step's own row appended at lens - 1, NaN beyond it
    kn = _round(RNG.standard_normal((B, H, 1, D)).astype(np.float32), dtype)
    vn = _round(RNG.standard_normal((B, H, 1, D)).astype(np.float32), dtype)
    got2 = gpu.decode_attention(_dev(gpu, q, dtype), _dev(gpu, kbad, dtype), _dev(gpu, vbad, dtype),
                                gpu.from_numpy(lens + 1), k_new=_dev(gpu, kn, dtype), v_new=_dev(gpu, vn, dtype))
    kref, vref = kc.copy(), vc.copy()
    for b in range(B):
        kref[b, :, lens[b]] = kn[b, :, 0]
        vref[b, :, lens[b]] = vn[b, :, 0]
    got2_h = _host(got2)
    assert np.isfinite(got2_h).all()
    assert rel_err(got2_h, _decode_ref(q, kref, vref, lens + 1)) < (1e-3 if dtype == "float32" else 2e-2)


def test_decode_attention_matches_attention_on_full_cache(gpu):
    """With every row valid and Tq = 1 it is the reference's decode attention
    (non-causal over the whole cache) — the fused attention kernel's answer."""
    B, H, Tmax, D = 2, 4, 96, 64
    q = RNG.standard_normal((B, H, 1, D)).astype(np.float32)
    kc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    vc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    qd, kd, vd = gpu.from_numpy(q), gpu.from_numpy(kc), gpu.from_numpy(vc)
    got = gpu.decode_attention(qd, kd, vd, gpu.from_numpy(np.full(B, Tmax, np.int32)))
    want = gpu.attention(qd, kd, vd)
    assert rel_err(_host(got), _host(want)) < 1e-5


def test_decode_attention_multi_query_is_causal_tail(gpu):
    """Tq new rows at the end of the cache: the causal attention of those rows
    over the cache's first len rows (chunked-prefill semantics)."""
    B, H, Tmax, D, Tq = 2, 2, 40, 64, 5
    kc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    vc = RNG.standard_normal((B, H, Tmax, D)).astype(np.float32)
    n = 23
    q = RNG.standard_normal((B, H, Tq, D)).astype(np.float32)
    got = gpu.decode_attention(gpu.from_numpy(q), gpu.from_numpy(kc), gpu.from_numpy(vc),
                               gpu.from_numpy(np.full(B, n, np.int32)))
    # the same rows through a full causal attention over [0, n)
    qf = np.zeros((B, H, n, D), np.float32)
    qf[:, :, n - Tq:] = q
    full = O.attention(qf, kc[:, :, :n], vc[:, :, :n], causal=True)[:, :, n - Tq:]
    assert rel_err(_host(got), full) < 1e-3


def test_decode_attention_rejects_bad_operands(gpu):
    q = gpu.zeros([2, 2, 1, 64], "float16")
    kc = gpu.zeros([2, 2, 16, 64], "float16")
    lens = gpu.from_numpy(np.ones(2, np.int32))
    with pytest.raises(ValueError, match="decode_attention"):
        gpu.decode_attention(q, gpu.zeros([2, 2, 16, 64], "float32"), kc, lens)
    with pytest.raises(ValueError, match="decode_attention"):
        gpu.decode_attention(q, kc, kc, gpu.from_numpy(np.ones(3, np.int32)))
    with pytest.raises(ValueError, match="decode_attention"):
        gpu.decode_attention(gpu.zeros([2, 2, 1, 48], "float16"), gpu.zeros([2, 2, 16, 48], "float16"),
                             gpu.zeros([2, 2, 16, 48], "float16"), lens)


# ── batched greedy generation ──────────────────────────────────────────────
TINY = dict(n_layer=2, n_head=4, n_embd=256, vocab_size=1000, n_positions=64)


def _tiny_model(dtype="float16", seed=11, std=0.2):
    from applegpu_runtime.models import gpt2 as G
    w = G.random_weights(TINY, seed=seed, std=std)
    model = G.load_model(w, TINY, dtype=dtype)
    # the oracle sees the device's rounded weights
    wr = {k: _round(v, dtype) for k, v in w.items()}
    return G, model, wr


def _check_teacher_forced(prompt, toks, logits, wr, cfg, tol):
    """Step s of sequence b must give the oracle's logits at position T-1+s
    of prompt + generated tokens, fed the device's own tokens; each greedy
    pick must be the oracle's argmax unless the oracle's top two are within
    the tolerance."""
    B, T = prompt.shape
    n = toks.shape[1]
    for b in range(B):
        seq = np.concatenate([prompt[b], toks[b, :-1]])
        ref, _ = M.gpt2_forward_np(wr, cfg, seq)
        ref_steps = ref[T - 1:T - 1 + n]
        assert rel_err(logits[:, b], ref_steps) < tol, b
        for s in range(n):
            top2 = np.sort(ref_steps[s])[-2:]
            if top2[1] - top2[0] > tol * np.abs(ref_steps[s]).max():
                assert toks[b, s] == int(np.argmax(ref_steps[s])), (b, s)


@pytest.mark.parametrize("capture", [False, True])
def test_generate_greedy_tiny_vs_oracle(gpu, capture):
    G, model, wr = _tiny_model()
    B, T, n = 3, 13, 6
    prompt = np.random.default_rng(5).integers(0, TINY["vocab_size"], (B, T)).astype(np.int32)
    toks, logits = G.generate_greedy(model, prompt, n, capture=capture, keep_logits=True)
    assert toks.shape == (B, n + 1) and toks.dtype == np.int32
    assert logits.shape == (n + 1, B, TINY["vocab_size"])
    np.testing.assert_array_equal(toks, logits.argmax(-1).T)
    _check_teacher_forced(prompt, toks, logits, wr, TINY, 1e-2)


def test_generate_greedy_fp32_tight(gpu):
    """The same path in fp32 at the fp32 attention/matmul bar."""
    G, model, wr = _tiny_model(dtype="float32", seed=12)
    B, T, n = 2, 9, 4
    prompt = np.random.default_rng(6).integers(0, TINY["vocab_size"], (B, T)).astype(np.int32)
    toks, logits = G.generate_greedy(model, prompt, n, capture=True, keep_logits=True)
    _check_teacher_forced(prompt, toks, logits, wr, TINY, 1e-3)


def test_generate_replay_matches_eager_bitwise(gpu):
    """Graph replay launches the same kernels on the same data: identical
    tokens and logits."""
    G, model, _ = _tiny_model(seed=13)
    prompt = np.random.default_rng(7).integers(0, TINY["vocab_size"], (4, 10)).astype(np.int32)
    t0, l0 = G.generate_greedy(model, prompt, 5, capture=False, keep_logits=True)
    t1, l1 = G.generate_greedy(model, prompt, 5, capture=True, keep_logits=True)
    np.testing.assert_array_equal(t0, t1)
    np.testing.assert_array_equal(l0, l1)


def test_prefill_fills_cache_like_incremental_decode(gpu):
    """Prefill of prompt + generated tokens gives, at its last position, the
    logits the decode steps gave: incremental == full recompute."""
    G, model, _ = _tiny_model(seed=14)
    B, T, n = 2, 8, 5
    prompt = np.random.default_rng(8).integers(0, TINY["vocab_size"], (B, T)).astype(np.int32)
    toks, logits = G.generate_greedy(model, prompt, n, capture=True, keep_logits=True)
    full_ids = np.concatenate([prompt, toks[:, :-1]], axis=1)
    cache = G.KVCache(TINY, B, T + n, "float16")
    lg, nxt = G.gpt2_prefill(model, full_ids, cache)
    V = TINY["vocab_size"]
    last = lg.to_numpy().astype(np.float32).reshape(B, T + n, V)[:, -1]
    assert rel_err(logits[-1], last) < 1e-2
    np.testing.assert_array_equal(nxt.to_numpy(), toks[:, -1])


def test_kv_cache_capacity_is_checked(gpu):
    G, model, _ = _tiny_model(seed=15)
    cache = G.KVCache(TINY, 2, 10, "float16")
    with pytest.raises(ValueError):
        G.generate_greedy(model, np.zeros((2, 8), np.int32), 5, cache=cache)
    with pytest.raises(ValueError):
        G.KVCache(TINY, 2, TINY["n_positions"] + 1)
