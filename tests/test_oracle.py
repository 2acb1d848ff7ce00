"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each oracle function is checked against at least one of: the reference's own
known answers (tests/golden/reference_known_answers.json), PyTorch CPU (the
reference's ground truth; tests/golden/torch_cpu_fixtures.npz and live torch),
closed forms, or brute force — chosen so that a plausible slip (a dropped
term, a wrong sign, an off-by-one in the causal mask, a transposed operand,
the wrong rounding mode) fails.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as O
from oracle import models as M


def test_known_answers(known):
    for k in known:
        op = k["op"]
        if op == "matmul":
            got = O.matmul(np.array(k["a"], np.float32), np.array(k["b"], np.float32))
            np.testing.assert_array_equal(got, np.array(k["expect"], np.float32), err_msg=k["src"])
        elif op == "relu":
            np.testing.assert_array_equal(O.relu(np.array(k["x"], np.float32)), k["expect"])
        elif op == "softmax":
            np.testing.assert_allclose(O.softmax(np.array(k["x"], np.float32)), k["expect"], atol=k["atol"])
        elif op == "softmax_causal":
            np.testing.assert_allclose(O.softmax_causal(np.array(k["x"], np.float32)), k["expect"], atol=k["atol"])
        elif op == "attention_causal_row0":
            out = O.attention(*(np.array(k[n], np.float32) for n in "qkv"), causal=True)
            np.testing.assert_allclose(out[0], k["expect_row0"], atol=k["atol"])
        elif op == "softmax_rows_sum":
            np.testing.assert_allclose(O.softmax(np.array(k["x"], np.float32)).sum(-1), k["expect_row_sums"],
                                       atol=k["atol"])
        elif op == "transpose":
            np.testing.assert_array_equal(np.array(k["x"]).T, k["expect"])
        elif op == "layer_norm":
            got = O.layer_norm(np.array(k["x"], np.float32), np.array(k["gamma"], np.float32),
                               np.array(k["beta"], np.float32))
            np.testing.assert_allclose(got, k["expect"], rtol=k["rtol"], atol=1e-6)
        elif op == "gelu":
            np.testing.assert_allclose(O.gelu_tanh(np.array(k["x"], np.float32)), k["expect"], rtol=k["rtol"],
                                       atol=1e-7)
        elif op == "embedding":
            np.testing.assert_array_equal(O.embedding(np.array(k["w"], np.float32), k["idx"]),
                                          np.array(k["expect"], np.float32))
        elif op == "softmax_backward":
            got = O.softmax_backward(np.array(k["dy"], np.float32), np.array(k["y"], np.float32))
            np.testing.assert_allclose(got, k["expect"], atol=k["atol"], err_msg=k["src"])
            np.testing.assert_allclose(got.sum(-1), 0.0, atol=k["atol"])
        elif op == "softmax_backward_ones":
            y = O.softmax(np.array(k["x"], np.float32))
            got = O.softmax_backward(np.ones_like(y), y)
            assert np.abs(got).max() <= k["expect_abs_max"] + k["atol"], k["src"]
        elif op == "layer_norm_backward_row_sums":
            got = O.layer_norm_backward(np.array(k["dy"], np.float32), np.array(k["x"], np.float32),
                                        np.array(k["gamma"], np.float32))
            np.testing.assert_allclose(got.sum(-1), k["expect_row_sums"], atol=k["atol"], err_msg=k["src"])
        elif op == "embedding_backward":
            got = O.embedding_backward(np.array(k["dy"], np.float32), k["idx"], k["num_weights"])
            np.testing.assert_allclose(got, k["expect"], atol=k["atol"], err_msg=k["src"])
        else:
            raise AssertionError(f"unhandled known answer {op}")


@pytest.mark.parametrize("name", ["r7", "r768", "r2500"])
def test_rows_vs_torch(fixtures, name):
    x = fixtures[f"softmax_{name}_x"]
    np.testing.assert_allclose(O.softmax(x), fixtures[f"softmax_{name}_y"], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(O.log_softmax(x), fixtures[f"log_softmax_{name}_y"], rtol=1e-5, atol=1e-5)
    y = O.layer_norm(x, fixtures[f"layer_norm_{name}_g"], fixtures[f"layer_norm_{name}_b"])
    np.testing.assert_allclose(y, fixtures[f"layer_norm_{name}_y"], rtol=1e-4, atol=1e-5)


def test_softmax_causal_vs_torch(fixtures):
    np.testing.assert_allclose(O.softmax_causal(fixtures["softmax_causal_x"]), fixtures["softmax_causal_y"],
                               rtol=1e-5, atol=1e-7)
    # brute force on one matrix: row i is a plain softmax over x[i, :i+1]
    x = fixtures["softmax_causal_x"][1]
    got = O.softmax_causal(x)
    for i in range(x.shape[0]):
        e = np.exp(x[i, :i + 1].astype(np.float64) - x[i, :i + 1].max())
        np.testing.assert_allclose(got[i, :i + 1], e / e.sum(), rtol=1e-6)
        assert np.all(got[i, i + 1:] == 0)


def test_gelu_vs_torch(fixtures):
    np.testing.assert_allclose(O.gelu_tanh(fixtures["gelu_x"]), fixtures["gelu_tanh_y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(O.gelu_erf(fixtures["gelu_x"]), fixtures["gelu_erf_y"], rtol=1e-5, atol=1e-6)
    # the +-10 clamp of the reference is invisible at fp32: tanh(10) rounds to 1
    assert np.float32(np.tanh(10.0)) == np.float32(1.0)


def test_matmul_vs_torch_and_brute_force(fixtures):
    a, b = fixtures["matmul_a"], fixtures["matmul_b"]
    np.testing.assert_allclose(O.matmul(a, b), fixtures["matmul_y"], rtol=1e-4, atol=1e-4)
    # brute-force dot products on a corner (catches transposed operands)
    for i, j in [(0, 0), (5, 3), (36, 28)]:
        assert abs(O.matmul(a, b)[i, j] - sum(float(a[i, t]) * float(b[t, j]) for t in range(a.shape[1]))) < 1e-4
    # transposed-operand variants against explicit transposes
    np.testing.assert_allclose(O.matmul_ex(a.T.copy(), b, ta=True), O.matmul(a, b), rtol=1e-6)
    np.testing.assert_allclose(O.matmul_ex(a, b.T.copy(), tb=True), O.matmul(a, b), rtol=1e-6)
    # a 2-D B shared across batches
    a3 = np.stack([a, 2 * a])
    np.testing.assert_allclose(O.matmul(a3, b)[1], 2 * O.matmul(a, b), rtol=1e-6)


def test_attention_vs_torch(fixtures):
    q, k, v = fixtures["attn_q"], fixtures["attn_k"], fixtures["attn_v"]
    np.testing.assert_allclose(O.attention(q, k, v, causal=True), fixtures["attn_causal_y"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(O.attention(q, k, v), fixtures["attn_full_y"], rtol=1e-4, atol=1e-5)
    # the composition the reference records (ops.rs:1577-1620) equals the oracle
    s = O.matmul(q, np.swapaxes(k, -1, -2)) * np.float32(1 / math.sqrt(64))
    comp = O.matmul(O.softmax_causal(s), v)
    np.testing.assert_allclose(O.attention(q, k, v, causal=True), comp, rtol=1e-4, atol=1e-5)


def test_argmax_vs_torch(fixtures):
    np.testing.assert_array_equal(O.argmax(fixtures["argmax_x"]), fixtures["argmax_y"])
    x = np.array([[1, 3, 3, 2], [np.nan, 5, 1, np.nan], [0, 0, 0, 0], [2, np.nan, 9, 9]], np.float32)
    np.testing.assert_array_equal(O.argmax(x), torch.from_numpy(x).argmax(-1).numpy())
    assert O.argmax(np.array([4.0, 7.0, 7.0], np.float32)).tolist() == [1]


def test_quantize_per_row_vs_torch(fixtures):
    q, s = O.quantize_per_row(fixtures["quant_w"])
    np.testing.assert_array_equal(q, fixtures["quant_q"])
    np.testing.assert_array_equal(s, fixtures["quant_scale"])
    assert np.all(q[3] == 0) and s[3] == 0
    # ties round half to even: codes of the planted .5 multiples
    assert s[5] == np.float32(2.0 ** -10)
    assert q[5, :5].tolist() == [127, 0, 0, 2, -2]
    # dequantize against torch, two routes: fp32 arithmetic on torch's codes
    # and torch's per-channel quantized tensor (bit-exact; the products are
    # exact in fp32 up to one rounding)
    d = O.dequantize_per_row(fixtures["quant_q"], fixtures["quant_scale"])
    np.testing.assert_array_equal(d, fixtures["quant_deq"])
    np.testing.assert_array_equal(d, fixtures["quant_deq_qtensor"])
    # round trip: every value within half a step of its row's scale
    w = fixtures["quant_w"]
    assert np.all(np.abs(O.dequantize_per_row(q, s) - w) <= s[:, None] * 0.5000001)


def test_dequantize_per_tensor_vs_torch(fixtures):
    # (q - zp) * scale (kernel_templates.rs:2222-2240) against torch's
    # per-tensor quantized tensors, every int8 and uint8 code
    np.testing.assert_array_equal(O.dequantize_per_tensor(fixtures["dq_pt_i8_q"], 0.1, -3), fixtures["dq_pt_i8_y"])
    np.testing.assert_array_equal(O.dequantize_per_tensor(fixtures["dq_pt_u8_q"], 0.05, 7), fixtures["dq_pt_u8_y"])


def test_quantize_per_tensor_half_away():
    # MSL round(): half away from zero (kernel_templates.rs:2207-2212)
    x = np.array([0.25, -0.25, 0.75, -0.75, 1.25, 0.049999997, 100.0, -100.0], np.float32)
    q = O.quantize_per_tensor(x, 0.5)
    assert q.tolist() == [1, -1, 2, -2, 3, 0, 127, -128]
    assert O.quantize_per_tensor(np.array([0.3], np.float32), 0.1, zero_point=5, dtype="uint8").tolist() == [8]
    assert O.quantize_per_tensor(np.array([-3.0], np.float32), 0.5, dtype="uint8").tolist() == [0]
    # largest float below 0.5 must not round up (a naive floor(x + 0.5) does)
    below = np.nextafter(np.float32(0.5), np.float32(0))
    assert O.quantize_per_tensor(np.array([below], np.float32), 1.0).tolist() == [0]
    np.testing.assert_allclose(O.dequantize_per_tensor(np.array([3, -2], np.int8), 0.5, 1), [1.0, -1.5])


def test_embedding_and_gather_vs_torch(fixtures):
    np.testing.assert_array_equal(O.embedding(fixtures["emb_w"], fixtures["emb_idx"]), fixtures["emb_y"])
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    idx = np.array([[0, 0, 2, 1], [2, 1, 0, 0]], np.int32)
    np.testing.assert_array_equal(O.gather(x, 0, idx[:, :4][:2]),
                                  torch.gather(torch.from_numpy(x), 0, torch.from_numpy(idx).long()).numpy())
    np.testing.assert_array_equal(O.index_select(x, 1, np.array([3, 0])), x[:, [3, 0]])


def test_mse_vs_torch(fixtures):
    a, b = fixtures["mse_a"], fixtures["mse_b"]
    np.testing.assert_allclose(O.mse_loss(a, b), fixtures["mse_loss"], rtol=1e-6)
    np.testing.assert_allclose(O.mse_loss_backward(np.ones(1, np.float32), a, b), fixtures["mse_grad"], rtol=1e-5,
                               atol=1e-8)


def test_reductions_closed_form():
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    assert O.sum_dim(x, 1).shape == (2, 4)
    assert O.sum_dim(x, 1, keepdim=True).shape == (2, 1, 4)
    np.testing.assert_array_equal(O.sum_dim(x, 0), x[0] + x[1])
    assert O.mean_all(x).tolist() == [11.5]
    assert O.sum_dim(np.array([1.0, 2.0], np.float32), 0).shape == (1,)


def test_mlp_step_vs_torch_autograd(fixtures):
    """Config 1: the oracle's forward/MSE/backward/SGD against torch autograd."""
    params = [(fixtures["mlp_w0"], fixtures["mlp_b0"]), (fixtures["mlp_w1"], fixtures["mlp_b1"])]
    loss, out, grads, new = M.mlp_train_step_np(params, fixtures["mlp_x"], fixtures["mlp_y"], lr=0.01)
    np.testing.assert_allclose(out, fixtures["mlp_out"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(loss, fixtures["mlp_loss"], rtol=1e-5)
    for i in range(2):
        np.testing.assert_allclose(grads[i][0], fixtures[f"mlp_gw{i}"], rtol=1e-4, atol=1e-7)
        np.testing.assert_allclose(grads[i][1], fixtures[f"mlp_gb{i}"], rtol=1e-4, atol=1e-7)
        np.testing.assert_allclose(new[i][0], fixtures[f"mlp_w{i}_after"], rtol=1e-6, atol=1e-8)
        np.testing.assert_allclose(new[i][1], fixtures[f"mlp_b{i}_after"], rtol=1e-6, atol=1e-8)


def _tiny_cfg():
    return dict(n_layer=2, n_head=4, n_embd=64, vocab_size=97, n_positions=32)


def _tiny_weights(cfg, seed=3):
    sys_path_pkg()
    from applegpu_runtime.models.gpt2 import random_weights
    return random_weights(cfg, seed=seed, std=0.2)


def sys_path_pkg():
    import os
    import sys
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "applegpu-runtime_amd")
    if pkg not in sys.path:
        sys.path.insert(0, pkg)


def test_gpt2_oracle_vs_transformers():
    """The numpy GPT-2 recipe against HuggingFace's GPT2LMHeadModel with the
    same weights (library routine; no network, random init)."""
    transformers = pytest.importorskip("transformers")
    cfg = _tiny_cfg()
    w = _tiny_weights(cfg)
    hc = transformers.GPT2Config(n_layer=cfg["n_layer"], n_head=cfg["n_head"], n_embd=cfg["n_embd"],
                                 vocab_size=cfg["vocab_size"], n_positions=cfg["n_positions"],
                                 activation_function="gelu_new", resid_pdrop=0, embd_pdrop=0, attn_pdrop=0,
                                 layer_norm_epsilon=1e-5)
    model = transformers.GPT2LMHeadModel(hc).eval()
    sd = model.state_dict()
    with torch.no_grad():
        for k, v in w.items():
            sd[k].copy_(torch.from_numpy(v))
        sd["lm_head.weight"].copy_(torch.from_numpy(w["transformer.wte.weight"]))
    ids = np.array([5, 17, 3, 96, 0, 42, 42, 8, 1, 77, 31], np.int64)
    with torch.no_grad():
        ref = model(torch.from_numpy(ids)[None]).logits[0].numpy()
    got, _ = M.gpt2_forward_np(w, cfg, ids)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def test_gpt2_kv_cache_matches_full_forward():
    """Incremental decode with the cache reproduces the full causal forward's last row."""
    cfg = _tiny_cfg()
    w = _tiny_weights(cfg)
    ids = np.array([5, 17, 3, 96, 0, 42], np.int64)
    full, _ = M.gpt2_forward_np(w, cfg, ids)
    _, cache = M.gpt2_forward_np(w, cfg, ids[:-1])
    inc, _ = M.gpt2_forward_np(w, cfg, ids, past=cache)
    np.testing.assert_allclose(inc[0], full[-1], rtol=1e-5, atol=1e-5)


def test_torch_cpu_gpt2_matches_oracle():
    from oracle.torch_cpu import TorchGPT2
    cfg = _tiny_cfg()
    w = _tiny_weights(cfg)
    ids = np.array([1, 2, 3, 4, 5, 6, 7], np.int64)
    np.testing.assert_allclose(TorchGPT2(w, cfg).forward(ids).numpy(), M.gpt2_forward_np(w, cfg, ids)[0],
                               rtol=1e-4, atol=1e-4)


def test_torch_cpu_kv_decoder_matches_full_recompute():
    """Batched prefill + KV-cache decode on the CPU (the C4 baseline) gives the
    logits of a full causal forward over prompt + generated tokens, per
    sequence, from the independent numpy oracle."""
    from oracle.torch_cpu import TorchGPT2Decoder
    cfg = _tiny_cfg()
    w = _tiny_weights(cfg)
    B, T, n = 3, 7, 4
    ids = np.random.default_rng(0).integers(0, cfg["vocab_size"], (B, T))
    dec = TorchGPT2Decoder(w, cfg)
    lg = dec.prefill(ids, T + n)
    steps = [lg[:, -1].numpy()]
    toks = [steps[0].argmax(-1)]
    for _ in range(n):
        steps.append(dec.decode(toks[-1]).numpy())
        toks.append(steps[-1].argmax(-1))
    toks = np.stack(toks, 1)
    for b in range(B):
        ref, _ = M.gpt2_forward_np(w, cfg, np.concatenate([ids[b], toks[b, :-1]]))
        np.testing.assert_allclose(np.stack([s[b] for s in steps]), ref[T - 1:], rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(lg[b].numpy(), ref[:T], rtol=1e-4, atol=1e-4)


def _torch_grads(fn, dy, *xs):
    ts = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in xs]
    fn(*ts).backward(torch.tensor(dy, dtype=torch.float64))
    return [t.grad.numpy() for t in ts]


def test_backward_ops_vs_torch_autograd():
    """The backward restatements against torch's autograd of the forward op
    in float64, at ragged and GPT-2 widths (a dropped term or wrong sign in
    any of them moves the result far past these bounds)."""
    rng = np.random.default_rng(44)
    for rows, cols in [(3, 7), (16, 768), (5, 2500)]:
        x = rng.standard_normal((rows, cols)).astype(np.float32) * 2 + 0.5
        g = rng.standard_normal(cols).astype(np.float32)
        b = rng.standard_normal(cols).astype(np.float32)
        dy = rng.standard_normal((rows, cols)).astype(np.float32)
        tx, tg, tb = _torch_grads(lambda a, w, c: F.layer_norm(a, (cols,), w, c, 1e-5), dy, x, g, b)
        dx, dg, db = O.layer_norm_backward(dy, x, g, 1e-5, params=True)
        np.testing.assert_allclose(dx, tx, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(dg, tg, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(db, tb, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(O.layer_norm_backward(dy, x, g), dx)
        (ts,) = _torch_grads(lambda a: torch.softmax(a, -1), dy, x)
        np.testing.assert_allclose(O.softmax_backward(dy, O.softmax(x)), ts, rtol=1e-4, atol=1e-6)
        for approx, fn in (("tanh", O.gelu_tanh_backward), ("none", O.gelu_erf_backward)):
            (tgl,) = _torch_grads(lambda a: F.gelu(a, approximate=approx), dy, x)
            np.testing.assert_allclose(fn(dy, x), tgl, rtol=1e-5, atol=1e-6)
    # embedding: repeated, unused and every-row indices
    w = rng.standard_normal((50, 24)).astype(np.float32)
    idx = np.concatenate([rng.integers(0, 50, 300), [7] * 40, [49, 0]]).astype(np.int64)
    dy = rng.standard_normal((idx.size, 24)).astype(np.float32)
    tw = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    F.embedding(torch.tensor(idx), tw).backward(torch.tensor(dy, dtype=torch.float64))
    np.testing.assert_allclose(O.embedding_backward(dy, idx, 50), tw.grad.numpy(), rtol=1e-5, atol=1e-5)
    assert (O.embedding_backward(dy, idx, 60)[50:] == 0).all()


def test_oracle_catches_planted_mistakes(fixtures):
    """The checks above fail on the typical slips (planted in copies, on the CPU)."""
    x = np.random.default_rng(0).standard_normal((4, 9)).astype(np.float32)
    # causal mask off by one (j < i instead of j <= i) breaks row 0
    rows = np.arange(9)
    wrong = np.where(np.arange(9)[None, :] < rows[:4, None] + 0, 1, 0)
    assert not np.array_equal(wrong[0], (np.arange(9) <= 0).astype(int))
    # a dropped 1/sqrt(d) scale changes attention
    q = k = v = x[None]
    s = O.matmul(q, np.swapaxes(k, -1, -2))
    unscaled = O.matmul(O.softmax(s), v)
    assert not np.allclose(unscaled, O.attention(q, k, v), atol=1e-3)
    # round-half-away instead of half-even changes the planted ties
    assert O.quantize_per_tensor(np.array([2.5], np.float32), 1.0).tolist() == [3]
    assert np.rint(np.float32(2.5)) == 2.0
    # dequantize slips: the zero point added instead of subtracted, or the
    # scale taken per column, differ from torch's per-tensor / per-channel
    # dequantized values
    fx = fixtures
    q8 = fx["dq_pt_i8_q"]
    wrong_zp = ((q8.astype(np.int32) + (-3)).astype(np.float32) * np.float32(0.1))
    assert not np.array_equal(wrong_zp, fx["dq_pt_i8_y"])
    qr, sr = fx["quant_q"], fx["quant_scale"]
    wrong_axis = qr.astype(np.float32) * np.resize(sr, qr.shape[1])[None, :]
    assert not np.array_equal(wrong_axis, fx["quant_deq"])
