"""Parity of exactly what bench.py times, at full size, against the oracle.

- C2: the captured GPT-2-small forward (12 x 768, vocab 50257, seq 128,
  device-resident ids and positions, need_cache=False: the fused
  qkv_attention path, layer_norm computed in the split-K reductions, the
  fused embedding + ln_1 launch), replayed as a HIP graph.
- C3: the captured MLP 4096-4096-4096-1 train step, replayed twice, each
  replay teacher-forced against the oracle's backward + SGD.
- C4 model wiring at full GPT-2-large dimensions (36 x 1280, 20 heads,
  vocab 50257, fp16): prefill + greedy decode over the KV cache with the
  decode step graph-replayed, teacher-forced against the oracle.

The recipe the forward follows is the reference's gpt2_forward
(python/applegpu_runtime/models/gpt2.py:84-178); the train step is the
reference's MLP benchmark step (benchmarks/bench_mlp_cpp.py:29-52).
"""
import numpy as np
import pytest

from conftest import rel_err
from oracle import models as M

pytestmark = pytest.mark.gpu

GPT2_SMALL = dict(n_layer=12, n_head=12, n_embd=768, vocab_size=50257, n_positions=1024)
GPT2_LARGE = dict(n_layer=36, n_head=20, n_embd=1280, vocab_size=50257, n_positions=1024)


def test_captured_c2_forward_full_size_vs_oracle(gpu):
    """The C2 graph with unpacked fp32 weights (the tiled split-K GEMMs and
    qkv_attention): every replay at the fp32 matmul/attention bar (1e-3
    normwise, checked at 1e-4), replays bitwise identical to each other with
    eager work between them, greedy picks equal to the oracle's."""
    from applegpu_runtime.models import gpt2 as G
    print("C2 captured forward: 12x768, seq 128, unpacked weights", flush=True)
    wnp = G.random_weights(GPT2_SMALL, seed=42)
    model = G.load_model(wnp, GPT2_SMALL, x3=False)
    ids = np.random.default_rng(42).integers(0, GPT2_SMALL["vocab_size"], 128).astype(np.int32)
    _check_c2_graph(gpu, G, model, wnp, ids)


def test_captured_c2_forward_packed_weights_vs_oracle(gpu):
    """bench.py's C2 graph: the fp32 projection weights packed as bf16 hi/lo
    fragments (load_model's default), activations passed as packed rows
    written by the embedding, the layer_norm reductions and the fc epilogue,
    the packed-A row panels and split GEMMs."""
    from applegpu_runtime.models import gpt2 as G
    print("C2 captured forward, packed fp32 weights and rows", flush=True)
    wnp = G.random_weights(GPT2_SMALL, seed=42)
    model = G.load_model(wnp, GPT2_SMALL)
    assert model["x3"]
    ids = np.random.default_rng(42).integers(0, GPT2_SMALL["vocab_size"], 128).astype(np.int32)
    _check_c2_graph(gpu, G, model, wnp, ids)


def _check_c2_graph(gpu, G, model, wnp, ids):
    idx = gpu.from_numpy(ids)
    pos = gpu.from_numpy(np.arange(128, dtype=np.int32))
    graph = gpu.capture(lambda: G.gpt2_forward(model, idx, positions=pos, need_cache=False)[0])
    try:
        ref, _ = M.gpt2_forward_np(wnp, GPT2_SMALL, ids)
        outs = []
        for r in range(3):
            graph.replay()
            got = graph.outputs.to_numpy()
            assert got.shape == (128, GPT2_SMALL["vocab_size"])
            err = rel_err(got, ref)
            assert err < 1e-4, (r, err)
            outs.append(got)
            # eager work on the same stream between replays
            t = gpu.from_numpy(np.ones(1000, np.float32))
            (t + t).to_numpy()
        np.testing.assert_array_equal(outs[0], outs[1])
        np.testing.assert_array_equal(outs[0], outs[2])
        # greedy picks: equal wherever the oracle's top two are apart by more
        # than the tolerance
        top2 = np.sort(ref, axis=-1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 1e-4 * np.abs(ref).max()
        np.testing.assert_array_equal(outs[0].argmax(-1)[clear], ref.argmax(-1)[clear])
        # the uncaptured path with the same options gives the same logits
        eager = G.gpt2_forward(model, idx, positions=pos, need_cache=False)[0].to_numpy()
        np.testing.assert_array_equal(eager, outs[0])
    finally:
        graph.destroy()


def _teacher_forced_step(params, acts_gpu, y, lr):
    """The oracle's backward + SGD (float64) on the GPU's own forward
    activations; a pre-activation within rounding distance of zero may fall
    on either side of ReLU in two correct implementations, so the masks are
    taken from the device's activations."""
    acts = [a.astype(np.float64) for a in acts_gpu]
    out = acts[-1]
    g = 2.0 * (out - y.astype(np.float64)) / out.size
    new = [None] * len(params)
    for i in range(len(params) - 1, -1, -1):
        w, b = params[i]
        new[i] = (w.astype(np.float64) - lr * (g.T @ acts[i]), b.astype(np.float64) - lr * g.sum(0))
        if i > 0:
            g = (g @ w.astype(np.float64)) * (acts[i] > 0)
    return new


def test_captured_c3_step_replays_vs_oracle(gpu):
    """bench.py's C3 graph, replayed twice: each replay's loss against the
    oracle's forward, its parameter update against the oracle's backward +
    SGD on that step's activations (which the same forward kernels give
    eagerly, bit for bit), at the fp32 GEMM bar."""
    from applegpu_runtime import eager as E
    from applegpu_runtime.models.mlp import EagerMLP, torch_default_init
    print("C3 captured train step: 4096-4096-4096-1, batch 256", flush=True)
    params = torch_default_init([4096, 4096, 4096, 1], seed=42)
    rng = np.random.default_rng(42)
    x = rng.standard_normal((256, 4096), dtype=np.float32)
    y = rng.standard_normal((256, 1), dtype=np.float32)
    mlp = EagerMLP(params)
    tx, ty = E.from_numpy(x), E.from_numpy(y)
    graph = gpu.capture(lambda: mlp.train_step(tx, ty, lr=0.01))
    try:
        cur = mlp.numpy_params()
        # the capture records the step without running it
        for (w, b), (w0, b0) in zip(cur, params):
            np.testing.assert_array_equal(w, w0)
            np.testing.assert_array_equal(b, b0)
        for r in range(2):
            out, acts = mlp.forward(tx)
            acts_np = [a.numpy() for a in acts]
            loss_ref, out_ref, _, _ = M.mlp_train_step_np(cur, x, y, lr=0.01)
            assert rel_err(acts_np[-1], out_ref) < 1e-4, r
            graph.replay()
            loss = float(graph.outputs.numpy()[0])
            assert abs(loss - float(loss_ref[0])) <= 1e-4 * abs(float(loss_ref[0])), (r, loss, loss_ref)
            new_ref = _teacher_forced_step(cur, acts_np, y, 0.01)
            new = mlp.numpy_params()
            for li, ((w, b), (w0, b0), (wr, br)) in enumerate(zip(new, cur, new_ref)):
                assert rel_err(w - w0, wr - w0) < 1e-3, (r, li)
                assert rel_err(b - b0, br - b0) < 1e-3, (r, li)
                assert rel_err(w, wr) < 1e-5, (r, li)
            cur = new
    finally:
        graph.destroy()


def test_gpt2_large_full_dims_generation_teacher_forced(gpu):
    """GPT-2 large at full depth, width and vocabulary, fp16: batch 2, a
    16-token prompt, 4 greedy steps (decode step graph-replayed).  Each
    step's logits against the oracle's forward over prompt + the device's own
    tokens on the fp16-rounded weights, at the fp16 bar (1e-2)."""
    from applegpu_runtime.models import gpt2 as G
    print("GPT-2 large generation: 36x1280, vocab 50257, fp16, B=2, T=16, 4 steps", flush=True)
    w = G.random_weights(GPT2_LARGE, seed=42)
    model = G.load_model(w, GPT2_LARGE, dtype="float16")
    for k in w:
        w[k] = w[k].astype(np.float16).astype(np.float32)
    B, T, n = 2, 16, 4
    prompt = np.random.default_rng(43).integers(0, GPT2_LARGE["vocab_size"], (B, T)).astype(np.int32)
    toks, logits = G.generate_greedy(model, prompt, n, capture=True, keep_logits=True)
    assert toks.shape == (B, n + 1)
    np.testing.assert_array_equal(toks, logits.argmax(-1).T)
    tol = 1e-2
    for b in range(B):
        seq = np.concatenate([prompt[b], toks[b, :-1]])
        ref, _ = M.gpt2_forward_np(w, GPT2_LARGE, seq)
        ref_steps = ref[T - 1:T + n]
        got = logits[:, b].astype(np.float32)
        err = rel_err(got, ref_steps)
        print(f"  sequence {b}: rel err {err:.2e}", flush=True)
        assert err < tol, b
        for s in range(n + 1):
            top2 = np.sort(ref_steps[s])[-2:]
            if top2[1] - top2[0] > tol * np.abs(ref_steps[s]).max():
                assert toks[b, s] == int(np.argmax(ref_steps[s])), (b, s)
