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


def _perturb_norms_and_biases(w, seed=7):
    """Non-identity layer norms and nonzero biases (gamma = 1 + N(0, 0.1),
    beta and every bias N(0, 0.02)), so that the folds of ln_1 / ln_2 into the
    GEMMs (gamma into the weights, beta @ W into the bias, column sums) are
    exercised with every term nonzero."""
    rng = np.random.default_rng(seed)
    for k, v in w.items():
        if ".ln_" in k or k.startswith("transformer.ln_f"):
            if k.endswith(".weight"):
                w[k] = (1.0 + 0.1 * rng.standard_normal(v.shape)).astype(np.float32)
            else:
                w[k] = (0.02 * rng.standard_normal(v.shape)).astype(np.float32)
        elif k.endswith(".bias"):
            w[k] = (0.02 * rng.standard_normal(v.shape)).astype(np.float32)
    return w


def test_captured_c2_forward_full_size_vs_oracle(gpu):
    """The C2 graph with unpacked fp32 weights (the tiled split-K GEMMs and
    qkv_attention): every replay at the fp32 matmul/attention bar (1e-3
    normwise, checked at 1e-4), replays bitwise identical to each other with
    eager work between them, greedy picks equal to the oracle's."""
    from applegpu_runtime.models import gpt2 as G
    print("C2 captured forward: 12x768, seq 128, unpacked weights, perturbed norms and biases", flush=True)
    wnp = _perturb_norms_and_biases(G.random_weights(GPT2_SMALL, seed=42))
    model = G.load_model(wnp, GPT2_SMALL, x3=False)
    ids = np.random.default_rng(42).integers(0, GPT2_SMALL["vocab_size"], 128).astype(np.int32)
    _check_c2_graph(gpu, G, model, wnp, ids)


def test_captured_c2_forward_packed_weights_vs_oracle(gpu):
    """bench.py's C2 graph: the fp32 projection weights packed as bf16 hi/lo
    fragments (load_model's default), activations passed as packed rows
    written by the embedding, the layer_norm reductions and the fc epilogue,
    the packed-A row panels and split GEMMs, ln_2 folded into c_fc; layer
    norms and biases perturbed away from identity and zero."""
    from applegpu_runtime.models import gpt2 as G
    print("C2 captured forward, packed fp32 weights and rows, perturbed norms and biases", flush=True)
    wnp = _perturb_norms_and_biases(G.random_weights(GPT2_SMALL, seed=42))
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


def test_c4_generation_full_size_captured_vs_eager_and_teacher_forced(gpu):
    """Config C4 exactly as bench.py times it (models.gpt2.Generation):
    GPT-2 large fp16, 8 prompts of 512 random ids, the prefill and the decode
    step captured as HIP graphs, 128 greedy steps over the preallocated cache
    (contexts 513..640).  The captured generation's tokens and logits equal an
    op-by-op run of the same calls bit for bit; for two sequences every pick's
    logits (the prompt's last position, then decode steps 0..127) are checked,
    teacher-forced, against the reference's CPU path (torch CPU eager fp32 on
    the fp16-rounded weights, oracle/torch_cpu.py, itself pinned against the
    numpy oracle) at the fp16 bar (1e-2)."""
    import torch
    from applegpu_runtime.models import gpt2 as G
    from oracle.torch_cpu import TorchGPT2
    B, T, n = 8, 512, 128
    print(f"C4 full size: GPT-2 large fp16, B={B}, T={T}, {n} captured decode steps", flush=True)
    w = G.random_weights(GPT2_LARGE, seed=42)
    model = G.load_model(w, GPT2_LARGE, dtype="float16")
    ids = np.random.default_rng(42).integers(0, GPT2_LARGE["vocab_size"], (B, T)).astype(np.int32)
    gen = G.Generation(model, ids, n, capture=True)
    try:
        toks, logits = gen.run(keep_logits=True)
    finally:
        gen.destroy()
    del gen
    print("  captured generation done", flush=True)
    gen_e = G.Generation(model, ids, n, capture=False)
    toks_e, logits_e = gen_e.run(keep_logits=True)
    del gen_e, model
    print("  op-by-op generation done", flush=True)
    assert toks.shape == (B, n + 1) and logits.shape == (n + 1, B, GPT2_LARGE["vocab_size"])
    np.testing.assert_array_equal(toks, toks_e)
    np.testing.assert_array_equal(logits, logits_e)
    # every pick is the first maximum of its own logits
    np.testing.assert_array_equal(toks, logits.astype(np.float32).argmax(-1).T)

    for k in list(w):
        w[k] = w[k].astype(np.float16).astype(np.float32)
    ref_model = TorchGPT2(w, GPT2_LARGE)
    tol = 1e-2
    with torch.no_grad():
        for b in (0, 5):
            seq = np.concatenate([ids[b], toks[b, :-1]])            # 640 ids
            ref = ref_model.forward(seq).numpy()[T - 1:T + n]     # the 129 picks' positions
            got = logits[:, b].astype(np.float32)
            errs = [rel_err(got[s], ref[s]) for s in range(n + 1)]
            print(f"  sequence {b}: rel err prompt-last {errs[0]:.2e}, step 0 {errs[1]:.2e}, "
                  f"step 63 {errs[64]:.2e}, step 127 {errs[128]:.2e}, max {max(errs):.2e}", flush=True)
            for s in (0, 1, 64, 128):
                assert errs[s] < tol, (b, s, errs[s])
            assert max(errs) < tol, (b, int(np.argmax(errs)), max(errs))
            for s in range(n + 1):
                top2 = np.sort(ref[s])[-2:]
                if top2[1] - top2[0] > tol * np.abs(ref[s]).max():
                    assert toks[b, s] == int(np.argmax(ref[s])), (b, s)
