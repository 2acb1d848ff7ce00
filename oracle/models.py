"""Model-level oracles (test infrastructure only).

`gpt2_forward_np` restates the reference's GPT-2 op recipe
(python/applegpu_runtime/models/gpt2.py:47-180) with the numpy ops of
oracle/ops.py; `mlp_train_step_np` restates one training step of the
reference's MLP benchmark (benchmarks/bench_mlp_cpp.py:29-52: forward, MSE,
backward, SGD lr) as the autograd of nn.Linear/ReLU/MSELoss computes it.
"""
from __future__ import annotations

import numpy as np

from . import ops as O


def gpt2_forward_np(weights: dict, cfg: dict, ids, past=None):
    """logits [T, vocab] (and per-layer K/V [H, T, hd]) for one sequence.

    With `past` (list of (k, v) per layer) only the last token is processed and
    the attention is non-causal over the cache (gpt2.py:118-135)."""
    L, H, d = cfg["n_layer"], cfg["n_head"], cfg["n_embd"]
    hd = d // H
    ids = np.asarray(ids).reshape(-1)
    toks = ids[-1:] if past is not None else ids
    start = len(ids) - 1 if past is not None else 0
    T = len(toks)
    w = weights
    x = O.embedding(w["transformer.wte.weight"], toks) + O.embedding(w["transformer.wpe.weight"],
                                                                      np.arange(start, start + T))
    cache = []
    for i in range(L):
        p = f"transformer.h.{i}"
        h = O.layer_norm(x, w[f"{p}.ln_1.weight"], w[f"{p}.ln_1.bias"])
        qkv = O.add_bias(O.matmul(h, w[f"{p}.attn.c_attn.weight"]), w[f"{p}.attn.c_attn.bias"])
        q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(T, H, hd).transpose(1, 0, 2) for j in range(3))
        if past is not None:
            k = np.concatenate([past[i][0], k], axis=1)
            v = np.concatenate([past[i][1], v], axis=1)
        cache.append((k, v))
        a = O.attention(q, k, v, causal=past is None)
        a = a.transpose(1, 0, 2).reshape(T, d)
        x = x + O.add_bias(O.matmul(a, w[f"{p}.attn.c_proj.weight"]), w[f"{p}.attn.c_proj.bias"])
        h = O.layer_norm(x, w[f"{p}.ln_2.weight"], w[f"{p}.ln_2.bias"])
        f = O.gelu_tanh(O.add_bias(O.matmul(h, w[f"{p}.mlp.c_fc.weight"]), w[f"{p}.mlp.c_fc.bias"]))
        x = x + O.add_bias(O.matmul(f, w[f"{p}.mlp.c_proj.weight"]), w[f"{p}.mlp.c_proj.bias"])
    x = O.layer_norm(x, w["transformer.ln_f.weight"], w["transformer.ln_f.bias"])
    logits = O.matmul(x, w["transformer.wte.weight"].T)
    return logits, cache


def mlp_train_step_np(params, x, y, lr=0.01):
    """One step of Linear->ReLU->...->Linear, MSE(mean), SGD(lr).

    params: list of (W [out,in], b [out]) float32.  Returns
    (loss, out, grads, new_params).  x does not require grad (no dX for the
    first layer)."""
    acts = [x.astype(np.float32)]
    h = acts[0]
    n = len(params)
    for i, (w, b) in enumerate(params):
        h = O.linear(h, w, b)
        if i < n - 1:
            h = O.relu(h)
        acts.append(h)
    out = h
    loss = O.mse_loss(out, y)
    g = O.mse_loss_backward(np.ones(1, np.float32), out, y)
    grads = [None] * n
    for i in range(n - 1, -1, -1):
        w, _ = params[i]
        dw = O.matmul(g.T, acts[i])
        db = O.sum_dim(g, 0)
        grads[i] = (dw, db)
        if i > 0:
            g = O.threshold_backward(O.matmul(g, w), acts[i], 0.0)
    new = [((w - np.float32(lr) * dw).astype(np.float32), (b - np.float32(lr) * db).astype(np.float32))
           for (w, b), (dw, db) in zip(params, grads)]
    return loss, out, grads, new
