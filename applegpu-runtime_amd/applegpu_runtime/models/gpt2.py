"""GPT-2 forward pass on the lazy op surface.

Follows the op recipe of the reference's `gpt2_forward`
(python/applegpu_runtime/models/gpt2.py:47-180): token + position embedding,
per layer layer_norm -> x @ c_attn (HF Conv1D layout [in, out]) + bias ->
split Q/K/V -> heads [n_head, seq, d_head] -> causal attention -> merge heads
-> c_proj + bias -> residual -> layer_norm -> c_fc + bias -> gelu (tanh) ->
c_proj + bias -> residual; final layer_norm; logits = x @ wte^T (tied head).

On this backend the graph evaluates with: one GEMM per projection with the
bias, gelu and residual add fused into its epilogue; Q/K/V read in place from
the fused QKV projection (slices, reshapes and the head transpose are views);
one fused attention kernel per layer whose output is stored head-interleaved
so the merge transpose is free; the LM head reads wte as a transposed operand
(no 154 MB transpose per forward).

`random_weights` makes the synthetic GPT-2 of the benchmark configs: every
matrix and embedding N(0, 0.02), biases 0, layer-norm gamma 1 / beta 0, from a
seeded numpy generator (the reference's `load_gpt2_weights` downloads
pretrained weights, which this environment cannot).
"""
from __future__ import annotations

import numpy as np

import applegpu_runtime as gpu

GPT2_CONFIGS = {
    "gpt2": dict(n_layer=12, n_head=12, n_embd=768, vocab_size=50257, n_positions=1024),
    "gpt2-medium": dict(n_layer=24, n_head=16, n_embd=1024, vocab_size=50257, n_positions=1024),
    "gpt2-large": dict(n_layer=36, n_head=20, n_embd=1280, vocab_size=50257, n_positions=1024),
}


def weight_shapes(cfg: dict) -> dict:
    """HF GPT2LMHeadModel parameter names and shapes (Conv1D weights are [in, out])."""
    d, V, P = cfg["n_embd"], cfg["vocab_size"], cfg["n_positions"]
    shapes = {"transformer.wte.weight": (V, d), "transformer.wpe.weight": (P, d),
              "transformer.ln_f.weight": (d,), "transformer.ln_f.bias": (d,)}
    for i in range(cfg["n_layer"]):
        p = f"transformer.h.{i}"
        shapes.update({
            f"{p}.ln_1.weight": (d,), f"{p}.ln_1.bias": (d,),
            f"{p}.attn.c_attn.weight": (d, 3 * d), f"{p}.attn.c_attn.bias": (3 * d,),
            f"{p}.attn.c_proj.weight": (d, d), f"{p}.attn.c_proj.bias": (d,),
            f"{p}.ln_2.weight": (d,), f"{p}.ln_2.bias": (d,),
            f"{p}.mlp.c_fc.weight": (d, 4 * d), f"{p}.mlp.c_fc.bias": (4 * d,),
            f"{p}.mlp.c_proj.weight": (4 * d, d), f"{p}.mlp.c_proj.bias": (d,),
        })
    return shapes


def random_weights(cfg: dict, seed: int = 42, std: float = 0.02) -> dict:
    """numpy float32 weights: matrices/embeddings N(0, std), biases 0, LN gamma 1 / beta 0."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shp in weight_shapes(cfg).items():
        if name.endswith(".bias"):
            out[name] = np.zeros(shp, np.float32)
        elif ".ln_" in name:
            out[name] = np.ones(shp, np.float32)
        else:
            out[name] = (rng.standard_normal(shp, dtype=np.float32) * np.float32(std)).astype(np.float32)
    return out


def load_model(np_weights: dict, cfg: dict, dtype: str = "float32") -> dict:
    """Upload numpy weights; returns the model dict the forward pass takes."""
    gpu.init_backend()
    w = {}
    for k, v in np_weights.items():
        t = gpu.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
        if dtype != "float32":
            t = gpu.cast(t, dtype)
            t.eval()
        w[k] = t
    return {"weights": w, "config": dict(cfg), "dtype": dtype}


def gpt2_forward(model: dict, input_ids, kv_cache=None, positions=None):
    """Returns (logits [seq, vocab], new_kv_cache) for one sequence.

    input_ids: list/array of token ids, or an int32 GpuTensor [T] already on
    the device (then `positions`, an int32 GpuTensor [T], may be given too;
    both device-resident inputs let the forward run under `gpu.capture`).
    With kv_cache (list of (k, v) per layer, each [n_head, past, d_head]) only
    the last token is processed.
    """
    w = model["weights"]
    cfg = model["config"]
    L, H, d = cfg["n_layer"], cfg["n_head"], cfg["n_embd"]
    hd = d // H
    cached = kv_cache is not None
    if isinstance(input_ids, gpu.GpuTensor):
        if cached:
            raise ValueError("gpt2_forward: device-resident ids take no kv_cache")
        idx = input_ids
        T = idx.shape[0]
        pos = positions if positions is not None else gpu.from_numpy(np.arange(T, dtype=np.int32))
    else:
        ids = list(np.asarray(input_ids).reshape(-1))
        toks = ids[-1:] if cached else ids
        start = len(ids) - 1 if cached else 0
        T = len(toks)
        idx = gpu.from_numpy(np.asarray(toks, dtype=np.int32))
        pos = gpu.from_numpy(np.arange(start, start + T, dtype=np.int32))
    x = gpu.embedding(w["transformer.wte.weight"], idx) + gpu.embedding(w["transformer.wpe.weight"], pos)

    new_cache = []
    for i in range(L):
        p = f"transformer.h.{i}"
        h = gpu.layer_norm(x, w[f"{p}.ln_1.weight"], w[f"{p}.ln_1.bias"])
        qkv = gpu.add_bias(h @ w[f"{p}.attn.c_attn.weight"], w[f"{p}.attn.c_attn.bias"])

        def heads(lo):
            part = gpu.slice(qkv, 1, lo, lo + d)
            return gpu.transpose_dims(gpu.reshape(part, [T, H, hd]), 0, 1)

        q, k, v = heads(0), heads(d), heads(2 * d)
        if cached:
            pk, pv = kv_cache[i]
            k = gpu.concat(pk, k, 1)
            v = gpu.concat(pv, v, 1)
        new_cache.append((k, v))
        a = gpu.attention(q, k, v) if cached else gpu.attention_causal(q, k, v)
        a = gpu.reshape(gpu.transpose_dims(a, 0, 1), [T, d])
        x = x + gpu.add_bias(a @ w[f"{p}.attn.c_proj.weight"], w[f"{p}.attn.c_proj.bias"])

        h = gpu.layer_norm(x, w[f"{p}.ln_2.weight"], w[f"{p}.ln_2.bias"])
        f = gpu.gelu(gpu.add_bias(h @ w[f"{p}.mlp.c_fc.weight"], w[f"{p}.mlp.c_fc.bias"]))
        x = x + gpu.add_bias(f @ w[f"{p}.mlp.c_proj.weight"], w[f"{p}.mlp.c_proj.bias"])

    x = gpu.layer_norm(x, w["transformer.ln_f.weight"], w["transformer.ln_f.bias"])
    logits = x @ gpu.transpose(w["transformer.wte.weight"])
    return logits, new_cache
