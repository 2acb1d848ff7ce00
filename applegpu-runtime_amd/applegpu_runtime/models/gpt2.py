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


CONV1D = (".attn.c_attn.weight", ".attn.c_proj.weight", ".mlp.c_fc.weight", ".mlp.c_proj.weight")


def load_model(np_weights: dict, cfg: dict, dtype: str = "float32", kmajor=None, packed=None, x3=None) -> dict:
    """Upload numpy weights; returns the model dict the forward pass takes.

    kmajor (default: on for fp16/bf16) stores the Conv1D projection weights
    transposed, [out, in], contiguous along the reduction: the layout the
    decode-step GEMM streams with one 16-byte load per MFMA operand.  The
    forward multiplies by a transposed view of them, so the arithmetic is
    the recipe's x @ W either way.  packed (default: on with kmajor) also
    keeps every projection and the tied LM head in the skinny GEMM's packed
    layout (gpu.pack_weight) for calls with at most 16 token rows: one more
    copy of the weights (HBM is plentiful), read with contiguous 1 KB wave
    loads during decode.  x3 (default: on for fp32 [in, out] weights with
    n_embd a multiple of 16) keeps every fp32 projection weight split once
    into bf16 hi/lo MFMA fragments (gpu.pack_weight_x3), which the fp32 GEMMs
    of the forward read instead of splitting the weights on every call; the
    forward then also passes the activations after each layer_norm and gelu
    as packed rows (gpu.pack_rows_x3), written by their producers."""
    gpu.init_backend()
    if kmajor is None:
        kmajor = dtype != "float32"
    if packed is None:
        packed = kmajor
    if packed and (dtype == "float32" or not kmajor):
        raise ValueError("packed decode weights need fp16/bf16 k-major weights")
    if x3 is None:
        x3 = dtype == "float32" and not kmajor and cfg["n_embd"] % 16 == 0
    if x3 and (dtype != "float32" or kmajor or cfg["n_embd"] % 16 != 0):
        raise ValueError("fp32-packed weights need fp32 [in, out] weights with n_embd a multiple of 16")
    w = {}
    for k, v in np_weights.items():
        a = np.asarray(v, dtype=np.float32)
        if kmajor and k.endswith(CONV1D):
            a = a.T
        t = gpu.from_numpy(np.ascontiguousarray(a))
        if dtype != "float32":
            t = gpu.cast(t, dtype)
            t.eval()
        w[k] = t
    pk = {}
    if packed:
        for k, t in w.items():
            if k.endswith(CONV1D) or k == "transformer.wte.weight":
                p = gpu.pack_weight(t)
                p.eval()
                pk[k] = (p, t.shape[0], "rows16")
    fold, fold1 = {}, {}
    if x3:
        for k, t in w.items():
            if k.endswith(CONV1D):
                p = gpu.pack_weight_x3(t)
                p.eval()
                pk[k] = (p, t.shape[1], "x3")
        # the tied LM head as B = wte^T, for the vocabulary-head GEMM
        wte = w["transformer.wte.weight"]
        p = gpu.pack_weight_x3(gpu.transpose(wte))
        p.eval()
        pk["transformer.wte.weight"] = (p, wte.shape[0], "x3")
        if cfg["n_embd"] in _FOLD_WIDTHS:
            for i in range(cfg["n_layer"]):
                fold[i] = _fold_ln(np_weights, f"transformer.h.{i}", "ln_2", "mlp.c_fc")
            # ln_1 of layers after the first: the previous layer's MLP c_proj
            # writes x with its packed rows and row statistics when its plan
            # finishes its output in one launch (a row panel, split or not)
            d = cfg["n_embd"]
            if gpu.x3_rows_out_ok(_ROWS_HINT, d, 4 * d):
                for i in range(1, cfg["n_layer"]):
                    fold1[i] = _fold_ln(np_weights, f"transformer.h.{i}", "ln_1", "attn.c_attn")
    return {"weights": w, "config": dict(cfg), "dtype": dtype, "kmajor": bool(kmajor), "packed": pk,
            "x3": bool(x3), "fold_ln2": fold, "fold_ln1": fold1}


# Widths whose c_proj and c_fc run unsplit packed-row panel GEMMs (K a
# multiple of 256 up to 1536), the condition for folding ln_2 into c_fc (and
# ln_1 into c_attn).
_FOLD_WIDTHS = (256, 512, 768, 1024, 1280, 1536)
# The row count the ln_1 fold is planned for (C2's sequence length): the
# MLP c_proj of that many rows must write its output, packed rows and row
# statistics in one launch.
_ROWS_HINT = 128


def _fold_ln(np_weights: dict, p: str, ln: str, proj: str):
    """A layer_norm folded into the projection that reads it (ln_2 into c_fc,
    ln_1 into c_attn): layer_norm(x, g, b) @ W + c = inv * (x @ (g W) -
    mean * colsum(g W)) + (b @ W + c) per row, so that the projection can
    read the residual stream x itself (as packed rows with the row
    statistics the producing GEMM writes) instead of a normalised copy.  g W
    is rounded to fp32 once, and colsum is taken over those fp32 values so
    that the mean term cancels against the product of the same weights."""
    g = np.asarray(np_weights[f"{p}.{ln}.weight"], np.float64)
    b = np.asarray(np_weights[f"{p}.{ln}.bias"], np.float64)
    W = np.asarray(np_weights[f"{p}.{proj}.weight"], np.float64)
    c = np.asarray(np_weights[f"{p}.{proj}.bias"], np.float64)
    gw = (g[:, None] * W).astype(np.float32)
    cs = gw.astype(np.float64).sum(0).astype(np.float32)
    bb = (b @ W + c).astype(np.float32)
    packed = gpu.pack_weight_x3(gpu.from_numpy(gw))
    cs_t, bb_t = gpu.from_numpy(cs), gpu.from_numpy(bb)
    for t in (packed, cs_t, bb_t):
        t.eval()
    return packed, cs_t, bb_t, W.shape[1]


def _mm(model: dict, x, name: str, rows: int = None):
    """x @ W for a Conv1D weight (HF layout [in, out]) or x @ wte^T, whichever
    way the weight is stored; fp32 weights use their hi/lo packed copy, and
    16-bit ones their decode-packed copy for calls with at most 16 rows."""
    pk = model.get("packed", {}).get(name)
    if pk is not None and (pk[2] == "x3" or (rows is not None and rows <= 16)):
        return gpu.matmul_packed(x, pk[0], pk[1])
    w = model["weights"][name]
    if name == "transformer.wte.weight":
        return x @ gpu.transpose(w)
    return x @ (gpu.transpose(w) if model.get("kmajor") else w)


def _mm_rows(model: dict, x, name: str, rows: int):
    """x @ W for an fp32 packed-weight model with x split into MFMA row
    fragments first (gpu.pack_rows_x3): inside the lazy graph, x's producer
    (the fused embedding or a split-K reduction computing layer_norm, or the
    GEMM epilogue computing gelu) writes the fragments itself, so the product
    reads both operands without conversion."""
    pk = model["packed"][name]
    return gpu.matmul_pp(gpu.pack_rows_x3(x), rows, pk[0], pk[1])


def gpt2_forward(model: dict, input_ids, kv_cache=None, positions=None, need_cache=True):
    """Returns (logits [seq, vocab], new_kv_cache) for one sequence.

    input_ids: list/array of token ids, or an int32 GpuTensor [T] already on
    the device (then `positions`, an int32 GpuTensor [T], may be given too;
    both device-resident inputs let the forward run under `gpu.capture`).
    With kv_cache (list of (k, v) per layer, each [n_head, past, d_head]) only
    the last token is processed.  need_cache=False (a full forward whose K/V
    are not kept; new_kv_cache is then None) lets each layer run its QKV
    projection and attention as one `qkv_attention` op.
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

    # fp32 packed-weight models: every projection takes its activations as
    # packed rows, written by their producer (the embedding or a split-K
    # reduction computing layer_norm, the attention kernel, a GEMM epilogue)
    rows = model.get("x3", False)
    mm_in = (lambda t, name: _mm_rows(model, t, name, T)) if rows else (lambda t, name: _mm(model, t, name))
    new_cache = []
    for i in range(L):
        p = f"transformer.h.{i}"
        fold1 = model.get("fold_ln1", {}).get(i) if rows else None
        h = None if fold1 is not None else gpu.layer_norm(x, w[f"{p}.ln_1.weight"], w[f"{p}.ln_1.bias"])
        if not cached and not need_cache and not model.get("kmajor") and not model.get("x3"):
            # projection + head split + causal attention in one op
            a = gpu.qkv_attention(h, w[f"{p}.attn.c_attn.weight"], w[f"{p}.attn.c_attn.bias"], H, causal=True)
        else:
            if fold1 is not None:
                # ln_1 folded into c_attn: the previous layer's MLP c_proj
                # wrote x as packed rows with row statistics
                packed1, cs1, bb1, n_qkv = fold1
                qkv = gpu.add_bias(gpu.matmul_pp_norm(gpu.pack_rows_x3(x), gpu.row_stats_x3(x), T, packed1, cs1,
                                                      n_qkv), bb1)
            else:
                qkv = gpu.add_bias(mm_in(h, f"{p}.attn.c_attn.weight"), w[f"{p}.attn.c_attn.bias"])

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
        x = x + gpu.add_bias(mm_in(a, f"{p}.attn.c_proj.weight"), w[f"{p}.attn.c_proj.bias"])

        fold = model.get("fold_ln2", {}).get(i)
        if fold is not None:
            # ln_2 folded into c_fc: the proj GEMM writes x as packed rows and
            # row statistics besides fp32, c_fc normalises in its epilogue
            packed, cs, bb, n_fc = fold
            h = gpu.matmul_pp_norm(gpu.pack_rows_x3(x), gpu.row_stats_x3(x), T, packed, cs, n_fc)
            f = gpu.gelu(gpu.add_bias(h, bb))
        else:
            h = gpu.layer_norm(x, w[f"{p}.ln_2.weight"], w[f"{p}.ln_2.bias"])
            f = gpu.gelu(gpu.add_bias(mm_in(h, f"{p}.mlp.c_fc.weight"), w[f"{p}.mlp.c_fc.bias"]))
        x = x + gpu.add_bias(mm_in(f, f"{p}.mlp.c_proj.weight"), w[f"{p}.mlp.c_proj.bias"])

    x = gpu.layer_norm(x, w["transformer.ln_f.weight"], w["transformer.ln_f.bias"])
    if rows:
        logits = mm_in(x, "transformer.wte.weight")
    else:
        logits = x @ gpu.transpose(w["transformer.wte.weight"])
    return logits, (new_cache if need_cache or cached else None)


# ── batched prefill + greedy decode over a preallocated KV cache ────────────
class KVCache:
    """Per-layer K and V caches, [batch, n_head, max_len, d_head] each, plus
    `pos`, an int32 device tensor [batch] holding the rows filled so far.

    The reference grows its cache by concatenation every step
    (python/applegpu_runtime/models/gpt2.py:122-126); here the cache is
    allocated once and written in place (`gpu.kv_write`), and every length
    the decode step needs lives in device memory, so one decode step can be
    captured as a HIP graph and replayed for every generated token."""

    def __init__(self, cfg: dict, batch: int, max_len: int, dtype: str = "float16"):
        gpu.init_backend()
        H, d = cfg["n_head"], cfg["n_embd"]
        if max_len > cfg["n_positions"]:
            raise ValueError(f"max_len {max_len} exceeds n_positions {cfg['n_positions']}")
        shape = [batch, H, max_len, d // H]
        self.batch, self.max_len, self.dtype = batch, max_len, dtype
        self.k = [gpu.zeros(shape, dtype) for _ in range(cfg["n_layer"])]
        self.v = [gpu.zeros(shape, dtype) for _ in range(cfg["n_layer"])]
        self.pos = gpu.from_numpy(np.zeros(batch, np.int32))
        self.one = gpu.from_numpy(np.ones(1, np.int32))
        self.length = 0   # host mirror of pos (all sequences advance together)

    def nbytes(self) -> int:
        n = 0
        for t in self.k + self.v:
            c = 1
            for s in t.shape:
                c *= s
            n += c * gpu.dtype_size(self.dtype)
        return n


def _block(model, i, x, B, T, attend):
    """One transformer layer on x [B*T, d]; `attend(i, q, k, v)` gets the
    heads as [B, H, T, hd] views of the fused QKV projection and returns the
    attention output [B, H, T, hd]."""
    w = model["weights"]
    cfg = model["config"]
    H, d = cfg["n_head"], cfg["n_embd"]
    hd = d // H
    p = f"transformer.h.{i}"
    # layer-norm outputs stay anonymous temporaries: the graph can then fold
    # each layer_norm into the projection that consumes it
    R = B * T
    qkv = gpu.add_bias(_mm(model, gpu.layer_norm(x, w[f"{p}.ln_1.weight"], w[f"{p}.ln_1.bias"]),
                           f"{p}.attn.c_attn.weight", R), w[f"{p}.attn.c_attn.bias"])

    def heads(lo):
        part = gpu.slice(qkv, 1, lo, lo + d)
        return gpu.transpose_dims(gpu.reshape(part, [B, T, H, hd]), 1, 2)

    a = attend(i, heads(0), heads(d), heads(2 * d))
    a = gpu.reshape(gpu.transpose_dims(a, 1, 2), [B * T, d])
    x = x + gpu.add_bias(_mm(model, a, f"{p}.attn.c_proj.weight", R), w[f"{p}.attn.c_proj.bias"])
    f = gpu.gelu(gpu.add_bias(_mm(model, gpu.layer_norm(x, w[f"{p}.ln_2.weight"], w[f"{p}.ln_2.bias"]),
                                  f"{p}.mlp.c_fc.weight", R), w[f"{p}.mlp.c_fc.bias"]))
    return x + gpu.add_bias(_mm(model, f, f"{p}.mlp.c_proj.weight", R), w[f"{p}.mlp.c_proj.bias"])


def _head(model, x, rows):
    w = model["weights"]
    x = gpu.layer_norm(x, w["transformer.ln_f.weight"], w["transformer.ln_f.bias"])
    return _mm(model, x, "transformer.wte.weight", rows)


def gpt2_prefill(model: dict, ids, cache: KVCache, positions=None):
    """Causal forward of a batch of prompts [B, T] into an empty cache.

    Returns (logits [B*T, vocab], next_tokens int32 [B] on the device: the
    greedy pick at each prompt's last position).  Follows the reference's
    first generate step (python/applegpu_runtime/models/generate.py:110-119:
    gpt2_forward over the prompt, argmax of the last position's logits) for B
    prompts at once; the K/V rows of every layer are written into `cache`.
    `ids` may be a numpy array or an int32 GpuTensor [B, T]; `positions`
    (int32 GpuTensor [B*T], 0..T-1 per sequence) keeps the call free of host
    copies so it can be captured."""
    w = model["weights"]
    cfg = model["config"]
    if isinstance(ids, gpu.GpuTensor):
        B, T = ids.shape
        idx = gpu.reshape(ids, [B * T])
    else:
        ids = np.asarray(ids, dtype=np.int32)
        B, T = ids.shape
        idx = gpu.from_numpy(ids.reshape(-1))
    if B != cache.batch:
        raise ValueError(f"batch {B} does not match the cache's {cache.batch}")
    if T > cache.max_len:
        raise ValueError(f"prompt length {T} exceeds the cache length {cache.max_len}")
    if cache.length != 0:
        raise ValueError("gpt2_prefill needs an empty cache")
    if positions is None:
        positions = gpu.from_numpy(np.tile(np.arange(T, dtype=np.int32), B))
    x = gpu.embedding(w["transformer.wte.weight"], idx) + gpu.embedding(w["transformer.wpe.weight"], positions)

    def attend(i, q, k, v):
        gpu.kv_write_pair(cache.k[i], cache.v[i], k, v, cache.pos)
        return gpu.attention_causal(q, k, v)

    for i in range(cfg["n_layer"]):
        x = _block(model, i, x, B, T, attend)
    logits = _head(model, x, B * T)
    V = logits.shape[-1]
    last = gpu.reshape(gpu.slice(gpu.reshape(logits, [B, T, V]), 1, T - 1, T), [B, V])
    return logits, gpu.argmax(last)


def gpt2_decode_step(model: dict, tokens, cache: KVCache):
    """One greedy decode step for the whole batch: tokens int32 [B] (device)
    at positions cache.pos.  Appends each layer's K/V row in place, attends
    over the first pos+1 cache rows, and returns (logits [B, vocab],
    next_tokens int32 [B], lens int32 [B] = pos + 1), all on the device.

    The reference's decode step (python/applegpu_runtime/models/gpt2.py:84-178
    with kv_cache, generate.py:110-119) processes the last token of one
    sequence against its concatenated cache with non-causal attention; this
    is the same computation for B sequences, with the cache append and the
    lengths on the device.  The caller advances the cache with
    `gpu.blit_copy(lens, cache.pos)` once the step's results are consumed."""
    w = model["weights"]
    cfg = model["config"]
    B = cache.batch
    x = gpu.embedding(w["transformer.wte.weight"], tokens) + gpu.embedding(w["transformer.wpe.weight"], cache.pos)
    lens = cache.pos + cache.one

    def attend(i, q, k, v):
        # the attention kernel stores k, v as cache row pos (= lens - 1)
        return gpu.decode_attention(q, cache.k[i], cache.v[i], lens, k_new=k, v_new=v)

    for i in range(cfg["n_layer"]):
        x = _block(model, i, x, B, 1, attend)
    logits = _head(model, x, B)
    return logits, gpu.argmax(logits), lens


def generate_greedy(model: dict, prompt_ids, n_steps: int, cache: KVCache = None, capture: bool = True,
                    keep_logits: bool = False):
    """Greedy generation for a batch of equal-length prompts [B, T]: one
    prefill, then `n_steps` decode steps.  Returns int32 tokens [B, n_steps+1]
    (the prefill's pick, then one per decode step), plus the per-step logits
    (numpy [n_steps+1, B, vocab]) when keep_logits.

    With capture=True the decode step is recorded once as a HIP graph and
    replayed for every token: positions, the cache append and the next-token
    argmax all stay on the device, so a step costs one graph launch."""
    prompt_ids = np.asarray(prompt_ids, dtype=np.int32)
    B, T = prompt_ids.shape
    if cache is None:
        cache = KVCache(model["config"], B, T + n_steps, model.get("dtype", "float16"))
    if T + n_steps > cache.max_len:
        raise ValueError(f"prompt {T} + {n_steps} steps exceeds the cache length {cache.max_len}")
    logits, nxt = gpt2_prefill(model, prompt_ids, cache)
    tokens = gpu.zeros([B], "int32")
    gpu.blit_copy(nxt, tokens)
    gpu.blit_copy(cache.pos + gpu.from_numpy(np.full(1, T, np.int32)), cache.pos)
    cache.length = T
    out = gpu.zeros([n_steps + 1, B], "int32")
    gpu.blit_copy(tokens, gpu.slice(out, 0, 0, 1))
    kept = []
    if keep_logits:
        V = logits.shape[-1]
        kept.append(gpu.reshape(gpu.slice(gpu.reshape(logits, [B, T, V]), 1, T - 1, T), [B, V]).to_numpy())
    del logits, nxt

    def step():
        lg, nx, lens = gpt2_decode_step(model, tokens, cache)
        gpu.blit_copy(nx, tokens)
        gpu.blit_copy(lens, cache.pos)
        return lg

    graph = gpu.capture(step) if capture and n_steps > 0 else None
    for s in range(n_steps):
        if graph is not None:
            graph.replay()
            lg = graph.outputs
        else:
            lg = step()
        cache.length += 1
        gpu.blit_copy(tokens, gpu.slice(out, 0, s + 1, s + 2))
        if keep_logits:
            kept.append(lg.to_numpy())
    toks = out.to_numpy().T.copy()
    if graph is not None:
        graph.destroy()
    if keep_logits:
        return toks, np.stack(kept)
    return toks


class Generation:
    """Greedy generation for B prompts of T ids as config C4 runs it: the
    prefill and one decode step are each captured once as a HIP graph
    (capture=True) over device-resident ids, positions, cache lengths and
    tokens, so a generation is one prefill replay and `n_steps` decode
    replays with no host work between them.  The picked tokens land in
    `out` [n_steps + 1, B] on the device.  With capture=False the same calls
    run op by op (the same kernels, launched one at a time).

    The steps follow the reference's generate loop
    (python/applegpu_runtime/models/generate.py:110-119: gpt2_forward over the
    prompt, argmax of the last position, then one token per step against the
    KV cache, python/applegpu_runtime/models/gpt2.py:84-178) for B sequences
    at once."""

    def __init__(self, model: dict, prompt_ids, n_steps: int, capture: bool = True):
        prompt = np.asarray(prompt_ids, dtype=np.int32)
        if prompt.ndim != 2:
            raise ValueError("prompt_ids must be [batch, length]")
        B, T = prompt.shape
        self.model, self.B, self.T, self.n_steps = model, B, T, n_steps
        self.cache = KVCache(model["config"], B, T + n_steps, model.get("dtype", "float16"))
        self.ids = gpu.from_numpy(prompt)
        self.positions = gpu.from_numpy(np.tile(np.arange(T, dtype=np.int32), B))
        self._zeros = gpu.from_numpy(np.zeros(B, np.int32))
        self._prompt_len = gpu.from_numpy(np.full(B, T, np.int32))
        self.tokens = gpu.zeros([B], "int32")
        self.out = gpu.zeros([n_steps + 1, B], "int32")
        self._slots = [gpu.slice(self.out, 0, s, s + 1) for s in range(n_steps + 1)]
        self.graphs = None
        if capture:
            self.graphs = (gpu.capture(self._prefill), gpu.capture(self._step) if n_steps > 0 else None)

    def _prefill(self):
        gpu.blit_copy(self._zeros, self.cache.pos)
        logits, nxt = gpt2_prefill(self.model, self.ids, self.cache, positions=self.positions)
        gpu.blit_copy(nxt, self.tokens)
        gpu.blit_copy(self._prompt_len, self.cache.pos)
        return logits

    def _step(self):
        logits, nxt, lens = gpt2_decode_step(self.model, self.tokens, self.cache)
        gpu.blit_copy(nxt, self.tokens)
        gpu.blit_copy(lens, self.cache.pos)
        return logits

    def prefill(self):
        """Runs the prefill; returns its logits [B*T, vocab] (device) and
        stores the first pick in out[0]."""
        if self.graphs is not None:
            self.graphs[0].replay()
            logits = self.graphs[0].outputs
        else:
            logits = self._prefill()
            logits.eval()
        gpu.blit_copy(self.tokens, self._slots[0])
        return logits

    def step(self, s: int):
        """Runs decode step s (0-based; input token out[s]); returns its
        logits [B, vocab] (device) and stores the pick in out[s + 1]."""
        if not 0 <= s < self.n_steps:
            raise ValueError(f"decode step {s} outside 0..{self.n_steps - 1}")
        if self.graphs is not None:
            self.graphs[1].replay()
            logits = self.graphs[1].outputs
        else:
            logits = self._step()
            logits.eval()
        gpu.blit_copy(self.tokens, self._slots[s + 1])
        return logits

    def last_logits(self, prefill_logits):
        """The prefill logits at each prompt's last position, [B, vocab]."""
        V = prefill_logits.shape[-1]
        return gpu.reshape(gpu.slice(gpu.reshape(prefill_logits, [self.B, self.T, V]), 1, self.T - 1, self.T),
                           [self.B, V])

    def run(self, keep_logits: bool = False):
        """One whole generation.  Returns the tokens [B, n_steps + 1] (numpy),
        and with keep_logits the logits of every pick, [n_steps + 1, B, vocab]
        (numpy; copying them out synchronises after every step)."""
        kept = []
        lg = self.prefill()
        if keep_logits:
            kept.append(self.last_logits(lg).to_numpy())
        for s in range(self.n_steps):
            lg = self.step(s)
            if keep_logits:
                kept.append(lg.to_numpy())
        toks = self.out.to_numpy().T.copy()
        return (toks, np.stack(kept)) if keep_logits else toks

    def destroy(self):
        if self.graphs is not None:
            for g in self.graphs:
                if g is not None:
                    g.destroy()
            self.graphs = None
