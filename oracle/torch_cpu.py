"""The reference's CPU path: PyTorch CPU eager (test infrastructure / CPU baseline only).

The reference measures its published numbers against PyTorch CPU eager
(benchmarks/bench_mlp_cpp.py:74-76, python/tests/bench_comparison.py:44-51;
torch 2.10.0 pinned in uv.lock:1352-1353) and uses it as ground truth in its
tests (python/tests/test_cpp_backend.py:121-133, 267-371).  These functions
restate those CPU workloads: the MLP training step of bench_mlp_cpp.py and a
GPT-2 forward with the recipe of python/applegpu_runtime/models/gpt2.py:47-180
written as torch CPU ops.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


class TorchMLP:
    """nn.Linear/ReLU stack + MSELoss + SGD on the CPU (bench_mlp_cpp.py:16-52)."""

    def __init__(self, params_np, lr=0.01):
        layers = []
        n = len(params_np)
        for i, (w, b) in enumerate(params_np):
            lin = torch.nn.Linear(w.shape[1], w.shape[0])
            with torch.no_grad():
                lin.weight.copy_(torch.from_numpy(np.asarray(w)))
                lin.bias.copy_(torch.from_numpy(np.asarray(b)))
            layers.append(lin)
            if i < n - 1:
                layers.append(torch.nn.ReLU())
        self.model = torch.nn.Sequential(*layers)
        self.opt = torch.optim.SGD(self.model.parameters(), lr=lr)
        self.crit = torch.nn.MSELoss()

    def step(self, x, y):
        self.opt.zero_grad()
        loss = self.crit(self.model(x), y)
        loss.backward()
        self.opt.step()
        return loss


class TorchGPT2:
    """GPT-2 forward in torch CPU ops with the weights of models.gpt2.random_weights."""

    def __init__(self, np_weights: dict, cfg: dict):
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in np_weights.items()}
        self.cfg = cfg

    @torch.no_grad()
    def forward(self, ids):
        w, cfg = self.w, self.cfg
        L, H, d = cfg["n_layer"], cfg["n_head"], cfg["n_embd"]
        hd = d // H
        ids = torch.as_tensor(np.asarray(ids).reshape(-1), dtype=torch.long)
        T = ids.shape[0]
        x = w["transformer.wte.weight"][ids] + w["transformer.wpe.weight"][:T]
        for i in range(L):
            p = f"transformer.h.{i}"
            h = F.layer_norm(x, (d,), w[f"{p}.ln_1.weight"], w[f"{p}.ln_1.bias"], 1e-5)
            qkv = h @ w[f"{p}.attn.c_attn.weight"] + w[f"{p}.attn.c_attn.bias"]
            q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(T, H, hd).transpose(0, 1) for j in range(3))
            s = (q @ k.transpose(1, 2)) * (1.0 / math.sqrt(hd))
            mask = torch.ones(T, T, dtype=torch.bool).tril()
            a = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1) @ v
            a = a.transpose(0, 1).reshape(T, d)
            x = x + (a @ w[f"{p}.attn.c_proj.weight"] + w[f"{p}.attn.c_proj.bias"])
            h = F.layer_norm(x, (d,), w[f"{p}.ln_2.weight"], w[f"{p}.ln_2.bias"], 1e-5)
            f = F.gelu(h @ w[f"{p}.mlp.c_fc.weight"] + w[f"{p}.mlp.c_fc.bias"], approximate="tanh")
            x = x + (f @ w[f"{p}.mlp.c_proj.weight"] + w[f"{p}.mlp.c_proj.bias"])
        x = F.layer_norm(x, (d,), w["transformer.ln_f.weight"], w["transformer.ln_f.bias"], 1e-5)
        return x @ w["transformer.wte.weight"].T


class TorchGPT2Decoder:
    """Batched greedy generation with a KV cache in torch CPU ops: the
    reference's generate loop (python/applegpu_runtime/models/generate.py:
    110-119: a prompt forward, then one token per step against the cache,
    argmax of the last position) for B equal-length prompts, on the recipe of
    python/applegpu_runtime/models/gpt2.py:84-178.  fp32 arithmetic on the
    given weights (pass the fp16-rounded ones to mirror an fp16 device model).
    """

    def __init__(self, np_weights: dict, cfg: dict):
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)) for k, v in np_weights.items()}
        self.cfg = cfg
        self.k = self.v = None
        self.length = 0

    def _layer(self, i, x, B, T, causal):
        w, cfg = self.w, self.cfg
        H, d = cfg["n_head"], cfg["n_embd"]
        hd = d // H
        p = f"transformer.h.{i}"
        h = F.layer_norm(x, (d,), w[f"{p}.ln_1.weight"], w[f"{p}.ln_1.bias"], 1e-5)
        qkv = h @ w[f"{p}.attn.c_attn.weight"] + w[f"{p}.attn.c_attn.bias"]
        q, k, v = (qkv[..., j * d:(j + 1) * d].reshape(B, T, H, hd).transpose(1, 2) for j in range(3))
        s0 = self.length
        self.k[i][:, :, s0:s0 + T] = k
        self.v[i][:, :, s0:s0 + T] = v
        kk, vv = self.k[i][:, :, :s0 + T], self.v[i][:, :, :s0 + T]
        s = (q @ kk.transpose(2, 3)) * (1.0 / math.sqrt(hd))
        if causal:
            mask = torch.ones(T, s0 + T, dtype=torch.bool).tril(s0)
            s = s.masked_fill(~mask, float("-inf"))
        a = torch.softmax(s, dim=-1) @ vv
        a = a.transpose(1, 2).reshape(B * T, d)
        x = x + (a @ w[f"{p}.attn.c_proj.weight"] + w[f"{p}.attn.c_proj.bias"])
        h = F.layer_norm(x, (d,), w[f"{p}.ln_2.weight"], w[f"{p}.ln_2.bias"], 1e-5)
        f = F.gelu(h @ w[f"{p}.mlp.c_fc.weight"] + w[f"{p}.mlp.c_fc.bias"], approximate="tanh")
        return x + (f @ w[f"{p}.mlp.c_proj.weight"] + w[f"{p}.mlp.c_proj.bias"])

    def _forward(self, ids, causal):
        w, cfg = self.w, self.cfg
        B, T = ids.shape
        pos = torch.arange(self.length, self.length + T).repeat(B)
        x = w["transformer.wte.weight"][ids.reshape(-1)] + w["transformer.wpe.weight"][pos]
        for i in range(cfg["n_layer"]):
            x = self._layer(i, x, B, T, causal)
        self.length += T
        x = F.layer_norm(x, (cfg["n_embd"],), w["transformer.ln_f.weight"], w["transformer.ln_f.bias"], 1e-5)
        return (x @ w["transformer.wte.weight"].T).reshape(B, T, -1)

    @torch.no_grad()
    def prefill(self, ids, max_len):
        """logits [B, T, vocab] of the prompts; allocates the cache."""
        ids = torch.as_tensor(np.asarray(ids), dtype=torch.long)
        B = ids.shape[0]
        H, d = self.cfg["n_head"], self.cfg["n_embd"]
        shape = (B, H, max_len, d // H)
        self.k = [torch.zeros(shape) for _ in range(self.cfg["n_layer"])]
        self.v = [torch.zeros(shape) for _ in range(self.cfg["n_layer"])]
        self.length = 0
        return self._forward(ids, causal=True)

    @torch.no_grad()
    def decode(self, tokens):
        """logits [B, vocab] of one new token per sequence."""
        ids = torch.as_tensor(np.asarray(tokens), dtype=torch.long).reshape(-1, 1)
        return self._forward(ids, causal=False)[:, 0]
