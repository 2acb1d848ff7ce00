"""Writes the golden fixtures used by the parity tests.

1. reference_known_answers.json — the known-answer vectors the reference's
   own tests assert (values transcribed from the cited test lines).
2. torch_cpu_fixtures.npz — seeded inputs and PyTorch CPU eager outputs
   (torch 2.10, the reference's parity oracle: python/tests/test_cpp_backend.py
   compares every op against torch CPU) for each hot-path op at small shapes.

Run from the repo root:  python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

KNOWN = [
    {"src": "crates/core/src/compute.rs:2811-2820", "op": "matmul", "a": [[1, 2], [3, 4]], "b": [[5, 6], [7, 8]],
     "expect": [[19, 22], [43, 50]], "atol": 0.0},
    {"src": "crates/core/src/compute.rs:2822-2831", "op": "matmul", "a": [[1, 2, 3], [4, 5, 6]],
     "b": [[7, 8], [9, 10], [11, 12]], "expect": [[58, 64], [139, 154]], "atol": 0.0},
    {"src": "crates/core/src/compute.rs:2800-2808", "op": "relu", "x": [-1.0, 0.0, 3.0, -4.0],
     "expect": [0.0, 0.0, 3.0, 0.0], "atol": 0.0},
    {"src": "crates/core/src/compute.rs:2911-2921", "op": "softmax", "x": [[1.0, 2.0, 3.0]],
     "expect": [[0.0900, 0.2447, 0.6652]], "atol": 1e-3},
    {"src": "crates/core/src/ops.rs:3171-3198", "op": "softmax_causal", "x": [[1.0] * 3] * 3,
     "expect": [[1, 0, 0], [0.5, 0.5, 0], [1 / 3, 1 / 3, 1 / 3]], "atol": 1e-3},
    {"src": "crates/core/src/ops.rs:3408-3431", "op": "attention_causal_row0", "q": [[1, 0], [0, 1]],
     "k": [[1, 0], [0, 1]], "v": [[1, 2], [3, 4]], "expect_row0": [1.0, 2.0], "atol": 0.1},
    {"src": "python/tests/test_attention.py:4-21", "op": "softmax_rows_sum", "x": [[1, 2, 3], [1, 1, 1]],
     "expect_row_sums": [1.0, 1.0], "atol": 1e-5},
    {"src": "python/tests/test_attention.py:15-21", "op": "softmax", "x": [[1.0, 1.0, 1.0, 1.0]],
     "expect": [[0.25, 0.25, 0.25, 0.25]], "atol": 1e-5},
    {"src": "python/tests/test_attention.py:24-37", "op": "transpose", "x": [[1, 2, 3], [4, 5, 6]],
     "expect": [[1, 4], [2, 5], [3, 6]], "atol": 0.0},
    {"src": "python/tests/test_transformer_ops.py:44-62", "op": "layer_norm",
     "x": [[1, 2, 3, 4], [2, 4, 6, 8]], "gamma": [1, 1, 1, 1], "beta": [0, 0, 0, 0],
     "expect": [[((v - 2.5) / math.sqrt(1.25 + 1e-5)) for v in (1, 2, 3, 4)],
                [((v - 5.0) / math.sqrt(5.0 + 1e-5)) for v in (2, 4, 6, 8)]], "rtol": 1e-4},
    {"src": "python/tests/test_transformer_ops.py:65-80", "op": "layer_norm", "x": [[1, 2, 3, 4]],
     "gamma": [2, 2, 2, 2], "beta": [1, 1, 1, 1],
     "expect": [[2.0 * ((v - 2.5) / math.sqrt(1.25 + 1e-5)) + 1.0 for v in (1, 2, 3, 4)]], "rtol": 1e-4},
    {"src": "python/tests/test_transformer_ops.py:14-24", "op": "gelu", "x": [0.0, 1.0, -1.0, 2.0],
     "expect": [v * 0.5 * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))
                for v in (0.0, 1.0, -1.0, 2.0)], "rtol": 1e-4},
    {"src": "python/tests/test_transformer_ops.py:102-120", "op": "embedding",
     "w": [[0.1, 0.2, 0.3], [1.1, 1.2, 1.3], [2.1, 2.2, 2.3], [3.1, 3.2, 3.3], [4.1, 4.2, 4.3]],
     "idx": [0, 3, 1], "expect": [[0.1, 0.2, 0.3], [3.1, 3.2, 3.3], [1.1, 1.2, 1.3]], "atol": 0.0},
    {"src": "crates/core/src/ops.rs:4573-4611", "op": "softmax_backward", "y": [[0.2, 0.3, 0.5], [0.1, 0.7, 0.2]],
     "dy": [[1.0, 0.0, 0.0], [0.0, 1.0, 0.0]], "expect": [[0.16, -0.06, -0.10], [-0.07, 0.21, -0.14]], "atol": 1e-5},
    {"src": "crates/core/src/ops.rs:4618-4647", "op": "softmax_backward_ones", "x": [[1.0, 2.0, 3.0], [4.0, 1.0, 2.0]],
     "expect_abs_max": 0.0, "atol": 1e-5},
    {"src": "crates/core/src/ops.rs:4699-4730", "op": "layer_norm_backward_row_sums",
     "x": [[1, 2, 3, 4], [5, 6, 7, 8]], "gamma": [1, 1, 1, 1], "dy": [[1] * 4] * 2, "expect_row_sums": [0.0, 0.0],
     "atol": 1e-4},
    {"src": "crates/core/src/ops.rs:4973-4998", "op": "embedding_backward", "dy": [[1, 2], [3, 4], [5, 6]],
     "idx": [0, 1, 0], "num_weights": 3, "expect": [[6, 8], [3, 4], [0, 0]], "atol": 1e-4},
    {"src": "crates/core/src/ops.rs:5000-5021", "op": "embedding_backward", "dy": [[10, 20], [30, 40], [50, 60]],
     "idx": [0, 1, 2], "num_weights": 3, "expect": [[10, 20], [30, 40], [50, 60]], "atol": 1e-4},
]


def main():
    with open(os.path.join(HERE, "reference_known_answers.json"), "w") as f:
        json.dump(KNOWN, f, indent=1)

    torch.manual_seed(42)
    fx = {}
    # rows: ragged widths (not multiples of 4) and the GPT-2 width
    for name, shape in {"r7": (5, 7), "r768": (6, 768), "r2500": (3, 2500)}.items():
        x = torch.randn(*shape) * 3
        fx[f"softmax_{name}_x"] = x.numpy()
        fx[f"softmax_{name}_y"] = torch.softmax(x, -1).numpy()
        fx[f"log_softmax_{name}_y"] = torch.log_softmax(x, -1).numpy()
        g = torch.randn(shape[-1])
        b = torch.randn(shape[-1])
        fx[f"layer_norm_{name}_g"] = g.numpy()
        fx[f"layer_norm_{name}_b"] = b.numpy()
        fx[f"layer_norm_{name}_y"] = F.layer_norm(x, (shape[-1],), g, b, 1e-5).numpy()
    xc = torch.randn(2, 9, 9)
    mask = torch.ones(9, 9, dtype=torch.bool).tril()
    fx["softmax_causal_x"] = xc.numpy()
    fx["softmax_causal_y"] = torch.softmax(xc.masked_fill(~mask, float("-inf")), -1).numpy()
    xg = torch.randn(4, 33) * 4
    fx["gelu_x"] = xg.numpy()
    fx["gelu_tanh_y"] = F.gelu(xg, approximate="tanh").numpy()
    fx["gelu_erf_y"] = F.gelu(xg).numpy()
    # GEMM, including a ragged shape
    a = torch.randn(37, 45)
    b = torch.randn(45, 29)
    fx["matmul_a"], fx["matmul_b"], fx["matmul_y"] = a.numpy(), b.numpy(), (a @ b).numpy()
    # attention (batched heads, causal and not)
    q, k, v = torch.randn(3, 70, 64), torch.randn(3, 70, 64), torch.randn(3, 70, 64)
    fx["attn_q"], fx["attn_k"], fx["attn_v"] = q.numpy(), k.numpy(), v.numpy()
    fx["attn_causal_y"] = F.scaled_dot_product_attention(q, k, v, is_causal=True).numpy()
    fx["attn_full_y"] = F.scaled_dot_product_attention(q, k, v).numpy()
    # argmax with ties (first index wins)
    am = torch.randint(0, 5, (6, 40)).float()
    fx["argmax_x"], fx["argmax_y"] = am.numpy(), am.argmax(-1).to(torch.int32).numpy()
    # per-row int8 quantize with exact .5 ties and a zero row
    w = torch.randn(8, 300) * 0.02
    w[3] = 0.0
    # exact ties: absmax 127 * 2^-10 gives scale 2^-10, so k.5 * 2^-10 / scale = k.5
    w[5] = 0.0
    w[5, :5] = torch.tensor([127.0, 0.5, -0.5, 1.5, -2.5]) * 2.0 ** -10
    scale = w.abs().amax(1) / 127
    qv = torch.round(w / scale[:, None]).clamp(-128, 127)
    qv[3] = 0  # zero row: 0/0 in the fp32 expression; codes are 0 by convention
    fx["quant_w"], fx["quant_scale"], fx["quant_q"] = w.numpy(), scale.numpy(), qv.to(torch.int8).numpy()
    # dequantize, two independent torch routes: fp32 arithmetic on the codes,
    # and torch's own per-channel quantized tensor (axis 0, zero points 0)
    q8 = qv.to(torch.int8)
    fx["quant_deq"] = (q8.to(torch.float32) * scale[:, None]).numpy()
    fx["quant_deq_qtensor"] = torch._make_per_channel_quantized_tensor(
        q8, scale.double(), torch.zeros(q8.shape[0], dtype=torch.long), 0).dequantize().numpy()
    # per-tensor dequantize (q - zp) * scale with nonzero zero points, int8 and
    # uint8 codes (torch's per-tensor quantized tensor; no RNG drawn here)
    codes8 = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8)
    codes_u8 = torch.arange(0, 256, dtype=torch.int16).to(torch.uint8)
    fx["dq_pt_i8_q"] = codes8.numpy()
    fx["dq_pt_i8_y"] = torch._make_per_tensor_quantized_tensor(codes8, 0.1, -3).dequantize().numpy()
    fx["dq_pt_u8_q"] = codes_u8.numpy()
    fx["dq_pt_u8_y"] = torch._make_per_tensor_quantized_tensor(codes_u8, 0.05, 7).dequantize().numpy()
    # embedding
    ew = torch.randn(50, 16)
    ei = torch.randint(0, 50, (11,), dtype=torch.int32)
    fx["emb_w"], fx["emb_idx"], fx["emb_y"] = ew.numpy(), ei.numpy(), F.embedding(ei.long(), ew).numpy()
    # MSE loss and its gradient through autograd
    pa = torch.randn(32, 10, requires_grad=True)
    pb = torch.randn(32, 10)
    loss = F.mse_loss(pa, pb)
    loss.backward()
    fx["mse_a"], fx["mse_b"] = pa.detach().numpy(), pb.numpy()
    fx["mse_loss"], fx["mse_grad"] = np.array([loss.item()], np.float32), pa.grad.numpy()
    # config 1: MLP 64->128->10, batch 32, one SGD step (lr 0.01)
    torch.manual_seed(42)
    x = torch.randn(32, 64)
    y = torch.randn(32, 10)
    model = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.ReLU(), torch.nn.Linear(128, 10))
    for i, m in enumerate([model[0], model[2]]):
        fx[f"mlp_w{i}"] = m.weight.detach().numpy().copy()
        fx[f"mlp_b{i}"] = m.bias.detach().numpy().copy()
    opt = torch.optim.SGD(model.parameters(), lr=0.01)
    out = model(x)
    loss = F.mse_loss(out, y)
    opt.zero_grad()
    loss.backward()
    for i, m in enumerate([model[0], model[2]]):
        fx[f"mlp_gw{i}"] = m.weight.grad.numpy().copy()
        fx[f"mlp_gb{i}"] = m.bias.grad.numpy().copy()
    opt.step()
    for i, m in enumerate([model[0], model[2]]):
        fx[f"mlp_w{i}_after"] = m.weight.detach().numpy().copy()
        fx[f"mlp_b{i}_after"] = m.bias.detach().numpy().copy()
    fx["mlp_x"], fx["mlp_y"] = x.numpy(), y.numpy()
    fx["mlp_out"], fx["mlp_loss"] = out.detach().numpy(), np.array([loss.item()], np.float32)
    np.savez_compressed(os.path.join(HERE, "torch_cpu_fixtures.npz"), **fx)
    print(f"wrote {len(KNOWN)} known answers and {len(fx)} arrays")


if __name__ == "__main__":
    main()
