"""Benchmark of the MI355X backend on BASELINE.json's headline metric:
GPT-2-small forward ms at seq 128 (config 2) + MLP h=4096 train ms/step
(config 3), on one MI355X, with the roofline fraction of the dominant kernel.

A step = one GPT-2-small fp32 forward over 128 token ids (the lazy graph of
the reference's gpt2_forward recipe, evaluated on the device; logits stay in
HBM) + one training step of Linear(4096,4096)-ReLU-Linear(4096,4096)-ReLU-
Linear(4096,1) at batch 256 (forward, MSE, backward, SGD lr 0.01) through
the eager C ABI.  Weights are random (N(0,0.02) for GPT-2; torch's default
Linear init for the MLP) and inputs synthetic, seeded; everything is resident
in HBM before the timed region.

Prints ONE JSON line.  `python bench.py --gpus N` with N > 1 exits: this
build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "applegpu-runtime_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

METRIC = "GPT-2-small fwd ms @seq128 + MLP h=4096 train ms/step, 1 MI355X; % roofline"
FP32_MFMA_PEAK_TFLOPS = 157.3
GPT2_CFG = dict(n_layer=12, n_head=12, n_embd=768, vocab_size=50257, n_positions=1024)
MLP_SIZES = [4096, 4096, 4096, 1]
MLP_BATCH = 256
SEQ = 128


def gpt2_flops(cfg, T):
    d, V, L, H = cfg["n_embd"], cfg["vocab_size"], cfg["n_layer"], cfg["n_head"]
    hd = d // H
    per_layer = 2 * T * d * 3 * d + 2 * T * d * d + 2 * T * d * 4 * d + 2 * T * 4 * d * d + 2 * (2 * H * T * T * hd)
    return L * per_layer + 2 * T * V * d


def mlp_flops(sizes, B):
    f = 0
    for i, (fin, fout) in enumerate(zip(sizes[:-1], sizes[1:])):
        f += 2 * B * fin * fout          # forward
        f += 2 * fin * fout * B          # dW
        if i > 0:
            f += 2 * B * fout * fin      # dX
    return f


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-s", type=float, default=15.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is described in DESIGN.md, not built).", file=sys.stderr)
        sys.exit(2)

    import applegpu_runtime as gpu
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    from applegpu_runtime.models import gpt2 as G
    from applegpu_runtime.models.mlp import EagerMLP, torch_default_init

    gpu.init_backend()
    dev = gpu.device_name()

    # ── inputs resident in HBM ──────────────────────────────────────────────
    wnp = G.random_weights(GPT2_CFG, seed=42)
    model = G.load_model(wnp, GPT2_CFG)
    ids = np.random.default_rng(42).integers(0, GPT2_CFG["vocab_size"], SEQ)

    params = torch_default_init(MLP_SIZES, seed=42)
    rng = np.random.default_rng(42)
    xnp = rng.standard_normal((MLP_BATCH, MLP_SIZES[0]), dtype=np.float32)
    ynp = rng.standard_normal((MLP_BATCH, MLP_SIZES[-1]), dtype=np.float32)
    mlp = EagerMLP(params)
    x, y = E.from_numpy(xnp), E.from_numpy(ynp)
    lib.applegpu_ffi_synchronize()

    def gpt2_step():
        logits, _ = G.gpt2_forward(model, ids)
        logits.eval()
        return logits

    def mlp_step():
        return mlp.train_step(x, y, lr=0.01)

    for _ in range(args.warmup):
        gpt2_step()
        mlp_step()
    lib.applegpu_ffi_synchronize()

    # ── timed region: K steps, each = GPT-2 forward + MLP train step ────────
    t_g = t_m = 0.0
    for _ in range(args.steps):
        lib.applegpu_ffi_synchronize()
        t0 = time.perf_counter()
        gpt2_step()
        lib.applegpu_ffi_synchronize()
        t1 = time.perf_counter()
        mlp_step()
        lib.applegpu_ffi_synchronize()
        t2 = time.perf_counter()
        t_g += t1 - t0
        t_m += t2 - t1
    gpt2_ms = 1e3 * t_g / args.steps
    mlp_ms = 1e3 * t_m / args.steps
    ms_per_step = gpt2_ms + mlp_ms

    # ── dominant kernel: the MLP forward GEMM (x W^T, 256x4096x4096 fp32 on
    #    v_mfma_f32_32x32x2_f32), timed with HIP events on the library stream ─
    w0 = mlp.params[1][0]
    h = E.from_numpy(rng.standard_normal((MLP_BATCH, 4096), dtype=np.float32))
    for _ in range(3):
        E.linear(h, w0, None, 0)
    reps = 50
    lib.applegpu_ffi_event_record(0)
    outs = [E.linear(h, w0, None, 0) for _ in range(reps)]
    lib.applegpu_ffi_event_record(1)
    gemm_ms = lib.applegpu_ffi_event_elapsed_ms(0, 1) / reps
    del outs
    gemm_flop = 2.0 * MLP_BATCH * 4096 * 4096
    achieved = gemm_flop / (gemm_ms * 1e-3) / 1e12

    result = {
        "metric": METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C2 GPT-2 small fp32 fwd (1x128 tokens, random N(0,0.02) weights) + C3 MLP "
                        "4096-4096-4096-1 fp32 train step (batch 256, MSE, SGD lr 0.01)",
            "gpt2_fwd_ms": round(gpt2_ms, 4),
            "mlp_train_ms": round(mlp_ms, 4),
            "gpt2_fwd_tflops": round(gpt2_flops(GPT2_CFG, SEQ) / (gpt2_ms * 1e-3) / 1e12, 2),
            "mlp_train_tflops": round(mlp_flops(MLP_SIZES, MLP_BATCH) / (mlp_ms * 1e-3) / 1e12, 2),
            "device": dev,
        },
        "roofline": {
            "kernel": "gemm_f32_mfma (x W^T, M=256 N=4096 K=4096, split-K + reduce)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "avg_launch_ms": round(gemm_ms, 5),
            "flop_per_launch": gemm_flop,
            "traffic": None,
        },
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wnp, params, ids, xnp, ynp, args.cpu_sample_s)
    print(json.dumps(result), flush=True)


def cpu_baseline(wnp, params, ids, xnp, ynp, budget_s):
    """The reference's CPU path (PyTorch CPU eager) on a bounded sample of the
    same workload: GPT-2 forwards and MLP steps alternate until ~budget_s."""
    import torch
    from oracle.torch_cpu import TorchGPT2, TorchMLP
    g = TorchGPT2(wnp, GPT2_CFG)
    m = TorchMLP(params, lr=0.01)
    tx, ty = torch.from_numpy(xnp), torch.from_numpy(ynp)
    g.forward(ids)
    m.step(tx, ty)
    tg = tm = 0.0
    n = 0
    start = time.perf_counter()
    while n < 2 or (time.perf_counter() - start < budget_s and n < 50):
        t0 = time.perf_counter()
        g.forward(ids)
        t1 = time.perf_counter()
        m.step(tx, ty)
        t2 = time.perf_counter()
        tg += t1 - t0
        tm += t2 - t1
        n += 1
    return {
        "value": round(1e3 * (tg + tm) / n, 3),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{n} x (GPT-2 small fwd seq128 + MLP 4096 train step), torch {torch.__version__} CPU eager; "
                  f"gpt2 {1e3 * tg / n:.1f} ms, mlp {1e3 * tm / n:.1f} ms; host cpus {os.cpu_count()}",
    }


if __name__ == "__main__":
    main()
