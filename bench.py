"""Benchmark of the MI355X backend on BASELINE.json's headline metric:
GPT-2-small forward ms at seq 128 (config 2) + MLP h=4096 train ms/step
(config 3), on one MI355X, with the roofline fraction of the kernel that
takes the most time per step.

A step = one GPT-2-small fp32 forward over 128 token ids (the lazy graph of
the reference's gpt2_forward recipe) + one training step of
Linear(4096,4096)-ReLU-Linear(4096,4096)-ReLU-Linear(4096,1) at batch 256
(forward, MSE, backward, SGD lr 0.01, parameters updated in place) through
the eager C ABI.  Both are recorded once with gpu.capture and replayed as HIP
graphs; the same work issued op by op (no capture) is reported beside it.
Weights are random (N(0,0.02) for GPT-2; torch's default Linear init for the
MLP) and inputs synthetic, seeded; everything is resident in HBM before the
timed region.  value = gpt2_fwd_ms + mlp_train_ms, each the mean over
--steps replays bracketed by stream synchronisations.

Roofline (`roofline`): the kernel with the largest time per step, the
packed-A row-panel GEMM gemm_x3_rows_pk<6>, at each of the three shapes it
runs at in the forward, 12 launches each: qkv (128 x 768 x 2304, ln_1 folded
in, bias), the attention projection (128 x 768 x 768, bias + residual, x also
written as packed rows and row statistics) and fc (128 x 768 x 3072, ln_2
folded in, bias + gelu, packed rows out).  Both operands are pre-split bf16
hi/lo MFMA fragments (three bf16 MFMAs per product) and the weights are read
once per launch, so the kernel is bound by HBM: algorithmic bytes per launch
= packed A + packed weights + bias (+ the folded norm's statistics and column
sums, the residual) + every output.  Each shape's launch duration is timed
with HIP events on the library stream over a captured graph of back-to-back
launches that rotate through 40 weight sets (more than the 256 MB Infinity
Cache holds, so the weights stream from HBM as in the forward); the
aggregate is the bytes of one launch of each shape over their summed time.
The same launches in MFMA terms are reported beside it (against the fp32
MFMA peak and against the bf16x3 ceiling, one third of the bf16 MFMA peak).
`roofline_mlp_dw` is the MLP weight-gradient GEMM with its SGD step
(W += -lr g^T h, M = N = 4096, K = 256), one update alone: one launch packs
g^T and h as bf16 hi/lo fragments, a second (gemm_x3_outer) multiplies them
in 128 x 128 tiles and updates W in place (the step pairs its two updates
in one pack and one GEMM launch with the same tile code); its floor is W's read and write through HBM
(algorithmic bytes: W twice plus g and h once).  HBM traffic comes from
the rocprofv3 --pmc summaries committed under profiles/ (FETCH_SIZE,
WRITE_SIZE of each kernel, scaled by the same counters read for the 256 MiB
calibration copy this script runs), when present.

Prints ONE JSON line: the headline, with the other configs of BASELINE.json
as sub-records (`c1`, `c4`, `c5`), each with its own roofline and CPU
baseline (`--headline-only` leaves them out).  `python bench.py --gpus N`
with N > 1 exits: this build runs on one GPU.
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
BF16_MFMA_PEAK_TFLOPS = 2516.6
HBM_PEAK_GBS = 8000.0
GPT2_CFG = dict(n_layer=12, n_head=12, n_embd=768, vocab_size=50257, n_positions=1024)
MLP_SIZES = [4096, 4096, 4096, 1]
MLP_BATCH = 256
SEQ = 128
CALIB_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mlp_dw_gemm_traffic.json")
PROJ_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gpt2_proj_gemm_traffic.json")
C5_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c5_quantize_traffic.json")
C4_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c4_decode_step_traffic.json")
BF16X3_CEILING_TFLOPS = BF16_MFMA_PEAK_TFLOPS / 3


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


def load_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch of a roofline kernel from a committed PMC summary."""
    try:
        with open(path) as f:
            t = json.load(f)
        return float(t["bytes_per_launch"]), t
    except (OSError, KeyError, ValueError):
        return None, None


def load_step_traffic(path=C4_TRAFFIC_FILE):
    """HBM bytes of one C4 decode step from a committed PMC summary: the
    profiled step at the median context, with that context and its ratio to
    the step's algorithmic bytes."""
    try:
        with open(path) as f:
            t = json.load(f)
        steps = sorted(t["steps"], key=lambda s: s["context"])
        s = steps[len(steps) // 2]
        return float(s["bytes"]), {"context": s["context"], "ratio": s["ratio"]}
    except (OSError, KeyError, ValueError, TypeError, IndexError):
        return None, None


PANEL_SHAPES = (("qkv", 2304), ("proj", 768), ("fc", 3072))


def panel_roofline(gpu, lib, rng, reps=4, nw=40):
    """The dominant kernel, gemm_x3_rows_pk<6>, at each shape and with each
    epilogue it runs with in the forward (12 launches of each per forward):

    - qkv   128 x 768 -> 2304: ln_1 folded in (the previous layer's x as packed
            rows with its row statistics), bias; fp32 output;
    - proj  128 x 768 -> 768: packed attention rows in, bias + residual; x
            written as fp32, packed rows and row statistics;
    - fc    128 x 768 -> 3072: ln_2 folded in, bias + gelu; packed rows out.

    Each shape: one captured graph of `nw` launches over `nw` weight sets
    (more than the 256 MB Infinity Cache holds, so the weights stream from
    HBM as in the forward), replayed `reps` times between HIP events on the
    library stream.  Algorithmic bytes per launch: packed A, packed weights,
    bias (and folded-norm column sums, statistics, residual) read once,
    every output written once."""
    M, K = SEQ, GPT2_CFG["n_embd"]
    x = gpu.from_numpy(rng.standard_normal((M, K), dtype=np.float32))
    apk, ast = gpu.pack_rows_x3(x), gpu.row_stats_x3(x)
    res = gpu.from_numpy(rng.standard_normal((M, K), dtype=np.float32))
    for t in (apk, ast, res):
        t.eval()
    out = {}
    for name, N in PANEL_SHAPES:
        ws = [gpu.pack_weight_x3(gpu.from_numpy(rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)))
              for _ in range(nw)]
        bias = gpu.from_numpy(np.zeros(N, np.float32))
        cs = gpu.from_numpy(rng.standard_normal(N, dtype=np.float32) * np.float32(0.1))
        for t in ws + [bias, cs]:
            t.eval()

        def launches():
            last = None
            for w in ws:
                if name == "qkv":
                    y = gpu.add_bias(gpu.matmul_pp_norm(apk, ast, M, w, cs, N), bias)
                    y.eval()
                    last = y
                elif name == "fc":
                    y = gpu.pack_rows_x3(gpu.gelu(gpu.add_bias(gpu.matmul_pp_norm(apk, ast, M, w, cs, N), bias)))
                    y.eval()
                    last = y
                else:
                    y = res + gpu.add_bias(gpu.matmul_pp(apk, M, w, N), bias)
                    pk, st = gpu.pack_rows_x3(y), gpu.row_stats_x3(y)
                    gpu.eval_many([y, pk, st])
                    last = y
            return last

        before = gpu.graph_stats()["launcher_calls"]
        g = gpu.capture(launches)
        calls = gpu.graph_stats()["launcher_calls"] - before
        if calls != nw:
            raise RuntimeError(f"{name}: {calls} launches for {nw} products (epilogue not fused)")
        g.replay()
        lib.applegpu_ffi_synchronize()
        lib.applegpu_ffi_event_record(0)
        for _ in range(reps):
            g.replay()
        lib.applegpu_ffi_event_record(1)
        ms = lib.applegpu_ffi_event_elapsed_ms(0, 1) / (reps * nw)
        g.destroy()
        # packed A and weights (hi + lo: 4 bytes per element), bias
        nbytes = 4 * M * K + 4 * K * N + 4 * N
        if name in ("qkv", "fc"):
            nbytes += 4 * N + 8 * M * (K // 32) + 4 * M * N   # column sums, A's statistics, output
        else:
            nbytes += 4 * M * N + 4 * M * N + 4 * M * N + 8 * M * (N // 32)  # residual, C, packed C, statistics
        out[name] = {"M": M, "N": N, "K": K, "launches_per_fwd": GPT2_CFG["n_layer"], "avg_launch_ms": round(ms, 5),
                     "algorithmic_bytes": nbytes, "flop": 2 * M * N * K,
                     "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "epilogue": {"qkv": "folded ln_1, bias", "fc": "folded ln_2, bias + gelu, packed rows out",
                                  "proj": "bias + residual; fp32, packed rows and row statistics out"}[name]}
        del ws
    return out


def c2_replays(n):
    """The headline's C2 forward graph alone, replayed n times; prints the
    mean replay time.  Under rocprofv3 --kernel-trace every dispatch of the
    run is then one of the forward's kernels."""
    import applegpu_runtime as gpu
    from applegpu_runtime._native import lib
    from applegpu_runtime.models import gpt2 as G
    gpu.init_backend()
    wnp = G.random_weights(GPT2_CFG, seed=42)
    model = G.load_model(wnp, GPT2_CFG)
    ids = np.random.default_rng(42).integers(0, GPT2_CFG["vocab_size"], SEQ).astype(np.int32)
    idx = gpu.from_numpy(ids)
    pos = gpu.from_numpy(np.arange(SEQ, dtype=np.int32))
    g = gpu.capture(lambda: G.gpt2_forward(model, idx, positions=pos, need_cache=False)[0])
    g.replay()
    lib.applegpu_ffi_synchronize()
    lib.applegpu_ffi_event_record(0)
    for _ in range(n):
        g.replay()
    lib.applegpu_ffi_event_record(1)
    lib.applegpu_ffi_synchronize()
    print(json.dumps({"c2_replays": n, "ms_per_replay": round(lib.applegpu_ffi_event_elapsed_ms(0, 1) / n, 4)}))
    g.destroy()


def c3_replays(n):
    """The headline's C3 MLP train step graph alone, replayed n times; prints
    the mean replay time (each replay updates the parameters in place, as in
    the headline).  Under rocprofv3 --kernel-trace every dispatch after the
    parameter uploads is one of the step's kernels."""
    import applegpu_runtime as gpu
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    from applegpu_runtime.models.mlp import EagerMLP, torch_default_init
    gpu.init_backend()
    params = torch_default_init(MLP_SIZES, seed=42)
    rng = np.random.default_rng(42)
    x = E.from_numpy(rng.standard_normal((MLP_BATCH, MLP_SIZES[0]), dtype=np.float32))
    y = E.from_numpy(rng.standard_normal((MLP_BATCH, MLP_SIZES[-1]), dtype=np.float32))
    mlp = EagerMLP(params)
    g = gpu.capture(lambda: mlp.train_step(x, y, lr=0.01))
    g.replay()
    lib.applegpu_ffi_synchronize()
    lib.applegpu_ffi_event_record(0)
    for _ in range(n):
        g.replay()
    lib.applegpu_ffi_event_record(1)
    lib.applegpu_ffi_synchronize()
    print(json.dumps({"c3_replays": n, "ms_per_replay": round(lib.applegpu_ffi_event_elapsed_ms(0, 1) / n, 4)}))
    g.destroy()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-s", type=float, default=15.0,
                    help="time budget of the bounded C4 CPU-baseline sample")
    ap.add_argument("--suite", action="store_true",
                    help="instead of the headline line, print one JSON line per hot-path kernel "
                         "(cache-busting working sets, roofline fractions)")
    ap.add_argument("--only", default="",
                    help="with --suite: run only the sections whose name contains this text "
                         "(rows, c5, c4, decode)")
    ap.add_argument("--c1", action="store_true",
                    help="instead of the headline line, run config C1 (MLP 64-128-10 train step, batch 32) and "
                         "print its JSON line: ms/step and kernels/step, with the CPU baseline")
    ap.add_argument("--c5", action="store_true",
                    help="instead of the headline line, run config C5 (int8 per-row quantize, dequantize and the "
                         "[64,8192] x [8192,8192]^T GEMM) and print its JSON line, with the CPU baseline")
    ap.add_argument("--c4", action="store_true",
                    help="instead of the headline line, run config C4 (GPT-2 large fp16 prefill + greedy "
                         "decode over a KV cache) and print its JSON line")
    ap.add_argument("--c4-steps", type=int, default=C4_STEPS)
    ap.add_argument("--c4-reps", type=int, default=3)
    ap.add_argument("--c4-eager", action="store_true",
                    help="C4 with op-by-op launches instead of graph replays (same kernels; for kernel traces)")
    ap.add_argument("--c2-replays", type=int, default=0,
                    help="instead of the headline line, capture the C2 forward and replay it this many times "
                         "(nothing else runs: a per-forward kernel trace of exactly the timed graph)")
    ap.add_argument("--headline-only", action="store_true",
                    help="print the C2 + C3 headline line without the c1, c4 and c5 sub-records")
    ap.add_argument("--c3-replays", type=int, default=0,
                    help="instead of the headline line, capture the C3 MLP train step and replay it this many "
                         "times (a per-step kernel trace of exactly the timed graph)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is designed, not built).", file=sys.stderr)
        sys.exit(2)
    if args.c2_replays > 0:
        c2_replays(args.c2_replays)
        return
    if args.c3_replays > 0:
        c3_replays(args.c3_replays)
        return
    if args.suite:
        kernel_suite(args.only)
        return
    if args.c4:
        print(json.dumps(c4_generate(args)), flush=True)
        return
    if args.c1:
        print(json.dumps(c1_train(args)), flush=True)
        return
    if args.c5:
        print(json.dumps(c5_pipeline(args)), flush=True)
        return

    import applegpu_runtime as gpu
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    from applegpu_runtime.models import gpt2 as G
    from applegpu_runtime.models.mlp import EagerMLP, torch_default_init

    gpu.init_backend()
    dev = gpu.device_name()
    if not args.headline_only:
        # the c1 sub-record runs torch autograd on the PrivateUse1 device, whose
        # engine sizes its device queues the first time autograd runs: register
        # the device before the CPU baselines use autograd
        from applegpu_runtime.cpp_backend import load_cpp_backend
        load_cpp_backend()

    # ── inputs resident in HBM ──────────────────────────────────────────────
    wnp = G.random_weights(GPT2_CFG, seed=42)
    model = G.load_model(wnp, GPT2_CFG)
    ids = np.random.default_rng(42).integers(0, GPT2_CFG["vocab_size"], SEQ).astype(np.int32)
    idx = gpu.from_numpy(ids)
    pos = gpu.from_numpy(np.arange(SEQ, dtype=np.int32))

    params = torch_default_init(MLP_SIZES, seed=42)
    rng = np.random.default_rng(42)
    xnp = rng.standard_normal((MLP_BATCH, MLP_SIZES[0]), dtype=np.float32)
    ynp = rng.standard_normal((MLP_BATCH, MLP_SIZES[-1]), dtype=np.float32)
    mlp = EagerMLP(params)
    x, y = E.from_numpy(xnp), E.from_numpy(ynp)

    # calibration kernel for the PMC traffic counters: a plain 256 MiB copy
    csrc, cdst = E.empty((CALIB_BYTES // 4,)), E.empty((CALIB_BYTES // 4,))
    E.fill_(csrc, 1.0)
    if lib.applegpu_eager_copy_(cdst.id, csrc.id) != 0:
        raise RuntimeError("calibration copy failed")
    del csrc, cdst
    lib.applegpu_ffi_synchronize()

    # ── op-by-op (uncaptured) reference timing ──────────────────────────────
    def gpt2_eager():
        G.gpt2_forward(model, idx, positions=pos, need_cache=False)[0].eval()

    eager_mlp = EagerMLP(params)
    for _ in range(2):
        gpt2_eager()
        eager_mlp.train_step(x, y, lr=0.01)
    lib.applegpu_ffi_synchronize()
    n_eager = max(3, args.steps // 5)
    t0 = time.perf_counter()
    for _ in range(n_eager):
        gpt2_eager()
    lib.applegpu_ffi_synchronize()
    t1 = time.perf_counter()
    for _ in range(n_eager):
        eager_mlp.train_step(x, y, lr=0.01)
    lib.applegpu_ffi_synchronize()
    t2 = time.perf_counter()
    gpt2_eager_ms = 1e3 * (t1 - t0) / n_eager
    mlp_eager_ms = 1e3 * (t2 - t1) / n_eager
    del eager_mlp

    # ── captured graphs ──────────────────────────────────────────────────────
    g_fwd = gpu.capture(lambda: G.gpt2_forward(model, idx, positions=pos, need_cache=False)[0])
    g_train = gpu.capture(lambda: mlp.train_step(x, y, lr=0.01))
    for _ in range(args.warmup):
        g_fwd.replay()
        g_train.replay()
    lib.applegpu_ffi_synchronize()

    # ── timed region ─────────────────────────────────────────────────────────
    lib.applegpu_ffi_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g_fwd.replay()
    lib.applegpu_ffi_synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        g_train.replay()
    lib.applegpu_ffi_synchronize()
    t2 = time.perf_counter()
    gpt2_ms = 1e3 * (t1 - t0) / args.steps
    mlp_ms = 1e3 * (t2 - t1) / args.steps
    ms_per_step = gpt2_ms + mlp_ms
    logits = g_fwd.outputs.to_numpy()
    loss = float(g_train.outputs.numpy()[0])
    if not (np.isfinite(logits).all() and np.isfinite(loss)):
        raise RuntimeError("non-finite results")

    # ── roofline: the MLP weight-gradient GEMM with its SGD update, one
    # update alone: W += -lr * g^T h (bias-free; W a scratch copy).  The step
    # runs its two updates with the same tile code as one paired launch
    # (linear_backward_sgd_pair_) ──────────────────────────────────────────
    K_, M_, N_ = MLP_BATCH, MLP_SIZES[1], MLP_SIZES[0]
    g_act = E.from_numpy(rng.standard_normal((K_, M_), dtype=np.float32) * np.float32(1e-3))
    h_act = E.from_numpy(np.maximum(rng.standard_normal((K_, N_), dtype=np.float32), 0))
    w_scr = E.from_numpy(params[1][0])
    for _ in range(3):
        E.sgd_matmul_(w_scr, g_act, h_act, True, False, -0.01)
    lib.applegpu_ffi_synchronize()
    reps = 50
    lib.applegpu_ffi_event_record(0)
    for _ in range(reps):
        E.sgd_matmul_(w_scr, g_act, h_act, True, False, -0.01)
    lib.applegpu_ffi_event_record(1)
    gemm_ms = lib.applegpu_ffi_event_elapsed_ms(0, 1) / reps
    gemm_flop = 2.0 * M_ * N_ * K_
    achieved = gemm_flop / (gemm_ms * 1e-3) / 1e12
    dw_bytes = 4.0 * (2 * M_ * N_ + K_ * (M_ + N_))   # read and write W, read g and h
    dw_gbs = dw_bytes / (gemm_ms * 1e-3) / 1e9
    import ctypes
    plan = ctypes.create_string_buffer(96)
    lib.applegpu_ffi_gemm_plan(M_, N_, K_, 1, 0, False, False, plan, 96)
    traffic, tinfo = load_traffic()

    # ── roofline: the dominant kernel, every shape it runs at in the forward ─
    shapes = panel_roofline(gpu, lib, rng)
    # each shape runs 12 times per forward: the aggregate is total bytes over
    # total time of one launch of each
    p_ms = sum(v["avg_launch_ms"] for v in shapes.values())
    p_bytes = sum(v["algorithmic_bytes"] for v in shapes.values())
    p_flop = sum(v["flop"] for v in shapes.values())
    p_gbs = p_bytes / (p_ms * 1e-3) / 1e9
    p_tflops = p_flop / (p_ms * 1e-3) / 1e12
    p_traffic, p_tinfo = load_traffic(PROJ_TRAFFIC_FILE)

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
                        "4096-4096-4096-1 fp32 train step (batch 256, MSE, SGD lr 0.01); each replayed "
                        "as a captured HIP graph",
            "gpt2_fwd_ms": round(gpt2_ms, 4),
            "mlp_train_ms": round(mlp_ms, 4),
            "gpt2_fwd_eager_ms": round(gpt2_eager_ms, 4),
            "mlp_train_eager_ms": round(mlp_eager_ms, 4),
            "gpt2_fwd_tflops": round(gpt2_flops(GPT2_CFG, SEQ) / (gpt2_ms * 1e-3) / 1e12, 2),
            "mlp_train_tflops": round(mlp_flops(MLP_SIZES, MLP_BATCH) / (mlp_ms * 1e-3) / 1e12, 2),
            "fp32_gemm": "bf16x3 split on bf16 MFMA, fp32 accumulate",
            "device": dev,
        },
        "roofline": {
            "kernel": "gemm_x3_rows_pk<6>: packed-A row-panel GEMM of GPT-2's qkv, attention-projection and fc "
                      "projections (bf16 hi/lo fragments of both operands, 8 wavefronts x 6 k-steps, whole K per "
                      "block), 36 launches per forward; all three shapes with their forward epilogues",
            "bound": "hbm",
            "achieved": round(p_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(p_gbs / HBM_PEAK_GBS, 4),
            "traffic": p_traffic,
            "avg_launch_ms": round(p_ms / len(shapes), 5),
            "shapes": shapes,
            "mfma_view": {
                "achieved_tflops_fp32_equiv": round(p_tflops, 2),
                "frac_fp32_peak": round(p_tflops / FP32_MFMA_PEAK_TFLOPS, 4),
                "bf16x3_ceiling_tflops": round(BF16X3_CEILING_TFLOPS, 1),
                "frac_bf16x3_ceiling": round(p_tflops / BF16X3_CEILING_TFLOPS, 4),
            },
            "timing": "per shape, a captured graph of 40 back-to-back launches over 40 weight sets (cold, as in "
                      "the forward), HIP events on the library stream; aggregate = bytes / time of one launch of "
                      "each shape (each runs 12 times per forward)",
            "traffic_source": os.path.relpath(PROJ_TRAFFIC_FILE, ROOT) if p_tinfo else None,
        },
        "roofline_mlp_dw": {
            "kernel": "W += -lr * g^T h (MLP weight gradient with its SGD step in the epilogue; M=4096 N=4096 "
                      "K=256, fp32 via bf16x3): pack_x3_pair + gemm_x3_outer_kernel<16>, plan " + plan.value.decode(),
            "bound": "hbm",
            "achieved": round(dw_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dw_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "avg_ms_both_launches": round(gemm_ms, 5),
            "algorithmic_bytes": dw_bytes,
            "mfma_view": {
                "achieved_tflops_fp32_equiv": round(achieved, 2),
                "frac_fp32_peak": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                "bf16_mfma_utilisation": round(3 * achieved / BF16_MFMA_PEAK_TFLOPS, 4),
                "frac_bf16x3_ceiling": round(achieved / BF16X3_CEILING_TFLOPS, 4),
            },
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if tinfo else None,
        },
    }
    if not args.no_cpu_baseline:
        print("bench: headline CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(wnp, params, ids, xnp, ynp)
    g_fwd.destroy()
    g_train.destroy()
    if not args.headline_only:
        # the other configs of BASELINE.json, each with its own roofline and
        # CPU baseline, as sub-records of the one line
        del model, mlp
        for name, fn in (("c5", c5_pipeline), ("c4", c4_generate), ("c1", c1_train)):
            print(f"bench: {name}", file=sys.stderr, flush=True)
            result[name] = fn(args)
    print(json.dumps(result), flush=True)


def kernel_suite(only=""):
    """One JSON line per HBM-bound hot-path kernel and for the C4/C5 shapes.

    Inputs rotate over enough buffers that every launch reads data not in
    the 256 MB Infinity Cache; each line is the HIP-event mean over
    back-to-back launches on the library stream, with algorithmic bytes
    (each input read once, each output written once) over 8 TB/s."""
    import applegpu_runtime as gpu  # noqa: F401
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib

    gpu.init_backend()
    rng = np.random.default_rng(0)

    def timed(fn, inputs, reps):
        for i in range(2):
            fn(inputs[i % len(inputs)])
        lib.applegpu_ffi_synchronize()
        lib.applegpu_ffi_event_record(0)
        out = None
        for i in range(reps):
            out = None
            out = fn(inputs[i % len(inputs)])
        lib.applegpu_ffi_event_record(1)
        return lib.applegpu_ffi_event_elapsed_ms(0, 1) / reps, out

    def line(name, shape, nbytes, ms, flop=None, peak_tflops=None):
        r = {"kernel": name, "shape": shape, "us": round(ms * 1e3, 2),
             "bytes": int(nbytes), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
             "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if flop:
            r["TFLOP/s"] = round(flop / (ms * 1e-3) / 1e12, 2)
            r["mfma_frac"] = round(flop / (ms * 1e-3) / 1e12 / peak_tflops, 4)
        print(json.dumps(r), flush=True)

    def randn(shape, dtype=np.float32, scale=1.0):
        return E.from_numpy((rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(dtype))

    def want(section):
        return not only or only in section

    if want("rows"):
        rows_section(timed, line, randn)
    if want("c5"):
        c5_section(timed, line, randn)
    if want("c4"):
        c4_section(timed, line, randn)
    if want("decode"):
        decode_section(timed, line, randn)
    if want("decode") or want("dattn"):
        decode_attention_line(timed, line, randn)


def rows_section(timed, line, randn):
    from applegpu_runtime import eager as E
    # row kernels at [262144, 768] fp32: 805 MB per read, two inputs rotate
    R, C = 262144, 768
    xs = [randn((R, C)) for _ in range(2)]
    g, b = randn((C,)), randn((C,))
    row_bytes = 2 * R * C * 4
    ms, _ = timed(lambda x: E.softmax(x), xs, 20)
    line("softmax", [R, C], row_bytes, ms)
    ms, _ = timed(lambda x: E.op("log_softmax", [x]), xs, 20)
    line("log_softmax", [R, C], row_bytes, ms)
    ms, _ = timed(lambda x: E.op("softmax_causal", [x]), xs, 20)
    line("softmax_causal", [R, C], row_bytes, ms)
    ms, _ = timed(lambda x: E.layer_norm(x, g, b), xs, 20)
    line("layer_norm", [R, C], row_bytes + 2 * C * 4, ms)
    ms, _ = timed(lambda x: E.gelu(x), xs, 20)
    line("gelu", [R, C], row_bytes, ms)
    ms, _ = timed(lambda x: E.add(x, xs[0]), xs[1:], 20)
    line("add", [R, C], 3 * R * C * 4, ms)
    del xs
    # fp16 rows at GPT-2 large's width (C4's layer_norm and attention softmax dtype)
    R, C = 262144, 1280
    xs = [randn((R, C), np.float16) for _ in range(2)]
    g, b = randn((C,), np.float16), randn((C,), np.float16)
    row_bytes = 2 * R * C * 2
    ms, _ = timed(lambda x: E.softmax(x), xs, 20)
    line("softmax_fp16", [R, C], row_bytes, ms)
    ms, _ = timed(lambda x: E.layer_norm(x, g, b), xs, 20)
    line("layer_norm_fp16", [R, C], row_bytes + 2 * C * 2, ms)
    del xs


def c5_section(timed, line, randn):
    from applegpu_runtime import eager as E
    # C5: per-row int8 quantize / dequantize of W [8192, 8192] fp32, three
    # rotating inputs
    N = 8192
    ws = [randn((N, N), scale=0.02) for _ in range(3)]
    qbytes = 4 * N * N + N * N + 4 * N
    ms, qs = timed(lambda w: E.op("quantize_per_row", [w], nout=2), ws, 12)
    line("quantize_per_row", [N, N], qbytes, ms)
    q, sc = qs
    # six code copies (6 x 64 MiB), so that dequantize reads them from HBM
    dq_in = [E.op("quantize_per_row", [ws[i % 3]], nout=2) for i in range(6)]
    ms, _ = timed(lambda qs_: E.op("dequantize_per_row", list(qs_)), dq_in, 12)
    del dq_in
    line("dequantize_per_row", [N, N], qbytes, ms)
    deq = E.op("dequantize_per_row", [q, sc])
    del ws
    X = randn((64, N))
    ms, _ = timed(lambda w: E.matmul_ex(X, w, False, True), [deq], 20)
    line("gemm_c5 x @ deq^T", [64, N, N], 4 * (64 * N + N * N + 64 * N), ms, 2.0 * 64 * N * N, FP32_MFMA_PEAK_TFLOPS)
    ms, _ = timed(lambda qq: E.op("linear_int8", [X, qq, sc]), [q], 20)
    line("linear_int8 x @ (q*s)^T", [64, N, N], 4 * 64 * N + N * N + 4 * N + 4 * 64 * N, ms, 2.0 * 64 * N * N,
         FP32_MFMA_PEAK_TFLOPS)
    del q, sc, deq, X


def c4_section(timed, line, randn):
    from applegpu_runtime import eager as E
    # C4 shapes, fp16: prefill GEMMs at 8 x 512 tokens and causal attention
    M, d = 4096, 1280
    a16 = [randn((M, d), np.float16)]
    w16 = randn((d, 3 * d), np.float16, 0.02)
    ms, _ = timed(lambda a: E.matmul(a, w16), a16, 20)
    line("gemm_c4_qkv f16", [M, 3 * d, d], 2 * (M * d + d * 3 * d + M * 3 * d), ms, 2.0 * M * 3 * d * d,
         BF16_MFMA_PEAK_TFLOPS)
    BH, T, hd = 160, 512, 64
    qkv = [randn((BH, T, hd), np.float16) for _ in range(3)]
    ms, _ = timed(lambda q: E.op("attention_causal", [q, qkv[1], qkv[2]]), [qkv[0]], 20)
    line("attention_causal f16", [BH, T, hd], 2 * 4 * BH * T * hd, ms, 4.0 * BH * T * T * hd / 2,
         BF16_MFMA_PEAK_TFLOPS)
    kc = [randn((BH, 640, hd), np.float16) for _ in range(2)]
    q1 = randn((BH, 1, hd), np.float16)
    ms, _ = timed(lambda k: E.op("attention", [q1, k, kc[1]]), [kc[0]], 20)
    line("attention decode f16 (q_len 1, ctx 640)", [BH, 640, hd], 2 * (2 * BH * 640 * hd + 2 * BH * hd), ms)


def decode_attention_line(timed, line, randn):
    """decode_attention at the C4 decode shape: 8 x 20 heads, one query row,
    contexts 513..640 (the average of the 128 steps, 576), fp16 cache of 640."""
    from applegpu_runtime import eager as E
    B, H, Tmax, D = 8, 20, 640, 64
    layers = 12   # rotating caches: 12 x 2 x 26 MB beyond the Infinity Cache
    kc = [randn((B, H, Tmax, D), np.float16) for _ in range(layers)]
    vc = [randn((B, H, Tmax, D), np.float16) for _ in range(layers)]
    q = randn((B, H, 1, D), np.float16)
    lens = E.from_numpy(np.full(B, 576, np.int32))
    ms, _ = timed(lambda i: E.op("decode_attention", [q, kc[i], vc[i], lens]), list(range(layers)), 4 * layers)
    mode = os.environ.get("APPLEGPU_DECODE_ATTN", "auto")
    line(f"decode_attention f16 ({mode}) B=8 H=20 ctx 576 of 640", [B, H, 576, D], 2 * B * H * 576 * D * 2, ms)


def decode_section(timed, line, randn):
    """C4 decode-step shapes: 8 token rows against GPT-2 large weights (fp16,
    stored k-major as the fp16 model keeps them), weights rotating over more
    than the 256 MB Infinity Cache; each shape through the skinny kernel and
    through the MFMA tiles."""
    import ctypes
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    M, d, V = 8, 1280, 50257
    for name, K, N, bk in [("qkv", d, 3 * d, True), ("proj", d, d, True), ("fc", d, 4 * d, True),
                           ("fc2", 4 * d, d, True), ("lm_head", d, V, True)]:
        copies = max(2, int(320e6 // (K * N * 2)) + 1)
        ws = [randn((N, K) if bk else (K, N), np.float16, 0.02) for _ in range(copies)]
        x = randn((M, K), np.float16)
        pks = [E.op("pack_weight", [w]) for w in ws]
        ms, _ = timed(lambda pk: E.op("matmul_packed", [x, pk], i=(N,)), pks, 4 * copies)
        line(f"gemm_decode {name} f16 M={M} (skinny, packed weights)", [M, K, N], 2 * (K * N + M * K + M * N),
             ms, 2.0 * M * N * K, BF16_MFMA_PEAK_TFLOPS)
        del pks
        for skinny in (1, 0):
            prev = lib.applegpu_ffi_gemm_skinny(skinny)
            plan = ctypes.create_string_buffer(96)
            lib.applegpu_ffi_gemm_plan(M, N, K, 1, 1, True, bk, plan, 96)
            ms, _ = timed(lambda w: E.matmul_ex(x, w, False, bk), ws, 4 * copies)
            lib.applegpu_ffi_gemm_skinny(prev)
            line(f"gemm_decode {name} f16 M={M} ({plan.value.decode()})", [M, K, N], 2 * (K * N + M * K + M * N),
                 ms, 2.0 * M * N * K, BF16_MFMA_PEAK_TFLOPS)
        del ws


C4_B, C4_T, C4_STEPS = 8, 512, 128


def c4_work(cfg, B, T, n):
    """Algorithmic work of config C4: prefill FLOPs (full-square attention
    count), and per decode step s (context T+1+s) FLOPs and HBM bytes (every
    fp16 weight read once, plus the K/V cache rows attended to)."""
    d, V, L, H = cfg["n_embd"], cfg["vocab_size"], cfg["n_layer"], cfg["n_head"]
    hd = d // H
    P = L * (d * 3 * d + d * d + 2 * d * 4 * d)
    Pl = V * d
    prefill = 2 * B * T * (P + Pl) + L * B * H * 2 * (2 * T * T * hd)
    flop = byts = 0
    for s in range(n):
        ctx = T + 1 + s
        flop += 2 * B * (P + Pl) + L * B * H * 2 * (2 * ctx * hd)
        byts += 2 * (P + Pl) + L * 2 * B * H * ctx * hd * 2
    return prefill, flop, byts


def c4_generate(args):
    """Config C4 end to end: GPT-2 large, fp16 weights and activations, random
    N(0,0.02) init (drawn in fp32, rounded to fp16), 8 prompts of 512 random
    ids, prefill then 128 greedy decode steps over a preallocated KV cache.
    The prefill and one decode step are each captured once as HIP graphs; a
    generation is one prefill replay and 128 decode replays (positions, the
    cache append and the argmax stay on the device).  Prints one JSON line."""
    import applegpu_runtime as gpu
    from applegpu_runtime._native import lib
    from applegpu_runtime.models import gpt2 as G

    gpu.init_backend()
    cfg = G.GPT2_CONFIGS["gpt2-large"]
    B, T, n = C4_B, C4_T, args.c4_steps
    print("c4: drawing and loading GPT-2 large fp16 weights", file=sys.stderr, flush=True)
    wnp = G.random_weights(cfg, seed=42)
    model = G.load_model(wnp, cfg, dtype="float16")
    ids = np.random.default_rng(42).integers(0, cfg["vocab_size"], (B, T)).astype(np.int32)
    gen = G.Generation(model, ids, n, capture=not args.c4_eager)
    print(f"c4: model and cache resident ({gen.cache.nbytes() / 1e9:.2f} GB cache)", file=sys.stderr, flush=True)

    # eager (op-by-op) timings for comparison: one prefill, a few steps
    lib.applegpu_ffi_synchronize()
    t0 = time.perf_counter()
    gen._prefill().eval()
    lib.applegpu_ffi_synchronize()
    prefill_eager_ms = 1e3 * (time.perf_counter() - t0)
    n_eager = min(8, n)
    t0 = time.perf_counter()
    for _ in range(n_eager):
        gen._step().eval()
    lib.applegpu_ffi_synchronize()
    step_eager_ms = 1e3 * (time.perf_counter() - t0) / n_eager

    def generation():
        gen.prefill()
        for s in range(n):
            gen.step(s)

    for _ in range(args.warmup if args.warmup > 0 else 1):
        generation()
    lib.applegpu_ffi_synchronize()
    reps = max(1, args.c4_reps)
    pre_ms = dec_ms = 0.0
    t0 = time.perf_counter()
    for _ in range(reps):
        lib.applegpu_ffi_event_record(0)
        gen.prefill()
        lib.applegpu_ffi_event_record(1)
        for s in range(n):
            gen.step(s)
        lib.applegpu_ffi_event_record(2)
        pre_ms += lib.applegpu_ffi_event_elapsed_ms(0, 1)
        dec_ms += lib.applegpu_ffi_event_elapsed_ms(1, 2)
    lib.applegpu_ffi_synchronize()
    wall_ms = 1e3 * (time.perf_counter() - t0) / reps
    pre_ms /= reps
    dec_ms /= reps
    toks = gen.out.to_numpy().T
    if not ((toks >= 0) & (toks < cfg["vocab_size"])).all():
        raise RuntimeError("generated ids out of range")

    pre_flop, dec_flop, dec_bytes = c4_work(cfg, B, T, n)
    step_traffic, step_tinfo = load_step_traffic()
    step_ms = dec_ms / n
    total_ms = pre_ms + dec_ms
    tok_s = B * (n + 1) / (total_ms * 1e-3)
    dec_gbs = dec_bytes / n / (step_ms * 1e-3) / 1e9
    result = {
        "metric": "C4 GPT-2 large fp16 greedy generation, tokens/s (8 prompts x 512 + 128 decode steps), 1 MI355X",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"C4 GPT-2 large (36x1280, 20 heads, vocab 50257) fp16, random N(0,0.02) weights, "
                        f"batch {B} prompts of {T} random ids, prefill + {n} greedy decode steps over a "
                        f"preallocated KV cache; prefill and decode step each replayed as captured HIP graphs",
            "prefill_ms": round(pre_ms, 3),
            "decode_ms_total": round(dec_ms, 3),
            "decode_ms_per_step": round(step_ms, 4),
            "generation_ms": round(total_ms, 3),
            "generation_wall_ms": round(wall_ms, 3),
            "decode_tokens_per_s": round(B * n / (dec_ms * 1e-3), 1),
            "prefill_tflops": round(pre_flop / (pre_ms * 1e-3) / 1e12, 1),
            "prefill_mfma_frac": round(pre_flop / (pre_ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
            "prefill_eager_ms": round(prefill_eager_ms, 3),
            "decode_step_eager_ms": round(step_eager_ms, 4),
            "kv_cache_gb": round(gen.cache.nbytes() / 1e9, 3),
            "launch_mode": "op-by-op" if args.c4_eager else "graph replay",
            "reps": reps,
        },
        "roofline": {
            "kernel": "whole decode step (all kernels of one graph replay)",
            "bound": "hbm",
            "achieved": round(dec_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
            "traffic": step_traffic,
            "traffic_context": step_tinfo["context"] if step_traffic else None,
            "traffic_ratio": step_tinfo["ratio"] if step_traffic else None,
            "traffic_note": "HBM bytes of one decode step at the context given (op-by-op launches of the same "
                            "kernels); it grows with the context at the K/V rows' rate, and traffic_ratio is its "
                            "ratio to that step's algorithmic bytes" if step_traffic else None,
            "traffic_source": os.path.relpath(C4_TRAFFIC_FILE, ROOT) if step_traffic else None,
            "bytes_per_step_avg": int(dec_bytes / n),
            "flop_per_step_avg": int(dec_flop / n),
        },
    }
    if not args.no_cpu_baseline:
        print("c4: CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = c4_cpu_baseline(wnp, cfg, ids, args.cpu_sample_s)
    gen.destroy()
    return result


def c4_cpu_baseline(wnp, cfg, ids, budget_s):
    """torch CPU eager generation on the fp16-rounded weights in fp32: one
    prefill of the same 8 x 512 prompts, then decode steps until ~budget_s;
    tokens/s projected to the same prefill + 128 steps."""
    import torch
    from oracle.torch_cpu import TorchGPT2Decoder
    w16 = {k: v.astype(np.float16).astype(np.float32) for k, v in wnp.items()}
    dec = TorchGPT2Decoder(w16, cfg)
    del w16
    B, T = ids.shape
    t0 = time.perf_counter()
    lg = dec.prefill(ids, T + C4_STEPS)
    pre_s = time.perf_counter() - t0
    tok = lg[:, -1].argmax(-1)
    k = 0
    t1 = time.perf_counter()
    while k < 2 or (time.perf_counter() - t0 < budget_s and k < C4_STEPS):
        tok = dec.decode(tok).argmax(-1)
        k += 1
    step_s = (time.perf_counter() - t1) / k
    total = pre_s + C4_STEPS * step_s
    return {
        "value": round(B * (C4_STEPS + 1) / total, 2),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "host": host_info(),
        "sample": f"torch {torch.__version__} CPU eager fp32 on fp16-rounded weights: prefill {B}x{T} "
                  f"{1e3 * pre_s:.0f} ms + {k} decode steps at {1e3 * step_s:.1f} ms/step, projected to "
                  f"{C4_STEPS} steps; host cpus {os.cpu_count()}",
    }


C1_SIZES, C1_BATCH = [64, 128, 10], 32


def _launcher_calls():
    import applegpu_runtime as gpu
    return gpu.graph_stats()["launcher_calls"]


def c1_train(args):
    """Config C1: Linear(64,128)-ReLU-Linear(128,10), batch 32, MSE, SGD lr
    0.01 (torch.manual_seed(42), then the default Linear init, then x and y
    from torch.randn, as python/tests/bench_comparison.py:23-28 seeds it).

    value: the fused C-ABI training step (EagerMLP.train_step: the whole
    step, forward, MSE loss and gradient, backward and both SGD steps, is
    one mlp2_sgd_step_ launch at this size) issued op by op, timed as the
    reference times its loop (bench_comparison.py:23-38: 5 warm-up steps,
    then the wall-clock mean of 50, synchronised after the last).  Also
    reported: the same step replayed as a captured HIP graph (a one-node
    graph adds its own launch cost to each replay, so it is slower here),
    and the reference's own route, the torch model on the PrivateUse1
    device with autograd and torch.optim.SGD.  kernels/step counts the
    kernel launchers one step calls."""
    import torch
    import applegpu_runtime as gpu
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    from applegpu_runtime.models.mlp import EagerMLP
    from applegpu_runtime.cpp_backend import fallback_count, load_cpp_backend

    gpu.init_backend()
    load_cpp_backend()

    def make():
        torch.manual_seed(42)
        m = torch.nn.Sequential(torch.nn.Linear(C1_SIZES[0], C1_SIZES[1]), torch.nn.ReLU(),
                                torch.nn.Linear(C1_SIZES[1], C1_SIZES[2]))
        x = torch.randn(C1_BATCH, C1_SIZES[0])
        y = torch.randn(C1_BATCH, C1_SIZES[2])
        return m, x, y

    m, xt, yt = make()
    params = [(m[0].weight.detach().numpy().copy(), m[0].bias.detach().numpy().copy()),
              (m[2].weight.detach().numpy().copy(), m[2].bias.detach().numpy().copy())]
    xnp, ynp = xt.numpy().copy(), yt.numpy().copy()
    warm, iters = max(args.warmup, 5), max(args.steps, 50)

    # C-ABI fused step: op by op, then one captured graph
    mlp = EagerMLP(params)
    x, y = E.from_numpy(xnp), E.from_numpy(ynp)
    for _ in range(warm):
        mlp.train_step(x, y, lr=0.01)
    lib.applegpu_ffi_synchronize()
    k0 = _launcher_calls()
    mlp.train_step(x, y, lr=0.01)
    kernels_fused = _launcher_calls() - k0
    lib.applegpu_ffi_synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        mlp.train_step(x, y, lr=0.01)
    lib.applegpu_ffi_synchronize()
    eager_ms = 1e3 * (time.perf_counter() - t0) / iters
    mlp_g = EagerMLP(params)
    g = gpu.capture(lambda: mlp_g.train_step(x, y, lr=0.01))
    for _ in range(warm):
        g.replay()
    lib.applegpu_ffi_synchronize()
    t0 = time.perf_counter()
    lib.applegpu_ffi_event_record(0)
    for _ in range(iters):
        g.replay()
    lib.applegpu_ffi_event_record(1)
    lib.applegpu_ffi_synchronize()
    graph_wall_ms = 1e3 * (time.perf_counter() - t0) / iters
    graph_ms = lib.applegpu_ffi_event_elapsed_ms(0, 1) / iters
    g.destroy()

    # the reference's route: torch autograd on the PrivateUse1 device
    md, xd, yd = make()
    md = md.to("applegpu")
    xd, yd = xd.to("applegpu"), yd.to("applegpu")
    opt = torch.optim.SGD(md.parameters(), lr=0.01)

    def torch_step():
        loss = torch.nn.functional.mse_loss(md(xd), yd)
        loss.backward()
        opt.step()
        opt.zero_grad()

    for _ in range(warm):
        torch_step()
    torch.applegpu.synchronize()
    f0, k0 = fallback_count(), _launcher_calls()
    torch_step()
    torch.applegpu.synchronize()
    kernels_torch = _launcher_calls() - k0
    t0 = time.perf_counter()
    for _ in range(iters):
        torch_step()
    torch.applegpu.synchronize()
    torch_ms = 1e3 * (time.perf_counter() - t0) / iters
    fallbacks = fallback_count() - f0

    flop = mlp_flops(C1_SIZES, C1_BATCH)  # forward, dW of both layers, dX of the second
    result = {
        "metric": "C1 MLP 64-128-10 train ms/step (batch 32, MSE, SGD), 1 MI355X",
        "value": round(eager_ms, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": iters,
        "warmup": warm,
        "ms_per_step": round(eager_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C1 Linear(64,128)-ReLU-Linear(128,10) fp32, batch 32, MSE, SGD lr 0.01; the fused "
                        "C-ABI training step issued op by op, wall-clock mean of 50 steps",
            "kernels_per_step": kernels_fused,
            "graph_replay_ms": round(graph_ms, 5),
            "graph_replay_wall_ms": round(graph_wall_ms, 5),
            "capi_op_by_op_ms": round(eager_ms, 5),
            "torch_privateuse1_ms": round(torch_ms, 5),
            "torch_privateuse1_kernels_per_step": kernels_torch,
            "torch_privateuse1_cpu_fallbacks": fallbacks,
            "flop_per_step": flop,
        },
        "roofline": {
            "kernel": "whole training step (launch-bound: 38 KB of parameters, 1.29 MFLOP)",
            "bound": "launch",
            "achieved": None, "peak": None, "unit": None, "frac": None, "traffic": None,
            "ms_per_kernel": round(eager_ms / max(kernels_fused, 1), 5),
        },
    }
    if not args.no_cpu_baseline:
        mc, xc, yc = make()
        oc = torch.optim.SGD(mc.parameters(), lr=0.01)

        def cpu_step():
            loss = torch.nn.functional.mse_loss(mc(xc), yc)
            loss.backward()
            oc.step()
            oc.zero_grad()

        for _ in range(5):
            cpu_step()
        times = []
        for _ in range(50):
            t0 = time.perf_counter()
            cpu_step()
            times.append(time.perf_counter() - t0)
        result["cpu_baseline"] = {
            "value": round(1e3 * float(np.median(times)), 5),
            "unit": "ms",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "host": host_info(),
            "sample": f"torch {torch.__version__} CPU eager, 5 warm-up + 50 timed steps (python/tests/"
                      f"bench_comparison.py:23-38), median; mean {1e3 * float(np.mean(times)):.4f} ms",
        }
    return result


def c5_pipeline(args):
    """Config C5: W [8192, 8192] fp32 ~ N(0, 0.02) and X [64, 8192] ~ N(0, 1)
    (seeded); per-row int8 quantize (scale = absmax(row)/127, round half to
    even), dequantize, and Y = X @ deq^T, each stage timed on its own with
    HIP events over back-to-back launches; W rotates over three copies
    (805 MB) so the HBM-bound stages read past the 256 MB Infinity Cache.
    value = the three stages' sum.  The int8 codes and scales are checked
    bit for bit against a numpy restatement outside the timed region, Y
    against the float64 product at the fp32 matmul bar."""
    import applegpu_runtime as gpu
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    gpu.init_backend()
    N, Mx = 8192, 64
    rng = np.random.default_rng(42)
    wnp = (rng.standard_normal((N, N), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    xnp = rng.standard_normal((Mx, N), dtype=np.float32)
    ws = [E.from_numpy(wnp)] + [E.from_numpy(rng.standard_normal((N, N), dtype=np.float32) * np.float32(0.02))
                                for _ in range(2)]
    X = E.from_numpy(xnp)
    reps = max(args.steps, 12)

    def timed(fn, inputs):
        for i in range(2):
            fn(inputs[i % len(inputs)])
        lib.applegpu_ffi_synchronize()
        lib.applegpu_ffi_event_record(0)
        out = None
        for i in range(reps):
            out = None
            out = fn(inputs[i % len(inputs)])
        lib.applegpu_ffi_event_record(1)
        return lib.applegpu_ffi_event_elapsed_ms(0, 1) / reps, out

    q_ms, _ = timed(lambda w: E.op("quantize_per_row", [w], nout=2), ws)
    q, sc = E.op("quantize_per_row", [ws[0]], nout=2)
    qs = [q] + [E.op("quantize_per_row", [w], nout=2)[0] for w in ws[1:]]
    scs = [sc] + [E.op("quantize_per_row", [w], nout=2)[1] for w in ws[1:]]
    # dequantize rotates over six code copies (6 x 64 MiB, more than the
    # 256 MB Infinity Cache), so that its reads come from HBM too
    dq_in = [(qs[i], scs[i]) for i in range(3)] + [E.op("quantize_per_row", [w], nout=2) for w in ws]
    d_ms, _ = timed(lambda i: E.op("dequantize_per_row", list(dq_in[i])), list(range(6)))
    del dq_in
    deq = E.op("dequantize_per_row", [q, sc])
    gemm_ms, y = timed(lambda w: E.matmul_ex(X, w, False, True), [deq])
    fused_ms, yf = timed(lambda i: E.op("linear_int8", [X, qs[i], scs[i]]), [0])
    lib.applegpu_ffi_synchronize()

    # parity outside the timed region
    amax = np.abs(wnp).max(axis=1)
    scale_ref = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q_ref = np.clip(np.rint(wnp / scale_ref[:, None]), -128, 127)
    q_ref = np.where(scale_ref[:, None] == 0, 0, q_ref).astype(np.int8)
    codes_exact = bool(np.array_equal(q.numpy(), q_ref)) and bool(np.array_equal(sc.numpy(), scale_ref))
    deq_ref = q_ref.astype(np.float32) * scale_ref[:, None]
    y_ref = xnp.astype(np.float64) @ deq_ref.T.astype(np.float64)
    y_err = float(np.abs(y.numpy() - y_ref).max() / np.abs(y_ref).max())
    yf_err = float(np.abs(yf.numpy() - y_ref).max() / np.abs(y_ref).max())
    if not codes_exact or y_err > 1e-3 or yf_err > 1e-3:
        raise RuntimeError(f"C5 parity failed: codes exact {codes_exact}, gemm err {y_err}, fused err {yf_err}")

    qbytes = 4 * N * N + N * N + 4 * N
    gemm_flop = 2.0 * Mx * N * N
    total_ms = q_ms + d_ms + gemm_ms
    q_gbs = qbytes / (q_ms * 1e-3) / 1e9
    q_traffic, _ = load_traffic(C5_TRAFFIC_FILE)
    result = {
        "metric": "C5 int8 per-row quantize + dequantize + [64,8192]x[8192,8192]^T GEMM, ms, 1 MI355X",
        "value": round(total_ms, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": reps,
        "warmup": 2,
        "ms_per_step": round(total_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32->i8->f32",
        "data": "synthetic",
        "config": {
            "workload": "C5 W [8192,8192] fp32 N(0,0.02), X [64,8192] N(0,1); per-row absmax/127 int8 "
                        "quantize (RNE), dequantize, X @ deq^T; three rotating W copies (six code copies for dequantize)",
            "quantize_us": round(q_ms * 1e3, 2),
            "quantize_hbm_frac": round(q_gbs / HBM_PEAK_GBS, 4),
            "dequantize_us": round(d_ms * 1e3, 2),
            "dequantize_hbm_frac": round(qbytes / (d_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "gemm_us": round(gemm_ms * 1e3, 2),
            "gemm_tflops": round(gemm_flop / (gemm_ms * 1e-3) / 1e12, 2),
            "gemm_fp32_mfma_frac": round(gemm_flop / (gemm_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "linear_int8_fused_us": round(fused_ms * 1e3, 2),
            "codes_bit_exact": codes_exact,
            "gemm_rel_err": y_err,
            "linear_int8_rel_err": yf_err,
        },
        "roofline": {
            "kernel": "quantize_per_row (row absmax, RNE int8 codes), [8192, 8192] fp32",
            "bound": "hbm",
            "achieved": round(q_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(q_gbs / HBM_PEAK_GBS, 4),
            "traffic": q_traffic,
            "traffic_source": os.path.relpath(C5_TRAFFIC_FILE, ROOT) if q_traffic else None,
            "bytes_per_launch": qbytes,
        },
    }
    if not args.no_cpu_baseline:
        import torch
        Wt, Xt = torch.from_numpy(wnp), torch.from_numpy(xnp)

        def stage(fn, n=3):
            fn()
            t0 = time.perf_counter()
            for _ in range(n):
                out = fn()
            return 1e3 * (time.perf_counter() - t0) / n, out

        sc_ms, sct = stage(lambda: Wt.abs().amax(1) / 127.0)
        qc_ms, qt = stage(lambda: torch.round(Wt / sct[:, None]).clamp(-128, 127).to(torch.int8))
        dc_ms, dt = stage(lambda: qt.float() * sct[:, None])
        gc_ms, _ = stage(lambda: Xt @ dt.T)
        result["cpu_baseline"] = {
            "value": round(sc_ms + qc_ms + dc_ms + gc_ms, 3),
            "unit": "ms",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "host": host_info(),
            "sample": f"torch {torch.__version__} CPU eager, the same expressions, 3 timed runs per "
                      f"stage after one warm-up: scale {sc_ms:.1f} ms, quantize {qc_ms:.1f} ms, dequantize "
                      f"{dc_ms:.1f} ms, GEMM {gc_ms:.1f} ms",
        }
    return result


def host_info():
    """The CPU-baseline host: lscpu model name and core counts, the CPUs this
    process may run on, and the threads torch uses."""
    import subprocess
    import torch
    info = {"cpu_model": None, "sockets": None, "physical_cores": None, "logical_cpus": os.cpu_count(),
            "cpus_allowed": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "torch_threads": torch.get_num_threads(), "torch": torch.__version__}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            kv[k.strip()] = v.strip()
        info["cpu_model"] = kv.get("Model name")
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets or None
        info["physical_cores"] = sockets * per or None
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    return info


def cpu_baseline(wnp, params, ids, xnp, ynp):
    """The reference's CPU path (PyTorch CPU eager) on the same workload, as
    its benchmarks time it: GPT-2 forward under no_grad, 3 warm-up + 20
    timed forwards, median; MLP train step, 5 warm-up + 50 timed steps
    (python/tests/bench_comparison.py:23-38), median (the mean is reported
    beside it).  value = the two medians' sum."""
    import torch
    from oracle.torch_cpu import TorchGPT2, TorchMLP
    g = TorchGPT2(wnp, GPT2_CFG)
    m = TorchMLP(params, lr=0.01)
    tx, ty = torch.from_numpy(xnp), torch.from_numpy(ynp)

    def times(fn, warm, n):
        for _ in range(warm):
            fn()
        out = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            out.append(time.perf_counter() - t0)
        return np.array(out) * 1e3

    tg = times(lambda: g.forward(ids), 3, 20)
    tm = times(lambda: m.step(tx, ty), 5, 50)
    return {
        "value": round(float(np.median(tg) + np.median(tm)), 3),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "host": host_info(),
        "gpt2_fwd_ms_median": round(float(np.median(tg)), 3),
        "mlp_train_ms_median": round(float(np.median(tm)), 3),
        "sample": f"torch {torch.__version__} CPU eager: GPT-2 small fwd seq128 under no_grad, 3 warm-up + 20 "
                  f"timed, median {np.median(tg):.1f} ms (mean {tg.mean():.1f}); MLP 4096 train step, 5 warm-up + "
                  f"50 timed, median {np.median(tm):.1f} ms (mean {tm.mean():.1f}); host cpus {os.cpu_count()}",
    }


if __name__ == "__main__":
    main()
