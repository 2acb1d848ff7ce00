"""Benchmark of the MI355X backend on BASELINE.json's headline metric:
GPT-2-small forward ms at seq 128 (config 2) + MLP h=4096 train ms/step
(config 3), on one MI355X, with the roofline fraction of the dominant kernel.

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

Roofline: the dominant single kernel of the step, the MLP weight-gradient
GEMM dW = g^T h (M = N = 4096, K = 256; fp32 operands split into bf16 hi/lo,
three bf16 MFMAs per product), timed with HIP events on the library stream
over back-to-back launches; algorithmic work 2*M*N*K flop per launch.  Its
HBM traffic comes from the rocprofv3 --pmc summaries committed under
profiles/ (FETCH_SIZE, WRITE_SIZE of that kernel, scaled by the same counters
read for the 256 MiB calibration copy this script runs), when present.

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
BF16_MFMA_PEAK_TFLOPS = 2516.6
HBM_PEAK_GBS = 8000.0
GPT2_CFG = dict(n_layer=12, n_head=12, n_embd=768, vocab_size=50257, n_positions=1024)
MLP_SIZES = [4096, 4096, 4096, 1]
MLP_BATCH = 256
SEQ = 128
CALIB_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mlp_dw_gemm_traffic.json")


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


def load_traffic():
    """HBM bytes per launch of the roofline kernel from the committed PMC summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return float(t["bytes_per_launch"]), t
    except (OSError, KeyError, ValueError):
        return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-s", type=float, default=15.0)
    ap.add_argument("--suite", action="store_true",
                    help="instead of the headline line, print one JSON line per hot-path kernel "
                         "(cache-busting working sets, roofline fractions)")
    ap.add_argument("--only", default="",
                    help="with --suite: run only the sections whose name contains this text "
                         "(rows, c5, c4, decode)")
    ap.add_argument("--c4", action="store_true",
                    help="instead of the headline line, run config C4 (GPT-2 large fp16 prefill + greedy "
                         "decode over a KV cache) and print its JSON line")
    ap.add_argument("--c4-steps", type=int, default=C4_STEPS)
    ap.add_argument("--c4-reps", type=int, default=3)
    ap.add_argument("--c4-eager", action="store_true",
                    help="C4 with op-by-op launches instead of graph replays (same kernels; for kernel traces)")
    args = ap.parse_args()
    if args.suite:
        kernel_suite(args.only)
        return
    if args.c4:
        c4_generate(args)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is designed, not built).", file=sys.stderr)
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

    # ── roofline: the MLP weight-gradient GEMM with its SGD update, as the
    # step runs it: W += -lr * g^T h (bias-free; W a scratch copy) ──────────
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
    import ctypes
    plan = ctypes.create_string_buffer(96)
    lib.applegpu_ffi_gemm_plan(M_, N_, K_, 1, 0, False, False, plan, 96)
    traffic, tinfo = load_traffic()

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
            "kernel": "gemm_mf W += -lr * g^T h (MLP weight gradient with its SGD step in the epilogue; "
                      "M=4096 N=4096 K=256, fp32 via bf16x3), plan " + plan.value.decode(),
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "avg_launch_ms": round(gemm_ms, 5),
            "flop_per_launch": gemm_flop,
            "bf16_mfma_utilisation": round(3 * achieved / BF16_MFMA_PEAK_TFLOPS, 4),
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if tinfo else None,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wnp, params, ids, xnp, ynp, args.cpu_sample_s)
    g_fwd.destroy()
    g_train.destroy()
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


def c5_section(timed, line, randn):
    from applegpu_runtime import eager as E
    # C5: per-row int8 quantize / dequantize of W [8192, 8192] fp32, three rotating inputs
    N = 8192
    ws = [randn((N, N), scale=0.02) for _ in range(3)]
    qbytes = 4 * N * N + N * N + 4 * N
    ms, qs = timed(lambda w: E.op("quantize_per_row", [w], nout=2), ws, 12)
    line("quantize_per_row", [N, N], qbytes, ms)
    q, sc = qs
    ms, _ = timed(lambda qq: E.op("dequantize_per_row", [qq, sc]), [q], 12)
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
    wnp = G.random_weights(cfg, seed=42)
    model = G.load_model(wnp, cfg, dtype="float16")
    ids = np.random.default_rng(42).integers(0, cfg["vocab_size"], (B, T)).astype(np.int32)
    ids_dev = gpu.from_numpy(ids)
    pos_dev = gpu.from_numpy(np.tile(np.arange(T, dtype=np.int32), B))
    cache = G.KVCache(cfg, B, T + n, "float16")
    zeros_b = gpu.from_numpy(np.zeros(B, np.int32))
    t_b = gpu.from_numpy(np.full(B, T, np.int32))
    tokens = gpu.zeros([B], "int32")
    out = gpu.zeros([n + 1, B], "int32")
    print(f"c4: model and cache resident ({cache.nbytes() / 1e9:.2f} GB cache)", file=sys.stderr, flush=True)

    def prefill():
        gpu.blit_copy(zeros_b, cache.pos)
        lg, nxt = G.gpt2_prefill(model, ids_dev, cache, positions=pos_dev)
        gpu.blit_copy(nxt, tokens)
        gpu.blit_copy(t_b, cache.pos)
        return lg

    def step():
        lg, nx, lens = G.gpt2_decode_step(model, tokens, cache)
        gpu.blit_copy(nx, tokens)
        gpu.blit_copy(lens, cache.pos)
        return lg

    # eager (op-by-op) timings for comparison: one prefill, a few steps
    lib.applegpu_ffi_synchronize()
    t0 = time.perf_counter()
    prefill().eval()
    lib.applegpu_ffi_synchronize()
    prefill_eager_ms = 1e3 * (time.perf_counter() - t0)
    n_eager = min(8, n)
    t0 = time.perf_counter()
    for _ in range(n_eager):
        step().eval()
    lib.applegpu_ffi_synchronize()
    step_eager_ms = 1e3 * (time.perf_counter() - t0) / n_eager

    if args.c4_eager:
        # the same kernels issued op by op (for kernel traces of the step)
        g_pre = g_step = None
        run_pre = lambda: prefill().eval()  # noqa: E731
        run_step = lambda: step().eval()  # noqa: E731
    else:
        g_pre = gpu.capture(prefill)
        g_step = gpu.capture(step)
        run_pre, run_step = g_pre.replay, g_step.replay
    slots = [gpu.slice(out, 0, s, s + 1) for s in range(n + 1)]

    def generation():
        run_pre()
        gpu.blit_copy(tokens, slots[0])
        for s in range(n):
            run_step()
            gpu.blit_copy(tokens, slots[s + 1])

    for _ in range(args.warmup if args.warmup > 0 else 1):
        generation()
    lib.applegpu_ffi_synchronize()
    reps = max(1, args.c4_reps)
    pre_ms = dec_ms = 0.0
    t0 = time.perf_counter()
    for _ in range(reps):
        lib.applegpu_ffi_event_record(0)
        run_pre()
        gpu.blit_copy(tokens, slots[0])
        lib.applegpu_ffi_event_record(1)
        for s in range(n):
            run_step()
            gpu.blit_copy(tokens, slots[s + 1])
        lib.applegpu_ffi_event_record(2)
        pre_ms += lib.applegpu_ffi_event_elapsed_ms(0, 1)
        dec_ms += lib.applegpu_ffi_event_elapsed_ms(1, 2)
    lib.applegpu_ffi_synchronize()
    wall_ms = 1e3 * (time.perf_counter() - t0) / reps
    pre_ms /= reps
    dec_ms /= reps
    toks = out.to_numpy().T
    if not ((toks >= 0) & (toks < cfg["vocab_size"])).all():
        raise RuntimeError("generated ids out of range")

    pre_flop, dec_flop, dec_bytes = c4_work(cfg, B, T, n)
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
            "kv_cache_gb": round(cache.nbytes() / 1e9, 3),
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
            "traffic": None,
            "bytes_per_step_avg": int(dec_bytes / n),
            "flop_per_step_avg": int(dec_flop / n),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = c4_cpu_baseline(wnp, cfg, ids, args.cpu_sample_s)
    if g_pre is not None:
        g_pre.destroy()
        g_step.destroy()
    print(json.dumps(result), flush=True)


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
        "sample": f"torch {torch.__version__} CPU eager fp32 on fp16-rounded weights: prefill {B}x{T} "
                  f"{1e3 * pre_s:.0f} ms + {k} decode steps at {1e3 * step_s:.1f} ms/step, projected to "
                  f"{C4_STEPS} steps; host cpus {os.cpu_count()}",
    }


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
