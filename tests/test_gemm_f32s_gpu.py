"""fp32 products with few rows and large fp32 weights (config C5's
X [64, 8192] @ deq [8192, 8192]^T): the weight-streaming plan
(kernels/gemm_f32s.hip: every weight byte read once into registers and split
there into bf16 hi/lo, K split into ranges summed by the split-K reduction)
against the float64 oracle at the fp32 matmul bar (checked at 1e-4), with
the epilogue the reduction applies, one and two row strips with ragged row
counts, repeat launches bit for bit, and the shapes it leaves to the tiled
kernels.  The reference computes these products with
MPSMatrixMultiplication (swift/Sources/AppleGPUBridge/compute.swift:1544-1630)."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err
from oracle import ops as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(5150)


def f32(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def _plan(M, N, K):
    from applegpu_runtime._native import lib
    buf = ctypes.create_string_buffer(96)
    assert lib.applegpu_ffi_gemm_plan(M, N, K, 1, 0, True, True, buf, 96) == 0
    return buf.value.decode()


@pytest.mark.parametrize("M,N,K", [(64, 8192, 8192), (37, 2048, 4096), (20, 1024, 8192), (2, 4096, 2048),
                                   (33, 256, 32768)])
def test_stream_plan_matches_oracle(gpu, M, N, K):
    from applegpu_runtime import eager as E
    assert _plan(M, N, K).startswith("f32 stream"), _plan(M, N, K)
    x, w = f32(M, K), f32(N, K, scale=0.02)
    xt, wt = E.from_numpy(x), E.from_numpy(w)
    y = E.matmul_ex(xt, wt, False, True).numpy()
    assert rel_err(y, O.matmul(x, w.T)) < 1e-4
    np.testing.assert_array_equal(y, E.matmul_ex(xt, wt, False, True).numpy())


def test_stream_plan_epilogue(gpu):
    """Linear with bias and ReLU (addmm + relu) on the streaming plan: the
    split-K reduction applies the epilogue after summing the K ranges."""
    from applegpu_runtime import eager as E
    M, N, K = 48, 4096, 4096
    assert _plan(M, N, K).startswith("f32 stream")
    x, w, b = f32(M, K), f32(N, K, scale=0.02), f32(N, scale=0.1)
    y = E.linear(E.from_numpy(x), E.from_numpy(w), E.from_numpy(b), act=1).numpy()
    ref = np.maximum(O.matmul(x, w.T) + b.astype(np.float64), 0.0)
    assert rel_err(y, ref) < 1e-4
    assert (y[ref == 0.0] == 0.0).all()


def test_stream_plan_exact_on_small_integers(gpu):
    """Small-integer operands are exact in bf16 hi alone: the product is the
    exact integer result."""
    from applegpu_runtime import eager as E
    M, N, K = 64, 2048, 4096
    x = RNG.integers(-3, 4, (M, K)).astype(np.float32)
    w = RNG.integers(-3, 4, (N, K)).astype(np.float32)
    y = E.matmul_ex(E.from_numpy(x), E.from_numpy(w), False, True).numpy()
    np.testing.assert_array_equal(y, x @ w.T)


@pytest.mark.parametrize("M,N,K", [(65, 8192, 8192), (64, 8000, 8192), (64, 8192, 8000), (64, 512, 512),
                                   (1, 8192, 8192)])
def test_stream_plan_declines(gpu, M, N, K):
    """More than 64 rows, columns not a multiple of 256, K not a multiple of
    256, small weights, or one row: another plan."""
    assert not _plan(M, N, K).startswith("f32 stream"), _plan(M, N, K)
