"""Every GEMM tile configuration, split count and operand layout against a
float64 host reference (fp32 GEMM bar 1e-3; bf16x3 sits near 5e-6, checked
at 1e-4), on shapes that take the unmasked fast loads (K % 4 == 0) and on
shapes that take the masked path.  Each product is computed twice in a row:
repeated launches must agree and the result must be
bit-identical (the partial sums are added in split order)."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

N_CFG = 11


@pytest.fixture
def tune(gpu):
    from applegpu_runtime._native import lib
    yield lib
    lib.applegpu_ffi_gemm_tune(0, -1, 0)


def _operands(rng, M, N, K, ta, tb):
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    ref = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    return a, b, ref


@pytest.mark.parametrize("M,N,K", [(100, 136, 320), (70, 50, 318), (130, 260, 1024)])
def test_every_config_split_and_layout(tune, M, N, K):
    from applegpu_runtime import eager as E
    rng = np.random.default_rng(M * 7 + K)
    for ta in (False, True):
        for tb in (False, True):
            a, b, ref = _operands(rng, M, N, K, ta, tb)
            ga, gb = E.from_numpy(a), E.from_numpy(b)
            for cfg in range(N_CFG):
                for splits in (1, 2, 4, 8):
                    assert tune.applegpu_ffi_gemm_tune(0, cfg, splits) == 0
                    r1 = E.matmul_ex(ga, gb, ta, tb).numpy()
                    r2 = E.matmul_ex(ga, gb, ta, tb).numpy()
                    err = rel_err(r1, ref)
                    assert err < 1e-4, (ta, tb, cfg, splits, err)
                    assert np.array_equal(r1, r2), (ta, tb, cfg, splits)


def test_native_fp32_mode(tune):
    from applegpu_runtime import eager as E
    rng = np.random.default_rng(5)
    a, b, ref = _operands(rng, 200, 300, 500, False, True)
    assert tune.applegpu_ffi_gemm_tune(1, -1, 0) == 0
    got = E.matmul_ex(E.from_numpy(a), E.from_numpy(b), False, True).numpy()
    assert rel_err(got, ref) < 1e-5


def test_split_k_with_fused_epilogue(tune):
    """bias + gelu + residual applied once, after the split partials are summed."""
    import applegpu_runtime as gpu
    rng = np.random.default_rng(9)
    x = rng.standard_normal((128, 768)).astype(np.float32)
    w = (rng.standard_normal((768, 768)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(768).astype(np.float32)
    res = rng.standard_normal((128, 768)).astype(np.float32)
    pre = x.astype(np.float64) @ w + bias
    gel = 0.5 * pre * (1 + np.tanh(np.sqrt(2 / np.pi) * (pre + 0.044715 * pre ** 3)))
    want = gel + res
    for splits in (2, 4, 8):
        assert tune.applegpu_ffi_gemm_tune(0, 6, splits) == 0
        t = gpu.from_numpy(res) + gpu.gelu(gpu.add_bias(gpu.from_numpy(x) @ gpu.from_numpy(w), gpu.from_numpy(bias)))
        assert rel_err(t.to_numpy(), want) < 1e-4


def test_tune_rejects_bad_values(tune):
    assert tune.applegpu_ffi_gemm_tune(2, -1, 0) == -1
    assert tune.applegpu_ffi_gemm_tune(0, N_CFG, 0) == -1
    assert tune.applegpu_ffi_gemm_tune(0, -1, 65) == -1
    buf = ctypes.create_string_buffer(96)
    assert tune.applegpu_ffi_gemm_plan(256, 4096, 4096, 1, 0, True, True, buf, 96) == 0
    assert buf.value.startswith(b"mf")
