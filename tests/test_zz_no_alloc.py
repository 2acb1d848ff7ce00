"""The allocation-free linear entry point against the allocating one, through
the C ABI: the same kernels on the same inputs give the same bits.  Two
calls in a row (the second smaller) share the static scratch array; a
product whose split-K partials would not fit in it is rejected, and one whose
default plan's packed operands would not fit takes a plan that does."""
import ctypes
from ctypes import c_uint64

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(9090)


@pytest.fixture(scope="module")
def lib():
    import applegpu_runtime as gpu
    from applegpu_runtime._native import lib as L
    gpu.init_backend()
    assert L.applegpu_eager_init()
    return L


def _alloc(lib, shape, arr=None):
    dims = (c_uint64 * len(shape))(*shape)
    oid = c_uint64()
    assert lib.applegpu_eager_alloc(dims, len(shape), 0, ctypes.byref(oid))
    if arr is not None:
        a = np.ascontiguousarray(arr, np.float32)
        assert lib.applegpu_eager_copy_from_host(oid.value, a.ctypes.data, a.nbytes) == 0
    return oid.value


def _read(lib, tid, shape):
    out = np.empty(shape, np.float32)
    assert lib.applegpu_eager_copy_to_host(tid, out.ctypes.data, out.nbytes) == 0, lib.applegpu_eager_last_error()
    return out


def _plan(lib, M, N, K):
    buf = ctypes.create_string_buffer(96)
    lib.applegpu_ffi_gemm_plan(M, N, K, 1, 0, True, True, buf, 96)
    return buf.value.decode()


def _case(lib, M, K, N, act, with_bias):
    x = _alloc(lib, (M, K), RNG.standard_normal((M, K)))
    w = _alloc(lib, (N, K), RNG.standard_normal((N, K)) * 0.05)
    b = _alloc(lib, (N,), RNG.standard_normal(N)) if with_bias else 0
    want_id = c_uint64()
    assert lib.applegpu_eager_linear(x, w, b, act, ctypes.byref(want_id)), lib.applegpu_eager_last_error()
    out = _alloc(lib, (M, N))
    rc = lib.applegpu_eager_linear_noalloc(x, w, b, act, out)
    assert rc == 0, lib.applegpu_eager_last_error()
    lib.applegpu_eager_flush_and_wait()
    got, want = _read(lib, out, (M, N)), _read(lib, want_id.value, (M, N))
    for t in (x, w, out, want_id.value) + ((b,) if b else ()):
        lib.applegpu_eager_free(t)
    return got, want


@pytest.mark.parametrize("first,second", [
    ((256, 4096, 4096, 1, True), (128, 768, 768, 0, True)),   # 8-way then 4-way split K
    ((128, 3072, 768, 2, True), (33, 200, 70, 3, False)),     # split K, then a ragged unsplit shape
])
def test_noalloc_matches_linear_two_calls(lib, first, second):
    print(f"noalloc linear: {first} then {second}", flush=True)
    assert "splits=1" not in _plan(lib, first[0], first[2], first[1])
    for M, K, N, act, bias in (first, second):
        got, want = _case(lib, M, K, N, act, bias)
        np.testing.assert_array_equal(got, want)
        assert np.isfinite(got).all()


def test_noalloc_outer_shaped_product_takes_a_plan_that_fits(lib):
    """x [32768, 512] @ w [1024, 512]^T: the allocating linear takes the
    outer-product plan, whose packed operands ((M + N) K fp32 = 69 MB) would
    not fit the 64 MiB scratch; the allocation-free call takes a plan that
    fits and agrees with it (and with float64) at the fp32 GEMM bar.  Run
    twice, the second call smaller, as the other cases."""
    assert _plan(lib, 32768, 1024, 512).startswith("x3 outer")
    for M, K, N in ((32768, 512, 1024), (4096, 512, 512)):
        print(f"noalloc linear, outer-shaped: M={M} K={K} N={N}", flush=True)
        xa = RNG.standard_normal((M, K)).astype(np.float32)
        wa = (RNG.standard_normal((N, K)) * 0.05).astype(np.float32)
        ba = RNG.standard_normal(N).astype(np.float32)
        x, w, b = _alloc(lib, (M, K), xa), _alloc(lib, (N, K), wa), _alloc(lib, (N,), ba)
        want_id = c_uint64()
        assert lib.applegpu_eager_linear(x, w, b, 1, ctypes.byref(want_id)), lib.applegpu_eager_last_error()
        out = _alloc(lib, (M, N))
        rc = lib.applegpu_eager_linear_noalloc(x, w, b, 1, out)
        assert rc == 0, lib.applegpu_eager_last_error()
        lib.applegpu_eager_flush_and_wait()
        got, want = _read(lib, out, (M, N)), _read(lib, want_id.value, (M, N))
        ref = np.maximum(xa.astype(np.float64) @ wa.astype(np.float64).T + ba, 0)
        scale = np.abs(ref).max()
        assert np.abs(got - ref).max() / scale < 1e-4
        assert np.abs(got - want).max() / scale < 1e-4
        for t in (x, w, b, out, want_id.value):
            lib.applegpu_eager_free(t)


def test_noalloc_rejects_oversized_workspace_and_bad_operands(lib):
    M, K, N = 1024, 4096, 4096
    x = _alloc(lib, (M, K), np.ones((M, K), np.float32))
    w = _alloc(lib, (N, K), np.ones((N, K), np.float32))
    out = _alloc(lib, (M, N))
    # 8 forced splits of 1024 x 4096 fp32 partials: 128 MiB, past the 64 MiB array
    assert lib.applegpu_ffi_gemm_tune(0, -1, 8) == 0
    try:
        assert lib.applegpu_eager_linear_noalloc(x, w, 0, 0, out) == -1
        assert b"workspace" in lib.applegpu_eager_last_error()
    finally:
        assert lib.applegpu_ffi_gemm_tune(0, -1, 0) == 0
    # the output may not alias an input, and must have the product's shape
    assert lib.applegpu_eager_linear_noalloc(x, w, 0, 0, x) == -1
    small = _alloc(lib, (M, N - 1))
    assert lib.applegpu_eager_linear_noalloc(x, w, 0, 0, small) == -1
    assert lib.applegpu_eager_linear_noalloc(x, w, 0, 7, out) == -1
    # unforced, the same product fits and runs
    assert lib.applegpu_eager_linear_noalloc(x, w, 0, 0, out) == 0, lib.applegpu_eager_last_error()
    lib.applegpu_eager_flush_and_wait()
    np.testing.assert_array_equal(_read(lib, out, (M, N))[:2, :3], np.full((2, 3), K, np.float32))
    for t in (x, w, out, small):
        lib.applegpu_eager_free(t)
