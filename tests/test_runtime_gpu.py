"""Runtime semantics through the reference's C ABI (eager and graph paths):
ids, views, pool reuse, error conventions, *_out ops, readback, flush.
Mirrors crates/core/tests/eager_integration.rs and backend_ffi_integration.rs."""
import ctypes
from ctypes import c_float, c_uint32, c_uint64

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib(gpu):
    from applegpu_runtime._native import lib as L
    assert L.applegpu_eager_init()
    return L


def alloc(lib, arr):
    arr = np.ascontiguousarray(arr)
    dims = (c_uint64 * arr.ndim)(*arr.shape)
    oid = c_uint64()
    code = {np.float32: 0, np.int32: 5, np.float16: 1}[arr.dtype.type]
    p = lib.applegpu_eager_alloc(dims, arr.ndim, code, ctypes.byref(oid))
    assert p and oid.value > 0
    assert lib.applegpu_eager_copy_from_host(oid.value, arr.ctypes.data, arr.nbytes) == 0
    return oid.value, p


def read(lib, tid, shape, dtype=np.float32):
    out = np.empty(shape, dtype)
    assert lib.applegpu_eager_copy_to_host(tid, out.ctypes.data, out.nbytes) == 0, lib.applegpu_eager_last_error()
    return out


def test_eager_add_broadcast_and_shape(lib):
    # eager_integration.rs:41-64 style: [2,3] + [3]
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([10, 20, 30], np.float32)
    ia, _ = alloc(lib, a)
    ib, _ = alloc(lib, b)
    out = c_uint64()
    p = lib.applegpu_eager_add(ia, ib, ctypes.byref(out))
    assert p
    dims = (c_uint64 * 8)()
    nd = c_uint32()
    assert lib.applegpu_eager_shape(out.value, dims, ctypes.byref(nd)) == 0
    assert [dims[i] for i in range(nd.value)] == [2, 3]
    assert lib.applegpu_eager_dtype(out.value) == 0
    lib.applegpu_eager_flush_and_wait()
    np.testing.assert_array_equal(read(lib, out.value, (2, 3)), a + b)
    assert lib.applegpu_eager_find_by_data_ptr(p) == out.value


def test_eager_views_share_storage_and_offsets(lib):
    base = np.arange(24, dtype=np.float32).reshape(4, 6)
    ib, _ = alloc(lib, base)
    # transpose view
    vid = c_uint64()
    shp = (c_uint64 * 2)(6, 4)
    st = (c_uint64 * 2)(1, 6)
    assert lib.applegpu_eager_create_view(ib, shp, st, 2, 0, ctypes.byref(vid))
    np.testing.assert_array_equal(read(lib, vid.value, (6, 4)), base.T)
    # offset view: rows 1..3, cols 2..5
    vid2 = c_uint64()
    shp2 = (c_uint64 * 2)(2, 3)
    st2 = (c_uint64 * 2)(6, 1)
    assert lib.applegpu_eager_create_view(ib, shp2, st2, 2, 8, ctypes.byref(vid2))
    np.testing.assert_array_equal(read(lib, vid2.value, (2, 3)), base[1:3, 2:5])
    # unary on the offset view honours the byte offset (reference quirk fixed)
    out = c_uint64()
    assert lib.applegpu_eager_neg(vid2.value, ctypes.byref(out))
    np.testing.assert_array_equal(read(lib, out.value, (2, 3)), -base[1:3, 2:5])
    # out-of-bounds view is rejected
    bad = c_uint64()
    shp3 = (c_uint64 * 2)(5, 6)
    assert not lib.applegpu_eager_create_view(ib, shp3, st2, 2, 0, ctypes.byref(bad))
    assert b"exceeds" in lib.applegpu_eager_last_error()


def test_eager_inplace_and_errors(lib):
    p = np.ones((3, 4), np.float32)
    g = np.full((3, 4), 2.0, np.float32)
    ip, _ = alloc(lib, p)
    ig, _ = alloc(lib, g)
    assert lib.applegpu_eager_add_scaled_inplace(ip, ig, -0.25) == 0
    np.testing.assert_array_equal(read(lib, ip, (3, 4)), p - 0.5)
    assert lib.applegpu_eager_add_inplace(ip, ig) == 0
    np.testing.assert_array_equal(read(lib, ip, (3, 4)), p + 1.5)
    # in-place on a non-contiguous view is an error (eager.rs:626-630)
    vid = c_uint64()
    shp = (c_uint64 * 2)(4, 3)
    st = (c_uint64 * 2)(1, 4)
    assert lib.applegpu_eager_create_view(ip, shp, st, 2, 0, ctypes.byref(vid))
    assert lib.applegpu_eager_add_inplace(vid.value, vid.value) == -1
    assert b"non-contiguous" in lib.applegpu_eager_last_error()
    # unknown id
    out = c_uint64(12345)
    assert not lib.applegpu_eager_relu(10 ** 12, ctypes.byref(out))
    assert out.value == 12345  # *out_id written only on success
    assert b"not found" in lib.applegpu_eager_last_error()
    assert lib.applegpu_eager_dtype(10 ** 12) == -1
    # dtype mismatch
    ii, _ = alloc(lib, np.ones((3, 4), np.int32))
    assert not lib.applegpu_eager_add(ip, ii, ctypes.byref(out))
    assert b"mismatch" in lib.applegpu_eager_last_error().lower()
    # invalid dtype wire code
    dims = (c_uint64 * 1)(4)
    assert not lib.applegpu_eager_alloc(dims, 1, 42, ctypes.byref(out))
    assert b"dtype" in lib.applegpu_eager_last_error()


def test_eager_matmul_ex_and_sum_dim(lib):
    x = np.random.default_rng(0).standard_normal((32, 64)).astype(np.float32)
    g = np.random.default_rng(1).standard_normal((32, 16)).astype(np.float32)
    ix, _ = alloc(lib, x)
    ig, _ = alloc(lib, g)
    out = c_uint64()
    assert lib.applegpu_eager_matmul_ex(ig, ix, True, False, ctypes.byref(out))
    np.testing.assert_allclose(read(lib, out.value, (16, 64)), g.T @ x, rtol=1e-4, atol=1e-4)
    s = c_uint64()
    assert lib.applegpu_eager_sum_dim(ig, 0, False, ctypes.byref(s))
    np.testing.assert_allclose(read(lib, s.value, (16,)), g.sum(0), rtol=1e-5, atol=1e-5)
    s2 = c_uint64()
    assert lib.applegpu_eager_sum_dim(ig, -1, True, ctypes.byref(s2))
    np.testing.assert_allclose(read(lib, s2.value, (32, 1)), g.sum(1, keepdims=True), rtol=1e-5, atol=1e-5)


def test_eager_mean_all_threshold_scalar(lib):
    x = np.random.default_rng(2).standard_normal((7, 9)).astype(np.float32)
    ix, _ = alloc(lib, x)
    o = c_uint64()
    assert lib.applegpu_eager_mean_all(ix, ctypes.byref(o))
    np.testing.assert_allclose(read(lib, o.value, (1,)), [x.mean()], rtol=1e-5)
    o2 = c_uint64()
    assert lib.applegpu_eager_scalar_mul(ix, c_float(2.5), ctypes.byref(o2))
    np.testing.assert_array_equal(read(lib, o2.value, (7, 9)), x * np.float32(2.5))
    o3 = c_uint64()
    assert lib.applegpu_eager_threshold_backward(ix, ix, c_float(0.5), ctypes.byref(o3))
    np.testing.assert_array_equal(read(lib, o3.value, (7, 9)), np.where(x > 0.5, x, 0))


def test_pool_reuses_freed_buffers(gpu, lib):
    before = gpu.pool_stats()
    ids = [alloc(lib, np.zeros((1000,), np.float32))[0] for _ in range(4)]
    for i in ids:
        lib.applegpu_eager_free(i)
    ids2 = [alloc(lib, np.zeros((900,), np.float32))[0] for _ in range(4)]
    after = gpu.pool_stats()
    assert after["hits"] - before["hits"] >= 4
    for i in ids2:
        lib.applegpu_eager_free(i)


def test_alloc_failure_is_reported(gpu, lib):
    lib.applegpu_ffi_inject_alloc_failures(1)
    out = c_uint64()
    dims = (c_uint64 * 1)(12345679)
    assert not lib.applegpu_eager_alloc(dims, 1, 0, ctypes.byref(out))
    assert b"allocation" in lib.applegpu_eager_last_error()
    # the next allocation works again
    assert lib.applegpu_eager_alloc(dims, 1, 0, ctypes.byref(out))
    lib.applegpu_eager_free(out.value)


def test_graph_path_reference_surface(gpu, lib):
    """applegpu_ffi_* : alloc + register + ops + *_out + eval + read_f32."""
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    tid = c_uint64()
    p = lib.applegpu_ffi_alloc(a.nbytes, 0, ctypes.byref(tid))
    assert p
    dims = (c_uint64 * 2)(2, 3)
    assert lib.applegpu_ffi_register_tensor(tid.value, dims, 2, 0) == 0
    assert lib.applegpu_ffi_write_bytes(tid.value, a.ctypes.data, a.nbytes) == 0
    r = lib.applegpu_ffi_relu(lib.applegpu_ffi_neg(tid.value))
    s = lib.applegpu_ffi_add(tid.value, tid.value)
    assert r and s
    assert lib.applegpu_ffi_is_pending(s) == 1
    out_id = c_uint64()
    ptr = lib.applegpu_ffi_mul_out(s, tid.value, ctypes.byref(out_id))
    assert ptr
    assert lib.applegpu_ffi_eval(out_id.value) == 0
    buf = (c_float * 6)()
    assert lib.applegpu_ffi_read_f32(out_id.value, buf, 6) == 0
    np.testing.assert_array_equal(np.frombuffer(buf, np.float32).reshape(2, 3), 2 * a * a)
    assert lib.applegpu_ffi_read_f32(r, buf, 6) == 0
    np.testing.assert_array_equal(np.frombuffer(buf, np.float32), np.zeros(6))
    m = lib.applegpu_ffi_mean_all_out(tid.value, ctypes.byref(out_id))
    assert m
    assert lib.applegpu_ffi_read_f32(out_id.value, buf, 1) == 0
    assert buf[0] == pytest.approx(2.5)
    # matmul shape error gives id 0 and an error message
    assert lib.applegpu_ffi_matmul(tid.value, tid.value) == 0
    assert b"inner dimensions" in lib.applegpu_ffi_last_error()
    lib.applegpu_ffi_synchronize()


def test_lazy_graph_frees_dropped_intermediates(gpu):
    x = gpu.from_numpy(np.ones((64, 64), np.float32))
    n0 = gpu.tensor_count()
    y = x
    for _ in range(20):
        y = gpu.relu(y + x)
    assert gpu.tensor_count() - n0 == 1  # only `y` stays registered; the rest are graph-internal
    np.testing.assert_array_equal(y.to_numpy(), np.full((64, 64), 21.0, np.float32))
    assert not y.is_pending()
