// C ABI: the reference's applegpu_ffi.h surface plus the MI355X additions
// declared in include/applegpu_ffi.h.  Every entry point takes one global
// lock (crates/core/src/eager_ffi.rs:32-36), converts C++ exceptions into the
// reference's return conventions, and records the message in a thread-local
// last-error slot (eager_ffi.rs:38-46, backend_ffi.rs:26-34).
#include "../../include/applegpu_ffi.h"

#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "core.hpp"
#include "graph.hpp"
#include "kernels.hpp"
#include "ops.hpp"

using namespace agpu;

namespace {

std::recursive_mutex& big_lock() {
  static std::recursive_mutex* m = new std::recursive_mutex();
  return *m;
}

thread_local std::string t_eager_err;
thread_local bool t_eager_has_err = false;
thread_local std::string t_ffi_err;
thread_local bool t_ffi_has_err = false;

void set_eager_err(const std::string& s) { t_eager_err = s; t_eager_has_err = true; }
void set_ffi_err(const std::string& s) { t_ffi_err = s; t_ffi_has_err = true; }

enum Slot { kEager, kFfi };

template <typename R, typename F>
R guarded(Slot slot, R on_fail, F&& f) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  try {
    return f();
  } catch (const std::exception& e) {
    if (slot == kEager) set_eager_err(e.what());
    else set_ffi_err(e.what());
  } catch (...) {
    if (slot == kEager) set_eager_err("unknown error");
    else set_ffi_err("unknown error");
  }
  return on_fail;
}

Runtime& rt() { return Runtime::get(); }

std::vector<int64_t> dims_of(const uint64_t* d, uint32_t n) {
  if (n > (uint32_t)kMaxDims) fail("Shape has %u dimensions, maximum is %d", n, kMaxDims);
  if (n && !d) fail("null dims pointer");
  std::vector<int64_t> v(n);
  for (uint32_t i = 0; i < n; ++i) v[i] = (int64_t)d[i];
  return v;
}

DType wire(int8_t w) {
  DType d;
  if (!dtype_from_wire(w, &d)) fail("invalid dtype wire value: %d", (int)w);
  return d;
}

// Eager inputs: materialise lazily recorded tensors first.
TensorP eager_in(uint64_t id) {
  TensorP t = rt().lookup(id);
  if (t->pending()) eval(t);
  return t;
}

uint8_t* publish(const TensorP& t, uint64_t* out_id) {
  uint64_t id = rt().insert(t);
  if (out_id) *out_id = id;
  return (uint8_t*)t->data();
}

void check_capacity(const Tensor& t) {
  if (!t.buf) return;
  // Bounds are the owner's requested size, not the pool's rounded capacity.
  const size_t have = t.buf->requested > (size_t)t.offset ? t.buf->requested - (size_t)t.offset : 0;
  if (t.extent_bytes() > have)
    fail("shape %s with these strides reaches %zu bytes, past the %zu bytes of the allocation",
         shape_str(t.dims()).c_str(), t.extent_bytes(), have);
}

void no_capture(const char* what) {
  if (rt().pool().capturing()) fail("%s is not allowed while a graph capture is active", what);
}

void copy_to_host(const TensorP& t0, void* dst, uint64_t nbytes) {
  no_capture("reading a tensor to the host");
  TensorP t = t0;
  if (t->pending()) eval(t);
  if (nbytes != t->nbytes())
    fail("read of %llu bytes from a tensor of %zu bytes", (unsigned long long)nbytes, t->nbytes());
  if (nbytes == 0) return;
  TensorP c = ops::contiguous(t);
  AGPU_HIP(hipMemcpyAsync(dst, c->data(), nbytes, hipMemcpyDeviceToHost, rt().stream()));
  AGPU_HIP(hipStreamSynchronize(rt().stream()));
}

void copy_from_host(const TensorP& t, const void* src, uint64_t nbytes) {
  no_capture("writing a tensor from the host");
  if (t->pending()) fail("cannot write into a tensor with pending ops");
  if (nbytes != t->nbytes())
    fail("write of %llu bytes into a tensor of %zu bytes", (unsigned long long)nbytes, t->nbytes());
  if (nbytes == 0) return;
  if (t->is_contiguous()) {
    AGPU_HIP(hipMemcpyAsync(t->data(), src, nbytes, hipMemcpyHostToDevice, rt().stream()));
    AGPU_HIP(hipStreamSynchronize(rt().stream()));
    return;
  }
  // Strided destination: stage contiguously, then copy through the strides.
  TensorP tmp = rt().alloc(t->dtype, t->dims());
  AGPU_HIP(hipMemcpyAsync(tmp->data(), src, nbytes, hipMemcpyHostToDevice, rt().stream()));
  ops::copy_into(t, tmp);
  AGPU_HIP(hipStreamSynchronize(rt().stream()));
}

int32_t op_common(bool lazy, Slot slot, const char* op, const uint64_t* inputs, uint32_t n_in,
                  const double* f, uint32_t nf, const int64_t* iv, uint32_t ni, uint64_t* out_ids,
                  uint32_t max_out) {
  return guarded<int32_t>(slot, -1, [&]() -> int32_t {
    if (!op) fail("null op name");
    int code = op_code(op);
    if (code < 0) fail("unknown op '%s'", op);
    std::vector<TensorP> in(n_in);
    for (uint32_t i = 0; i < n_in; ++i) in[i] = lazy ? rt().lookup(inputs[i]) : eager_in(inputs[i]);
    std::vector<double> fv(f, f + nf);
    std::vector<int64_t> ivv(iv, iv + ni);
    std::vector<TensorP> outs = lazy ? record_op(code, in, fv, ivv) : run_op(code, in, fv, ivv);
    if (outs.size() > max_out) fail("%s produces %zu outputs, room for %u", op, outs.size(), max_out);
    for (size_t i = 0; i < outs.size(); ++i) out_ids[i] = rt().insert(outs[i]);
    return (int32_t)outs.size();
  });
}

uint64_t lazy1(const char* op, std::initializer_list<uint64_t> ids, std::initializer_list<double> f = {},
               std::initializer_list<int64_t> iv = {}) {
  std::vector<uint64_t> in(ids);
  std::vector<double> fv(f);
  std::vector<int64_t> ivv(iv);
  uint64_t out = 0;
  int32_t n = op_common(true, kFfi, op, in.data(), (uint32_t)in.size(), fv.data(), (uint32_t)fv.size(), ivv.data(),
                        (uint32_t)ivv.size(), &out, 1);
  return n == 1 ? out : 0;
}

// *_out graph variants: record, then preallocate the output so the caller
// holds its pointer (crates/core/src/backend_ffi.rs:341-362).
uint8_t* lazy_out(const char* op, std::initializer_list<uint64_t> ids, std::initializer_list<double> f,
                  uint64_t* out_id) {
  uint64_t id = lazy1(op, ids, f);
  if (!id) return nullptr;
  return guarded<uint8_t*>(kFfi, nullptr, [&]() -> uint8_t* {
    TensorP t = rt().lookup(id);
    if (t->pending()) t->buf = rt().pool().acquire(t->nbytes() ? t->nbytes() : 4);
    if (out_id) *out_id = id;
    return (uint8_t*)t->data();
  });
}

template <typename F>
uint8_t* eager_out(uint64_t* out_id, F&& f) {
  return guarded<uint8_t*>(kEager, nullptr, [&]() -> uint8_t* { return publish(f(), out_id); });
}

}  // namespace

extern "C" {

// ════════════════════════ graph path ════════════════════════════════════════
bool applegpu_ffi_init(void) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  std::string err;
  if (!Runtime::init(&err)) {
    set_ffi_err(err);
    return false;
  }
  return true;
}

const char* applegpu_ffi_last_error(void) { return t_ffi_has_err ? t_ffi_err.c_str() : nullptr; }

uint8_t* applegpu_ffi_alloc(uint64_t size_bytes, int8_t dtype_i8, uint64_t* out_tensor_id) {
  return guarded<uint8_t*>(kFfi, nullptr, [&]() -> uint8_t* {
    DType dt = wire(dtype_i8);
    if (!out_tensor_id) fail("null out_tensor_id");
    if (size_bytes == 0) {
      // zero-size allocation: an id with no storage (backend_ffi.rs:93-98)
      *out_tensor_id = rt().insert(make_meta(dt, {0}));
      return nullptr;
    }
    size_t es = dtype_size(dt);
    TensorP t = make_meta(dt, {(int64_t)(size_bytes / es)});
    t->buf = rt().pool().acquire(size_bytes);
    *out_tensor_id = rt().insert(t);
    return (uint8_t*)t->data();
  });
}

void applegpu_ffi_free(uint64_t tensor_id) {
  guarded<int>(kFfi, 0, [&]() {
    if (Runtime::initialized()) rt().erase(tensor_id);
    return 0;
  });
}

int32_t applegpu_ffi_register_tensor(uint64_t tensor_id, const uint64_t* dims, uint32_t ndim, int8_t dtype_i8) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    TensorP t = rt().lookup(tensor_id);
    if (t->pending()) fail("register_tensor: tensor %llu has pending ops", (unsigned long long)tensor_id);
    auto d = dims_of(dims, ndim);
    auto nt = make_meta(wire(dtype_i8), d);
    nt->buf = t->buf;
    nt->offset = t->offset;
    check_capacity(*nt);
    rt().replace(tensor_id, nt);
    return 0;
  });
}

int32_t applegpu_ffi_shape(uint64_t tensor_id, uint64_t* out_dims, uint32_t* out_ndim) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    TensorP t = rt().lookup(tensor_id);
    *out_ndim = (uint32_t)t->ndim;
    for (int i = 0; i < t->ndim; ++i) out_dims[i] = (uint64_t)t->shape[i];
    return 0;
  });
}

int8_t applegpu_ffi_dtype(uint64_t tensor_id) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  if (!Runtime::initialized()) return -1;
  TensorP t = rt().try_lookup(tensor_id);
  return t ? (int8_t)t->dtype : (int8_t)-1;
}

uint64_t applegpu_ffi_add(uint64_t a, uint64_t b) { return lazy1("add", {a, b}); }
uint64_t applegpu_ffi_matmul(uint64_t a, uint64_t b) { return lazy1("matmul", {a, b}); }
uint64_t applegpu_ffi_relu(uint64_t x) { return lazy1("relu", {x}); }
uint64_t applegpu_ffi_mul(uint64_t a, uint64_t b) { return lazy1("mul", {a, b}); }
uint64_t applegpu_ffi_sub(uint64_t a, uint64_t b) { return lazy1("sub", {a, b}); }
uint64_t applegpu_ffi_neg(uint64_t x) { return lazy1("neg", {x}); }

int32_t applegpu_ffi_copy(uint64_t src_id, uint64_t dst_id) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    // dst = src element-wise (crates/core/src/backend_ffi.rs copy); dst may be
    // a view of another tensor (e.g. a slice of a KV cache, evaluated here to
    // a view of that tensor's storage) with any strides.
    TensorP src = rt().lookup(src_id);
    if (src->pending()) eval(src);
    TensorP dst = rt().lookup(dst_id);
    if (dst->pending()) eval(dst);
    if (!dst->buf) fail("copy: destination has no storage");
    if (dst->extent_bytes() + (size_t)dst->offset > dst->buf->requested) fail("copy: destination too small");
    ops::copy_into(dst, src);
    return 0;
  });
}

static TensorP kv_operand(uint64_t id) {
  TensorP t = rt().lookup(id);
  if (t->pending()) eval(t);
  return t;
}

static TensorP kv_cache_operand(uint64_t id) {
  TensorP c = kv_operand(id);
  if (!c->buf) fail("kv_write: cache has no storage");
  if (c->extent_bytes() + (size_t)c->offset > c->buf->requested) fail("kv_write: cache view out of bounds");
  return c;
}

int32_t applegpu_kv_write(uint64_t cache_id, uint64_t rows_id, uint64_t pos_id) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    // In-place KV append at device-resident positions; replaces the
    // reference's per-step concat of the whole cache
    // (python/applegpu_runtime/models/gpt2.py:122-126).
    TensorP rows = kv_operand(rows_id), pos = kv_operand(pos_id);
    ops::kv_write(kv_cache_operand(cache_id), rows, pos);
    return 0;
  });
}

int32_t applegpu_kv_write_pair(uint64_t k_cache_id, uint64_t v_cache_id, uint64_t k_rows_id, uint64_t v_rows_id,
                               uint64_t pos_id) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    TensorP kr = kv_operand(k_rows_id), vr = kv_operand(v_rows_id), pos = kv_operand(pos_id);
    ops::kv_write(kv_cache_operand(k_cache_id), kr, pos, kv_cache_operand(v_cache_id), vr);
    return 0;
  });
}

uint8_t* applegpu_ffi_add_out(uint64_t a, uint64_t b, uint64_t* o) { return lazy_out("add", {a, b}, {}, o); }
uint8_t* applegpu_ffi_mul_out(uint64_t a, uint64_t b, uint64_t* o) { return lazy_out("mul", {a, b}, {}, o); }
uint8_t* applegpu_ffi_sub_out(uint64_t a, uint64_t b, uint64_t* o) { return lazy_out("sub", {a, b}, {}, o); }
uint8_t* applegpu_ffi_matmul_out(uint64_t a, uint64_t b, uint64_t* o) { return lazy_out("matmul", {a, b}, {}, o); }
uint8_t* applegpu_ffi_relu_out(uint64_t x, uint64_t* o) { return lazy_out("relu", {x}, {}, o); }
uint8_t* applegpu_ffi_neg_out(uint64_t x, uint64_t* o) { return lazy_out("neg", {x}, {}, o); }
uint8_t* applegpu_ffi_div_out(uint64_t a, uint64_t b, uint64_t* o) { return lazy_out("div", {a, b}, {}, o); }
uint8_t* applegpu_ffi_threshold_backward_out(uint64_t g, uint64_t x, float thr, uint64_t* o) {
  return lazy_out("threshold_backward", {g, x}, {thr}, o);
}
uint8_t* applegpu_ffi_scalar_mul_out(uint64_t x, float s, uint64_t* o) { return lazy_out("scalar_mul", {x}, {s}, o); }
uint8_t* applegpu_ffi_mean_all_out(uint64_t x, uint64_t* o) { return lazy_out("mean_all", {x}, {}, o); }

int32_t applegpu_ffi_eval(uint64_t tensor_id) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    eval(rt().lookup(tensor_id));
    return 0;
  });
}

int32_t applegpu_ffi_eval_many(const uint64_t* tensor_ids, uint32_t n) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (n > 0 && !tensor_ids) fail("eval_many: null id array");
    std::vector<TensorP> roots;
    roots.reserve(n);
    for (uint32_t i = 0; i < n; ++i) roots.push_back(rt().lookup(tensor_ids[i]));
    eval_all(roots);
    return 0;
  });
}

void applegpu_ffi_synchronize(void) {
  guarded<int>(kFfi, 0, [&]() {
    if (Runtime::initialized()) rt().sync();
    return 0;
  });
}

int32_t applegpu_ffi_read_f32(uint64_t tensor_id, float* out_ptr, uint64_t max_elements) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    no_capture("read_f32");
    TensorP t = rt().lookup(tensor_id);
    if (t->pending()) eval(t);
    TensorP f = ops::cast(t, DType::F32);
    TensorP c = ops::contiguous(f);
    uint64_t n = std::min<uint64_t>((uint64_t)c->numel(), max_elements);
    if (n) {
      AGPU_HIP(hipMemcpyAsync(out_ptr, c->data(), n * 4, hipMemcpyDeviceToHost, rt().stream()));
      AGPU_HIP(hipStreamSynchronize(rt().stream()));
    }
    return 0;
  });
}

int32_t applegpu_graph_op(const char* op, const uint64_t* inputs, uint32_t n_inputs, const double* fparams,
                          uint32_t n_f, const int64_t* iparams, uint32_t n_i, uint64_t* out_ids, uint32_t max_out) {
  return op_common(true, kFfi, op, inputs, n_inputs, fparams, n_f, iparams, n_i, out_ids, max_out);
}

int32_t applegpu_ffi_write_bytes(uint64_t tensor_id, const void* src, uint64_t nbytes) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    copy_from_host(rt().lookup(tensor_id), src, nbytes);
    return 0;
  });
}

int32_t applegpu_ffi_read_bytes(uint64_t tensor_id, void* dst, uint64_t nbytes) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    copy_to_host(rt().lookup(tensor_id), dst, nbytes);
    return 0;
  });
}

int32_t applegpu_ffi_is_pending(uint64_t tensor_id) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t { return rt().lookup(tensor_id)->pending() ? 1 : 0; });
}

int32_t applegpu_ffi_strides(uint64_t tensor_id, int64_t* out_strides, uint32_t* out_ndim) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    TensorP t = rt().lookup(tensor_id);
    *out_ndim = (uint32_t)t->ndim;
    for (int i = 0; i < t->ndim; ++i) out_strides[i] = t->strides[i];
    return 0;
  });
}

int32_t applegpu_ffi_pool_stats(uint64_t* out5) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    PoolStats s = rt().pool().stats();
    out5[0] = s.hits; out5[1] = s.misses; out5[2] = s.pooled_bytes; out5[3] = s.bucket_count; out5[4] = s.live_bytes;
    return 0;
  });
}

void applegpu_ffi_pool_drain(void) {
  guarded<int>(kFfi, 0, [&]() { rt().pool().drain(); return 0; });
}

void applegpu_ffi_set_pool_watermark(uint64_t bytes) {
  guarded<int>(kFfi, 0, [&]() { rt().pool().set_watermark(bytes); return 0; });
}

uint64_t applegpu_ffi_memory_usage(void) {
  return guarded<uint64_t>(kFfi, 0, [&]() -> uint64_t { return rt().memory_usage(); });
}

uint64_t applegpu_ffi_tensor_count(void) {
  return guarded<uint64_t>(kFfi, 0, [&]() -> uint64_t { return rt().count(); });
}

void applegpu_ffi_set_limits(uint64_t max_tensor_bytes, uint64_t max_memory_bytes, uint64_t max_tensors) {
  guarded<int>(kFfi, 0, [&]() {
    rt().max_tensor_bytes = max_tensor_bytes;
    rt().max_memory_bytes = max_memory_bytes;
    rt().max_tensors = max_tensors;
    return 0;
  });
}

int32_t applegpu_ffi_device_name(char* out, uint32_t cap) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    std::string s = rt().info().name + " (" + rt().info().arch + ", " + std::to_string(rt().info().cu_count) + " CUs)";
    if (cap) {
      std::strncpy(out, s.c_str(), cap - 1);
      out[cap - 1] = 0;
    }
    return 0;
  });
}

int32_t applegpu_ffi_graph_stats(uint64_t* out4) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  GraphStats s = graph_stats();
  out4[0] = s.evals; out4[1] = s.nodes; out4[2] = s.fused_gemm_epilogues; out4[3] = s.launches_saved;
  return 0;
}

uint32_t applegpu_ffi_graph_stats_ex(uint64_t* out, uint32_t cap) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  GraphStats s = graph_stats();
  const uint64_t v[] = {s.evals, s.nodes, s.fused_gemm_epilogues, s.launches_saved,
                        s.fused_chains, s.chain_nodes, s.launcher_calls};
  const uint32_t n = (uint32_t)(sizeof v / sizeof v[0]);
  for (uint32_t i = 0; i < n && i < cap; ++i) out[i] = v[i];
  return n;
}

// ── graph capture ──────────────────────────────────────────────────────────
namespace {
struct Captured {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  Arena* arena = nullptr;
};
std::unordered_map<int64_t, Captured*>& graphs() {
  static auto* m = new std::unordered_map<int64_t, Captured*>();
  return *m;
}
int64_t g_next_graph = 1;
Arena* g_capture = nullptr;

void drop_capture_state(Arena* a, hipGraph_t graph) {
  if (graph) (void)hipGraphDestroy(graph);
  rt().pool().release_arena(a);
  delete a;
}
}  // namespace

int32_t applegpu_capture_begin(void) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (g_capture) fail("a graph capture is already active");
    auto* a = new Arena();
    rt().pool().begin_capture(a);
    hipError_t e = hipStreamBeginCapture(rt().stream(), hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      rt().pool().end_capture();
      drop_capture_state(a, nullptr);
      fail("hipStreamBeginCapture failed: %s", hipGetErrorString(e));
    }
    g_capture = a;
    return 0;
  });
}

int64_t applegpu_capture_end(void) {
  return guarded<int64_t>(kFfi, -1, [&]() -> int64_t {
    if (!g_capture) fail("no graph capture is active");
    Arena* a = g_capture;
    g_capture = nullptr;
    rt().pool().end_capture();
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(rt().stream(), &graph);
    if (e != hipSuccess || !graph) {
      (void)hipGetLastError();
      drop_capture_state(a, graph);
      fail("hipStreamEndCapture failed: %s", hipGetErrorString(e));
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      drop_capture_state(a, graph);
      fail("hipGraphInstantiate failed: %s", hipGetErrorString(e));
    }
    auto* c = new Captured{graph, exec, a};
    const int64_t id = g_next_graph++;
    graphs()[id] = c;
    return id;
  });
}

int32_t applegpu_capture_abort(void) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (!g_capture) return 0;
    Arena* a = g_capture;
    g_capture = nullptr;
    rt().pool().end_capture();
    hipGraph_t graph = nullptr;
    (void)hipStreamEndCapture(rt().stream(), &graph);
    (void)hipGetLastError();
    drop_capture_state(a, graph);
    return 0;
  });
}

int32_t applegpu_graph_replay(int64_t handle) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (g_capture) fail("cannot replay a graph while a capture is active");
    auto it = graphs().find(handle);
    if (it == graphs().end()) fail("graph %lld not found", (long long)handle);
    AGPU_HIP(hipGraphLaunch(it->second->exec, rt().stream()));
    return 0;
  });
}

int32_t applegpu_graph_destroy(int64_t handle) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (!Runtime::initialized()) return 0;
    auto it = graphs().find(handle);
    if (it == graphs().end()) fail("graph %lld not found", (long long)handle);
    Captured* c = it->second;
    graphs().erase(it);
    // A replay may still be running: the graph's buffers return to the pool
    // only after the stream drains.
    AGPU_HIP(hipStreamSynchronize(rt().stream()));
    (void)hipGraphExecDestroy(c->exec);
    drop_capture_state(c->arena, c->graph);
    delete c;
    return 0;
  });
}

uint64_t applegpu_graph_bytes(int64_t handle) {
  return guarded<uint64_t>(kFfi, 0, [&]() -> uint64_t {
    auto it = graphs().find(handle);
    if (it == graphs().end()) fail("graph %lld not found", (long long)handle);
    return it->second->arena->bytes;
  });
}

int32_t applegpu_ffi_gemm_tune(int32_t f32_mode, int32_t cfg, int32_t splits) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (f32_mode != k::kF32Split3 && f32_mode != k::kF32Native) fail("gemm_tune: f32_mode must be 0 or 1");
    if (cfg < -1 || cfg >= k::kMfConfigs) fail("gemm_tune: cfg must be -1..%d", k::kMfConfigs - 1);
    if (splits < 0 || splits > 64) fail("gemm_tune: splits must be 0..64");
    k::GemmTune& t = k::gemm_tune();
    t.f32_mode = f32_mode;
    t.cfg = cfg;
    t.splits = splits;
    return 0;
  });
}

int32_t applegpu_ffi_gemm_skinny(int32_t enable) {
  k::GemmTune& t = k::gemm_tune();
  const int32_t prev = t.no_skinny ? 0 : 1;
  t.no_skinny = enable == 0;
  return prev;
}

int32_t applegpu_ffi_split_inkernel(int32_t enable) {
  k::GemmTune& t = k::gemm_tune();
  const int32_t prev = t.inkernel_splits ? 1 : 0;
  t.inkernel_splits = enable != 0;
  return prev;
}

int32_t applegpu_ffi_x3_rows_out(int64_t M, int64_t N, int64_t K) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (M < 1 || N < 1 || K < 1) fail("x3_rows_out: extents must be positive");
    return k::gemm_x3_rows_out_ok(M, N, K, true) ? 1 : 0;
  });
}

int32_t applegpu_ffi_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t batch, int8_t dtype_i8, bool a_kcontig,
                               bool b_kcontig, char* out, uint32_t cap) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (!out || cap == 0) fail("gemm_plan: null output buffer");
    k::Gemm g;
    g.dt = g.b_dt = wire(dtype_i8);
    g.M = M; g.N = N; g.K = K; g.batch = batch;
    g.a_sk = a_kcontig ? 1 : M; g.a_sm = a_kcontig ? K : 1;
    g.b_sk = b_kcontig ? 1 : N; g.b_sn = b_kcontig ? K : 1;
    g.c_sm = N;
    snprintf(out, cap, "%s", k::gemm_plan_name(g));
    return 0;
  });
}

void applegpu_ffi_inject_alloc_failures(int32_t n) {
  guarded<int>(kFfi, 0, [&]() { rt().pool().inject_failures(n); return 0; });
}

static hipEvent_t g_events[16];

int32_t applegpu_ffi_event_record(uint32_t slot) {
  return guarded<int32_t>(kFfi, -1, [&]() -> int32_t {
    if (slot >= 16) fail("event slot %u out of range", slot);
    if (!g_events[slot]) AGPU_HIP(hipEventCreate(&g_events[slot]));
    AGPU_HIP(hipEventRecord(g_events[slot], rt().stream()));
    return 0;
  });
}

float applegpu_ffi_event_elapsed_ms(uint32_t a, uint32_t b) {
  return guarded<float>(kFfi, -1.f, [&]() -> float {
    if (a >= 16 || b >= 16 || !g_events[a] || !g_events[b]) fail("event slots not recorded");
    no_capture("event_elapsed_ms");
    AGPU_HIP(hipEventSynchronize(g_events[b]));
    float ms = 0.f;
    AGPU_HIP(hipEventElapsedTime(&ms, g_events[a], g_events[b]));
    return ms;
  });
}

// ════════════════════════ eager path ═══════════════════════════════════════
bool applegpu_eager_init(void) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  if (getenv("APPLEGPU_SOCKET") || getenv("APPLEGPU_HOST")) {
    set_eager_err("remote mode (APPLEGPU_SOCKET / APPLEGPU_HOST) is not supported by the MI355X backend");
    return false;
  }
  std::string err;
  if (!Runtime::init(&err)) {
    set_eager_err(err);
    return false;
  }
  return true;
}

const char* applegpu_eager_last_error(void) { return t_eager_has_err ? t_eager_err.c_str() : nullptr; }

uint8_t* applegpu_eager_alloc(const uint64_t* dims, uint32_t ndim, int8_t dtype, uint64_t* out_id) {
  return eager_out(out_id, [&] { return rt().alloc(wire(dtype), dims_of(dims, ndim)); });
}

void applegpu_eager_free(uint64_t id) {
  guarded<int>(kEager, 0, [&]() {
    if (Runtime::initialized()) rt().erase(id);
    return 0;
  });
}

int32_t applegpu_eager_register_shape(uint64_t id, const uint64_t* dims, uint32_t ndim) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    TensorP t = rt().lookup(id);
    auto nt = make_meta(t->dtype, dims_of(dims, ndim));
    nt->buf = t->buf;
    nt->offset = t->offset;
    nt->node = t->node;
    check_capacity(*nt);
    rt().replace(id, nt);
    return 0;
  });
}

int32_t applegpu_eager_shape(uint64_t id, uint64_t* out_dims, uint32_t* out_ndim) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    TensorP t = rt().lookup(id);
    *out_ndim = (uint32_t)t->ndim;
    for (int i = 0; i < t->ndim; ++i) out_dims[i] = (uint64_t)t->shape[i];
    return 0;
  });
}

int8_t applegpu_eager_dtype(uint64_t id) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  if (!Runtime::initialized()) return -1;
  TensorP t = rt().try_lookup(id);
  return t ? (int8_t)t->dtype : (int8_t)-1;
}

uint8_t* applegpu_eager_add(uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::binary(k::kAdd, eager_in(a), eager_in(b)); });
}
uint8_t* applegpu_eager_sub(uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::binary(k::kSub, eager_in(a), eager_in(b)); });
}
uint8_t* applegpu_eager_mul(uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::binary(k::kMul, eager_in(a), eager_in(b)); });
}
uint8_t* applegpu_eager_div(uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::binary(k::kDiv, eager_in(a), eager_in(b)); });
}
uint8_t* applegpu_eager_relu(uint64_t x, uint64_t* o) {
  return eager_out(o, [&] { return ops::unary(k::kRelu, eager_in(x)); });
}
uint8_t* applegpu_eager_neg(uint64_t x, uint64_t* o) {
  return eager_out(o, [&] { return ops::unary(k::kNeg, eager_in(x)); });
}
uint8_t* applegpu_eager_matmul(uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::matmul(eager_in(a), eager_in(b)); });
}
uint8_t* applegpu_eager_matmul_ex(uint64_t a, uint64_t b, bool ta, bool tb, uint64_t* o) {
  return eager_out(o, [&] { return ops::matmul(eager_in(a), eager_in(b), ta, tb); });
}
uint8_t* applegpu_eager_threshold_backward(uint64_t g, uint64_t x, float thr, uint64_t* o) {
  return eager_out(o, [&] { return ops::threshold_backward(eager_in(g), eager_in(x), thr); });
}
uint8_t* applegpu_eager_scalar_mul(uint64_t x, float s, uint64_t* o) {
  return eager_out(o, [&] { return ops::unary(k::kScale, eager_in(x), s); });
}
uint8_t* applegpu_eager_mean_all(uint64_t x, uint64_t* o) {
  return eager_out(o, [&] { return ops::mean_all(eager_in(x)); });
}
uint8_t* applegpu_eager_sum_dim(uint64_t x, int64_t dim, bool keepdim, uint64_t* o) {
  return eager_out(o, [&] { return ops::sum_dim(eager_in(x), dim, keepdim); });
}

uint8_t* applegpu_eager_create_view(uint64_t base_id, const uint64_t* shape, const uint64_t* strides, uint32_t ndim,
                                    uint64_t offset, uint64_t* out_id) {
  return eager_out(out_id, [&] {
    TensorP base = eager_in(base_id);
    std::vector<int64_t> sh = dims_of(shape, ndim), st = dims_of(strides, ndim);
    // offset is in elements of the base, relative to the base's own offset
    // (crates/core/src/eager.rs:114-139)
    return ops::view(base, sh, st, (int64_t)offset);
  });
}

uint8_t* applegpu_eager_data_ptr(uint64_t id) {
  return guarded<uint8_t*>(kEager, nullptr, [&]() -> uint8_t* {
    TensorP t = eager_in(id);
    return (uint8_t*)t->data();
  });
}

uint8_t* applegpu_eager_view_typed(uint64_t base_id, const uint64_t* shape, const uint64_t* strides, uint32_t ndim,
                                   uint64_t offset_bytes, int8_t dtype_i8, uint64_t* out_id) {
  return eager_out(out_id, [&] {
    TensorP base = eager_in(base_id);
    std::vector<int64_t> sh = dims_of(shape, ndim), st = dims_of(strides, ndim);
    return ops::view_bytes(base, wire(dtype_i8), sh, st, (int64_t)offset_bytes);
  });
}

int32_t applegpu_eager_add_inplace(uint64_t self_id, uint64_t other_id) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    ops::axpy_inplace(eager_in(self_id), eager_in(other_id), 1.f);
    return 0;
  });
}

int32_t applegpu_eager_add_scaled_inplace(uint64_t self_id, uint64_t other_id, float alpha) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    ops::axpy_inplace(eager_in(self_id), eager_in(other_id), alpha);
    return 0;
  });
}

void applegpu_eager_flush_and_wait(void) {
  guarded<int>(kEager, 0, [&]() {
    if (Runtime::initialized()) rt().sync();
    return 0;
  });
}

void applegpu_eager_synchronize(void) { applegpu_eager_flush_and_wait(); }

uint8_t* applegpu_eager_embedding(uint64_t w, uint64_t idx, uint64_t* o) {
  return eager_out(o, [&] { return ops::embedding(eager_in(w), eager_in(idx)); });
}
uint8_t* applegpu_eager_layer_norm(uint64_t x, uint64_t g, uint64_t b, float eps, uint64_t* o) {
  return eager_out(o, [&] { return ops::layer_norm(eager_in(x), eager_in(g), eager_in(b), eps); });
}
uint8_t* applegpu_eager_gelu(uint64_t x, uint64_t* o) {
  return eager_out(o, [&] { return ops::unary(k::kGelu, eager_in(x)); });
}
uint8_t* applegpu_eager_softmax(uint64_t x, uint64_t* o) {
  return eager_out(o, [&] { return ops::softmax(eager_in(x), k::kSoftmax); });
}

uint64_t applegpu_eager_find_by_data_ptr(const uint8_t* ptr) {
  std::lock_guard<std::recursive_mutex> g(big_lock());
  if (!Runtime::initialized()) return 0;
  return rt().find_by_data_ptr(ptr);
}

int32_t applegpu_eager_execute_graph(const uint8_t* ops_data, uint32_t ops_len, const uint64_t* input_tids,
                                     uint32_t n_inputs, const uint16_t* output_indices, uint32_t n_outputs,
                                     uint64_t* out_tids, uint8_t** out_ptrs) {
  // crates/core/src/eager_ffi.rs:661-708: returns the number of outputs, or
  // -1 with "compiled graph failed: ..." set
  std::lock_guard<std::recursive_mutex> g(big_lock());
  try {
    execute_compiled(ops_data, ops_len, input_tids, n_inputs, output_indices, n_outputs, out_tids, out_ptrs);
    return (int32_t)n_outputs;
  } catch (const std::exception& e) {
    set_eager_err(std::string("compiled graph failed: ") + e.what());
  } catch (...) {
    set_eager_err("compiled graph failed: unknown error");
  }
  return -1;
}

int32_t applegpu_eager_op(const char* op, const uint64_t* inputs, uint32_t n_inputs, const double* fparams,
                          uint32_t n_f, const int64_t* iparams, uint32_t n_i, uint64_t* out_ids, uint32_t max_out) {
  return op_common(false, kEager, op, inputs, n_inputs, fparams, n_f, iparams, n_i, out_ids, max_out);
}

int32_t applegpu_eager_copy_from_host(uint64_t id, const void* src, uint64_t nbytes) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    copy_from_host(eager_in(id), src, nbytes);
    return 0;
  });
}

int32_t applegpu_eager_copy_to_host(uint64_t id, void* dst, uint64_t nbytes) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    copy_to_host(eager_in(id), dst, nbytes);
    return 0;
  });
}

int32_t applegpu_eager_copy_(uint64_t dst_id, uint64_t src_id) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    ops::copy_into(eager_in(dst_id), eager_in(src_id));
    return 0;
  });
}

int32_t applegpu_eager_fill(uint64_t id, double value) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    TensorP t = eager_in(id);
    TensorP f = ops::full(t->dtype, t->dims(), (float)value);
    ops::copy_into(t, f);
    return 0;
  });
}

uint8_t* applegpu_eager_linear(uint64_t x_id, uint64_t w_id, uint64_t bias_id, int32_t act, uint64_t* out_id) {
  return eager_out(out_id, [&] {
    ops::Epilogue e;
    if (bias_id) e.bias = eager_in(bias_id);
    e.act = act;
    return ops::matmul(eager_in(x_id), eager_in(w_id), false, true, &e);
  });
}

int32_t applegpu_eager_linear_noalloc(uint64_t x_id, uint64_t w_id, uint64_t bias_id, int32_t act,
                                      uint64_t out_id) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    // Inputs must hold values already: evaluating pending ops could allocate.
    auto ready = [&](uint64_t id, const char* what) {
      TensorP t = rt().lookup(id);
      if (t->pending()) fail("linear_noalloc: %s has pending ops; evaluate it before this call", what);
      if (!t->buf) fail("linear_noalloc: %s has no storage", what);
      return t;
    };
    TensorP x = ready(x_id, "x"), w = ready(w_id, "weight"), out = ready(out_id, "out");
    if (x->ndim != 2 || w->ndim != 2) fail("linear_noalloc: x [M, K] and weight [N, K] must be 2-D");
    if (act < 0 || act > 3) fail("linear_noalloc: activation %d is not 0 (none), 1 (relu), 2 (gelu) or 3 (gelu_erf)", act);
    if (out->buf == x->buf || out->buf == w->buf) fail("linear_noalloc: out must not share storage with x or weight");
    ops::Epilogue e;
    if (bias_id) {
      e.bias = ready(bias_id, "bias");
      if (out->buf == e.bias->buf) fail("linear_noalloc: out must not share storage with the bias");
    }
    e.act = act;
    ops::NoAlloc na;
    na.ws = noalloc_scratch(&na.cap);
    ops::matmul(x, w, false, true, &e, out, nullptr, &na);
    return 0;
  });
}

uint8_t* applegpu_eager_matmul_masked(uint64_t a_id, uint64_t b_id, bool ta, bool tb, uint64_t mask_id,
                                      uint64_t* out_id) {
  return eager_out(out_id, [&] {
    ops::Epilogue e;
    e.mask = eager_in(mask_id);
    return ops::matmul(eager_in(a_id), eager_in(b_id), ta, tb, &e);
  });
}

uint8_t* applegpu_eager_mse_loss(uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::mse_loss(eager_in(a), eager_in(b)); });
}

uint8_t* applegpu_eager_mse_loss_backward(uint64_t g, uint64_t a, uint64_t b, uint64_t* o) {
  return eager_out(o, [&] { return ops::mse_loss_backward(eager_in(g), eager_in(a), eager_in(b)); });
}

int32_t applegpu_eager_strides(uint64_t id, int64_t* out_strides, uint32_t* out_ndim) {
  return guarded<int32_t>(kEager, -1, [&]() -> int32_t {
    TensorP t = rt().lookup(id);
    *out_ndim = (uint32_t)t->ndim;
    for (int i = 0; i < t->ndim; ++i) out_strides[i] = t->strides[i];
    return 0;
  });
}

}  // extern "C"
