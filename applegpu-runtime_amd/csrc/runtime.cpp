// Runtime: device init, the single stream, the buffer pool and the id registry.
#include <atomic>
#include "core.hpp"
#include "kernels.hpp"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>

namespace agpu {

// ── dtypes (crates/core/src/tensor.rs:59-90) ───────────────────────────────
size_t dtype_size(DType d) {
  switch (d) {
    case DType::F32: return 4;
    case DType::F16: return 2;
    case DType::F64: return 8;
    case DType::I8: return 1;
    case DType::I16: return 2;
    case DType::I32: return 4;
    case DType::I64: return 8;
    case DType::U8: return 1;
    case DType::U32: return 4;
    case DType::Bool: return 1;
    case DType::BF16: return 2;
  }
  return 0;
}

const char* dtype_name(DType d) {
  switch (d) {
    case DType::F32: return "float32";
    case DType::F16: return "float16";
    case DType::F64: return "float64";
    case DType::I8: return "int8";
    case DType::I16: return "int16";
    case DType::I32: return "int32";
    case DType::I64: return "int64";
    case DType::U8: return "uint8";
    case DType::U32: return "uint32";
    case DType::Bool: return "bool";
    case DType::BF16: return "bfloat16";
  }
  return "?";
}

bool dtype_is_float(DType d) {
  return d == DType::F32 || d == DType::F16 || d == DType::BF16 || d == DType::F64;
}

bool dtype_from_wire(int v, DType* out) {
  if (v < 0 || v > 10) return false;
  *out = (DType)v;
  return true;
}

bool dtype_from_name(const std::string& s, DType* out) {
  static const std::pair<const char*, DType> names[] = {
      {"float32", DType::F32}, {"f32", DType::F32},   {"float16", DType::F16},
      {"f16", DType::F16},     {"float64", DType::F64}, {"f64", DType::F64},
      {"int8", DType::I8},     {"i8", DType::I8},     {"int16", DType::I16},
      {"i16", DType::I16},     {"int32", DType::I32}, {"i32", DType::I32},
      {"int64", DType::I64},   {"i64", DType::I64},   {"uint8", DType::U8},
      {"u8", DType::U8},       {"uint32", DType::U32}, {"u32", DType::U32},
      {"bool", DType::Bool},   {"bool_", DType::Bool}, {"bfloat16", DType::BF16},
      {"bf16", DType::BF16},
  };
  for (auto& p : names)
    if (s == p.first) { *out = p.second; return true; }
  return false;
}

// ── errors ─────────────────────────────────────────────────────────────────
void fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Error(buf);
}

static std::atomic<uint64_t> g_launcher_calls{0};
uint64_t launcher_calls() { return g_launcher_calls.load(std::memory_order_relaxed); }

void check_launch(const char* what) {
  g_launcher_calls.fetch_add(1, std::memory_order_relaxed);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail("kernel launch %s failed: %s", what, hipGetErrorString(e));
}

// ── tensors ────────────────────────────────────────────────────────────────
bool Tensor::is_contiguous() const {
  int64_t expect = 1;
  for (int i = ndim - 1; i >= 0; --i) {
    if (shape[i] != 1 && strides[i] != expect) return false;
    expect *= shape[i];
  }
  return true;
}

void Tensor::set_contiguous_strides() {
  int64_t s = 1;
  for (int i = ndim - 1; i >= 0; --i) {
    strides[i] = s;
    s *= shape[i];
  }
}

TensorP make_meta(DType dt, const std::vector<int64_t>& dims) {
  if (dims.size() > (size_t)kMaxDims)
    fail("Shape has %zu dimensions, maximum is %d", dims.size(), kMaxDims);
  auto t = std::make_shared<Tensor>();
  t->dtype = dt;
  t->ndim = (int)dims.size();
  for (int i = 0; i < t->ndim; ++i) {
    if (dims[i] < 0) fail("negative dimension %lld", (long long)dims[i]);
    t->shape[i] = dims[i];
  }
  t->set_contiguous_strides();
  return t;
}

std::vector<int64_t> broadcast_shapes(const std::vector<int64_t>& a, const std::vector<int64_t>& b) {
  size_t n = std::max(a.size(), b.size());
  std::vector<int64_t> out(n, 1);
  for (size_t i = 0; i < n; ++i) {
    int64_t x = i < a.size() ? a[a.size() - 1 - i] : 1;
    int64_t y = i < b.size() ? b[b.size() - 1 - i] : 1;
    if (x == y || y == 1) out[n - 1 - i] = x;
    else if (x == 1) out[n - 1 - i] = y;
    else
      fail("Cannot broadcast shapes %s and %s: dim %zu is %lld vs %lld", shape_str(a).c_str(),
           shape_str(b).c_str(), n - 1 - i, (long long)x, (long long)y);
  }
  return out;
}

std::string shape_str(const std::vector<int64_t>& d) {
  std::string s = "[";
  for (size_t i = 0; i < d.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(d[i]);
  }
  return s + "]";
}

static std::atomic<uint64_t> g_next_id{1};
uint64_t next_tensor_id() { return g_next_id.fetch_add(1, std::memory_order_relaxed); }

// ── pool (crates/core/src/pool.rs:35-66) ───────────────────────────────────
static size_t next_pow2(size_t n) {
  size_t p = 1;
  while (p < n) p <<= 1;
  return p;
}

BufferP Pool::acquire(size_t nbytes) {
  size_t cap = next_pow2(nbytes < 4 ? 4 : nbytes);
  Buffer* b = nullptr;
  Arena* arena = nullptr;
  {
    std::lock_guard<std::mutex> g(mu_);
    if (inject_fail_ > 0) {
      --inject_fail_;
      fail("device allocation of %zu bytes failed: injected failure (test hook)", cap);
    }
    arena = active_;
    if (arena) {
      auto it = arena->free.find(cap);
      if (it != arena->free.end() && !it->second.empty()) {
        b = it->second.back();
        it->second.pop_back();
        ++hits_;
      }
    }
    if (!b) {
      auto it = buckets_.find(cap);
      if (it != buckets_.end() && !it->second.empty()) {
        b = it->second.back();
        it->second.pop_back();
        pooled_ -= cap;
        ++hits_;
      } else {
        ++misses_;
      }
    }
    live_ += cap;
  }
  if (!b) {
    b = new Buffer();
    b->bytes = cap;
    hipError_t e;
    if (Runtime::get().host_visible) {
      e = hipHostMalloc(&b->ptr, cap, hipHostMallocDefault);
      b->host_visible = true;
    } else if (arena) {
      // No stream-ordered allocation inside a captured stream: it would
      // become a node of the graph.
      e = hipMalloc(&b->ptr, cap);
      b->stream_ordered = false;
    } else {
      e = hipMallocAsync(&b->ptr, cap, Runtime::get().stream());
    }
    if (e != hipSuccess && !arena) {
      // A failed allocation may be fragmentation: give back what the pool
      // holds and try once more.
      (void)hipGetLastError();
      drain();
      if (!b->host_visible) e = hipMallocAsync(&b->ptr, cap, Runtime::get().stream());
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      delete b;
      std::lock_guard<std::mutex> g(mu_);
      live_ -= cap;
      fail("device allocation of %zu bytes failed: %s", cap, hipGetErrorString(e));
    }
  }
  b->requested = nbytes;
  b->out = true;
  if (arena && b->arena != arena) {
    std::lock_guard<std::mutex> g(mu_);
    b->arena = arena;
    arena->owned.push_back(b);
    arena->bytes += b->bytes;
  }
  return BufferP(b, [this](Buffer* x) { release(x); });
}

void Pool::free_now(Buffer* b) {
  // Work still queued on the stream may read this buffer: free in stream
  // order (or after the stream drains, for memory that is not stream-ordered).
  if (b->host_visible) {
    (void)hipStreamSynchronize(Runtime::get().stream());
    (void)hipHostFree(b->ptr);
  } else if (b->stream_ordered) {
    (void)hipFreeAsync(b->ptr, Runtime::get().stream());
  } else {
    (void)hipStreamSynchronize(Runtime::get().stream());
    (void)hipFree(b->ptr);
  }
  delete b;
}

void Pool::release(Buffer* b) {
  bool keep;
  {
    std::lock_guard<std::mutex> g(mu_);
    live_ -= b->bytes;
    b->out = false;
    if (b->arena) {
      // Owned by a captured graph: reusable within its own capture only.
      if (b->arena->capturing) b->arena->free[b->bytes].push_back(b);
      return;
    }
    if (active_) {
      // Allocated before the capture and let go during it: a recorded kernel
      // may read it (an input of the graph), so it stays with the graph until
      // the graph is destroyed: neither reused by the graph's later nodes
      // (a replay would read what they wrote) nor by work after the capture.
      b->arena = active_;
      active_->owned.push_back(b);
      active_->bytes += b->bytes;
      return;
    }
    keep = pooled_ + b->bytes <= watermark_;
    if (keep) {
      buckets_[b->bytes].push_back(b);
      pooled_ += b->bytes;
    }
  }
  if (!keep) free_now(b);
}

void Pool::begin_capture(Arena* a) {
  std::lock_guard<std::mutex> g(mu_);
  if (active_) fail("a graph capture is already active");
  active_ = a;
}

void Pool::end_capture() {
  std::lock_guard<std::mutex> g(mu_);
  if (active_) active_->capturing = false;
  active_ = nullptr;
}

bool Pool::capturing() {
  std::lock_guard<std::mutex> g(mu_);
  return active_ != nullptr;
}

void Pool::release_arena(Arena* a) {
  std::vector<Buffer*> drop;
  {
    std::lock_guard<std::mutex> g(mu_);
    if (active_ == a) active_ = nullptr;
    for (Buffer* b : a->owned) {
      b->arena = nullptr;
      if (b->out) continue;  // still referenced: pooled when its last owner lets go
      if (pooled_ + b->bytes <= watermark_) {
        buckets_[b->bytes].push_back(b);
        pooled_ += b->bytes;
      } else {
        drop.push_back(b);
      }
    }
    a->owned.clear();
    a->free.clear();
  }
  for (Buffer* b : drop) free_now(b);
}

void Pool::set_watermark(size_t bytes) {
  std::vector<Buffer*> drop;
  {
    std::lock_guard<std::mutex> g(mu_);
    if (active_) fail("the pool cannot shrink while a graph capture is active");
    watermark_ = bytes;
    while (pooled_ > watermark_ && !buckets_.empty()) {
      auto it = std::prev(buckets_.end());  // largest bucket first
      if (it->second.empty()) { buckets_.erase(it); continue; }
      drop.push_back(it->second.back());
      it->second.pop_back();
      pooled_ -= drop.back()->bytes;
      if (it->second.empty()) buckets_.erase(it);
    }
  }
  for (Buffer* b : drop) free_now(b);
}

void Pool::drain() {
  size_t w;
  {
    std::lock_guard<std::mutex> g(mu_);
    w = watermark_;
  }
  set_watermark(0);
  std::lock_guard<std::mutex> g(mu_);
  watermark_ = w;
}

PoolStats Pool::stats() {
  std::lock_guard<std::mutex> g(mu_);
  PoolStats s;
  s.hits = hits_;
  s.misses = misses_;
  s.pooled_bytes = pooled_;
  s.live_bytes = live_;
  for (auto& kv : buckets_)
    if (!kv.second.empty()) ++s.bucket_count;
  return s;
}

// ── runtime ────────────────────────────────────────────────────────────────
static Runtime* g_rt = nullptr;
static std::string g_init_err;
static std::once_flag g_once;

static size_t env_mb(const char* name, size_t dflt) {
  const char* v = getenv(name);
  if (!v || !*v) return dflt;
  return (size_t)strtoull(v, nullptr, 10) * 1024 * 1024;
}

bool Runtime::init(std::string* err) {
  std::call_once(g_once, [] {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
      (void)hipGetLastError();
      g_init_err = std::string("no HIP device available: ") +
                   (e != hipSuccess ? hipGetErrorString(e) : "device count is 0");
      return;
    }
    auto* rt = new Runtime();
    if (hipSetDevice(0) != hipSuccess) {
      g_init_err = "hipSetDevice(0) failed";
      delete rt;
      return;
    }
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) {
      g_init_err = "hipGetDeviceProperties failed";
      delete rt;
      return;
    }
    rt->info_.name = p.name;
    rt->info_.arch = p.gcnArchName;
    rt->info_.cu_count = p.multiProcessorCount;
    rt->info_.lds_per_block = p.sharedMemPerBlock;
    rt->info_.total_mem = p.totalGlobalMem;
    rt->info_.warp_size = p.warpSize;
    if (rt->info_.arch.rfind("gfx950", 0) != 0) {
      g_init_err = "this build targets gfx950 (MI355X); device reports " + rt->info_.arch;
      delete rt;
      return;
    }
    if (!noalloc_setup(&g_init_err) || !k::split_counters_setup(&g_init_err)) {
      delete rt;
      return;
    }
    if (hipStreamCreateWithFlags(&rt->stream_, hipStreamNonBlocking) != hipSuccess) {
      g_init_err = "hipStreamCreate failed";
      delete rt;
      return;
    }
    // Stream-ordered allocations come from the device's default pool; keep
    // what it holds across synchronisations (the pool above caches buffers
    // by size class, so the driver pool only backs misses).
    hipMemPool_t mp;
    if (hipDeviceGetDefaultMemPool(&mp, 0) == hipSuccess) {
      uint64_t keep_all = UINT64_MAX;
      (void)hipMemPoolSetAttribute(mp, hipMemPoolAttrReleaseThreshold, &keep_all);
    }
    (void)hipGetLastError();
    const char* hv = getenv("APPLEGPU_HOST_VISIBLE");
    rt->host_visible = hv && *hv && *hv != '0';
    // The reference pool keeps 256 MB (crates/core/src/eager.rs:83); one
    // MI355X has 288 GB of HBM, so the default watermark here is 8 GB.
    rt->pool_ = new Pool(env_mb("APPLEGPU_POOL_WATERMARK_MB", (size_t)8 << 30));
    rt->max_tensor_bytes = env_mb("APPLEGPU_MAX_TENSOR_SIZE_MB", 0);
    rt->max_memory_bytes = env_mb("APPLEGPU_MAX_MEMORY_MB", 0);
    const char* mt = getenv("APPLEGPU_MAX_TENSORS");
    rt->max_tensors = mt ? strtoull(mt, nullptr, 10) : 0;
    g_rt = rt;
  });
  if (!g_rt && err) *err = g_init_err;
  return g_rt != nullptr;
}

bool Runtime::initialized() { return g_rt != nullptr; }

Runtime& Runtime::get() {
  if (!g_rt) {
    std::string err;
    if (!init(&err)) throw Error("applegpu runtime not initialized: " + err);
  }
  return *g_rt;
}

TensorP Runtime::alloc(DType dt, const std::vector<int64_t>& dims) {
  TensorP t = make_meta(dt, dims);
  size_t nb = t->nbytes();
  if (max_tensor_bytes && nb > max_tensor_bytes)
    fail("tensor of %zu bytes exceeds the limit of %zu bytes", nb, max_tensor_bytes);
  if (max_memory_bytes && pool_->stats().live_bytes + nb > max_memory_bytes)
    fail("allocation of %zu bytes exceeds the memory limit of %zu bytes", nb, max_memory_bytes);
  t->buf = pool_->acquire(nb == 0 ? 4 : nb);
  return t;
}

void Runtime::sync() {
  // While a capture records the stream nothing executes, so there is
  // nothing to wait for (and a synchronize would end the capture).
  if (pool_->capturing()) return;
  AGPU_HIP(hipStreamSynchronize(stream_));
}

uint64_t Runtime::insert(TensorP t) { return insert_with_id(next_tensor_id(), std::move(t)); }

uint64_t Runtime::insert_with_id(uint64_t id, TensorP t) {
  std::lock_guard<std::mutex> g(reg_mu_);
  if (max_tensors && tensors_.size() >= max_tensors)
    fail("tensor count limit of %zu reached", max_tensors);
  t->ext_refs++;
  auto it = tensors_.find(id);
  if (it != tensors_.end()) it->second->ext_refs--;
  tensors_[id] = std::move(t);
  return id;
}

TensorP Runtime::lookup(uint64_t id) {
  std::lock_guard<std::mutex> g(reg_mu_);
  auto it = tensors_.find(id);
  if (it == tensors_.end()) fail("tensor %llu not found", (unsigned long long)id);
  return it->second;
}

TensorP Runtime::try_lookup(uint64_t id) {
  std::lock_guard<std::mutex> g(reg_mu_);
  auto it = tensors_.find(id);
  return it == tensors_.end() ? nullptr : it->second;
}

void Runtime::replace(uint64_t id, TensorP t) {
  std::lock_guard<std::mutex> g(reg_mu_);
  t->ext_refs++;
  auto it = tensors_.find(id);
  if (it != tensors_.end()) it->second->ext_refs--;
  tensors_[id] = std::move(t);
}

bool Runtime::erase(uint64_t id) {
  TensorP keep;  // destroyed outside the registry lock
  std::lock_guard<std::mutex> g(reg_mu_);
  auto it = tensors_.find(id);
  if (it == tensors_.end()) return false;
  keep = std::move(it->second);
  keep->ext_refs--;
  tensors_.erase(it);
  return true;
}

size_t Runtime::count() {
  std::lock_guard<std::mutex> g(reg_mu_);
  return tensors_.size();
}

size_t Runtime::memory_usage() { return pool_->stats().live_bytes; }

// Reverse lookup (crates/core/src/eager_ffi.rs:612-633): prefer a base tensor
// (offset 0) whose storage starts at `p`, then any tensor on that storage.
uint64_t Runtime::find_by_data_ptr(const void* p) {
  std::lock_guard<std::mutex> g(reg_mu_);
  uint64_t any = 0;
  for (auto& kv : tensors_) {
    const TensorP& t = kv.second;
    if (!t->buf || t->buf->ptr != p) continue;
    if (t->offset == 0) return kv.first;
    if (!any) any = kv.first;
  }
  return any;
}

}  // namespace agpu
