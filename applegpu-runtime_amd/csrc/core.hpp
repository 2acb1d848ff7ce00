// Core types of the MI355X runtime: dtypes, device buffers and their pool,
// stride-aware tensors, the single HIP stream, and the process-wide registry
// that maps the C ABI's u64 ids to tensors.
//
// Reference semantics followed (paths relative to the reference checkout):
//   dtype wire codes            crates/core/src/tensor.rs:59-90
//   MAX_DIMS = 8                crates/core/src/tensor.rs:113
//   id counter starting at 1    crates/core/src/tensor.rs:292-299
//   power-of-two bucket pool    crates/core/src/pool.rs:35-66
//   EagerTensor {buffer,layout,dtype,byte offset}   crates/core/src/eager.rs:11-20
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace agpu {

// ── dtypes ────────────────────────────────────────────────────────────────
enum class DType : int8_t {
  F32 = 0, F16 = 1, F64 = 2, I8 = 3, I16 = 4, I32 = 5, I64 = 6,
  U8 = 7, U32 = 8, Bool = 9, BF16 = 10,
};

size_t dtype_size(DType d);
const char* dtype_name(DType d);
bool dtype_is_float(DType d);
bool dtype_from_wire(int v, DType* out);
bool dtype_from_name(const std::string& s, DType* out);

constexpr int kMaxDims = 8;

// ── errors ────────────────────────────────────────────────────────────────
struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};
[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define AGPU_HIP(call)                                                        \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess)                                                     \
      ::agpu::fail("%s failed: %s", #call, hipGetErrorString(e_));            \
  } while (0)

// Checks the launch that was just enqueued.
void check_launch(const char* what);
// Number of check_launch calls since the library loaded: one per kernel
// launcher call on this path (the lazy executor's fusion tests count them).
uint64_t launcher_calls();

// Device scratch of the allocation-free entry point (csrc/noalloc.hip):
// noalloc_setup looks up the scratch array's address on the current device
// (the runtime's init calls it once the device is current); noalloc_scratch
// returns that address and the array's size in bytes.
bool noalloc_setup(std::string* err);
void* noalloc_scratch(size_t* cap);

// ── device buffers ────────────────────────────────────────────────────────
struct Arena;

struct Buffer {
  void* ptr = nullptr;
  size_t bytes = 0;       // capacity (a power of two when pooled)
  size_t requested = 0;   // bytes the current owner asked for (bounds of views)
  bool host_visible = false;
  bool stream_ordered = true;  // hipMallocAsync'd; false: hipMalloc'd during a capture
  bool out = false;            // handed out and not yet released
  Arena* arena = nullptr;      // set while a captured graph owns the buffer
};
using BufferP = std::shared_ptr<Buffer>;

// The buffers of one captured graph: every buffer handed out while its
// capture is active.  Buffers released during the capture go back to the
// arena's own free lists (later ops of the same capture reuse them, in stream
// order); none leaves the arena until the graph is destroyed, because every
// replay writes them again.
struct Arena {
  std::vector<Buffer*> owned;
  std::map<size_t, std::vector<Buffer*>> free;
  bool capturing = true;
  size_t bytes = 0;
};

struct PoolStats {
  uint64_t hits = 0, misses = 0;
  size_t pooled_bytes = 0, bucket_count = 0, live_bytes = 0;
};

// Power-of-two bucketed pool over stream-ordered hipMallocAsync.  Every kernel runs on the one
// runtime stream, so a buffer released on the host can be handed to the next
// op at once: the next op's kernels are ordered after the last user's.
class Pool {
 public:
  explicit Pool(size_t watermark) : watermark_(watermark) {}
  BufferP acquire(size_t nbytes);
  void set_watermark(size_t bytes);
  void drain();
  PoolStats stats();
  // Test hook: make the next `n` device allocations fail.
  void inject_failures(int n) { inject_fail_ = n; }

  // Graph capture: route allocations through `a` until end_capture; then
  // the arena holds its buffers until release_arena hands them back.
  void begin_capture(Arena* a);
  void end_capture();
  void release_arena(Arena* a);
  bool capturing();

 private:
  void release(Buffer* b);
  void free_now(Buffer* b);
  Arena* active_ = nullptr;
  std::mutex mu_;
  std::map<size_t, std::vector<Buffer*>> buckets_;
  size_t watermark_;
  size_t pooled_ = 0;
  size_t live_ = 0;
  uint64_t hits_ = 0, misses_ = 0;
  int inject_fail_ = 0;
};

// ── tensors ───────────────────────────────────────────────────────────────
struct Node;  // pending lazy op (lazy.cpp)

struct Tensor {
  DType dtype = DType::F32;
  int ndim = 0;
  int64_t shape[kMaxDims] = {};
  int64_t strides[kMaxDims] = {};  // in elements
  int64_t offset = 0;              // in bytes from buf->ptr
  BufferP buf;                     // null while the tensor is pending
  std::shared_ptr<Node> node;      // set while pending (lazy graph)
  int ext_refs = 0;                // registry ids naming this tensor (C ABI handles)

  int64_t numel() const {
    int64_t n = 1;
    for (int i = 0; i < ndim; ++i) n *= shape[i];
    return n;
  }
  size_t nbytes() const { return (size_t)numel() * dtype_size(dtype); }
  // Bytes from data() to one past the last element the strides reach.
  size_t extent_bytes() const {
    if (numel() == 0) return 0;
    int64_t last = 0;
    for (int i = 0; i < ndim; ++i) last += (shape[i] - 1) * strides[i];
    return (size_t)(last + 1) * dtype_size(dtype);
  }
  bool is_contiguous() const;
  bool pending() const { return node != nullptr; }
  char* data() const { return buf ? (char*)buf->ptr + offset : nullptr; }
  std::vector<int64_t> dims() const { return std::vector<int64_t>(shape, shape + ndim); }
  void set_contiguous_strides();
};
using TensorP = std::shared_ptr<Tensor>;

// A tensor description without storage (used for shape inference).
TensorP make_meta(DType dt, const std::vector<int64_t>& dims);

// ── runtime ───────────────────────────────────────────────────────────────
struct DeviceInfo {
  std::string name, arch;
  int cu_count = 0;
  size_t lds_per_block = 0;
  size_t total_mem = 0;
  int warp_size = 64;
};

class Runtime {
 public:
  static Runtime& get();             // throws if init failed
  static bool init(std::string* err);  // idempotent
  static bool initialized();

  hipStream_t stream() const { return stream_; }
  Pool& pool() { return *pool_; }
  const DeviceInfo& info() const { return info_; }

  // Allocate a contiguous device tensor (zero-byte tensors get 4 bytes,
  // crates/core/src/eager.rs:99).
  TensorP alloc(DType dt, const std::vector<int64_t>& dims);
  void sync();

  // id registry
  uint64_t insert(TensorP t);
  uint64_t insert_with_id(uint64_t id, TensorP t);
  TensorP lookup(uint64_t id);           // throws on unknown id
  TensorP try_lookup(uint64_t id);       // null on unknown id
  bool erase(uint64_t id);
  size_t count();
  size_t memory_usage();
  uint64_t find_by_data_ptr(const void* p);
  void replace(uint64_t id, TensorP t);

  std::recursive_mutex& big_lock() { return big_; }

  // Resource limits (crates/core/src/limits.rs:39-77); 0 = unlimited.
  size_t max_tensor_bytes = 0, max_memory_bytes = 0, max_tensors = 0;

  // Optional host-visible allocations (APPLEGPU_HOST_VISIBLE=1) for callers
  // that poke returned pointers from the host.
  bool host_visible = false;

 private:
  Runtime() = default;
  hipStream_t stream_ = nullptr;
  Pool* pool_ = nullptr;
  DeviceInfo info_;
  std::recursive_mutex big_;
  std::mutex reg_mu_;
  std::unordered_map<uint64_t, TensorP> tensors_;
};

uint64_t next_tensor_id();

// Small helpers shared by ops and the graph.
std::vector<int64_t> broadcast_shapes(const std::vector<int64_t>& a, const std::vector<int64_t>& b);
std::string shape_str(const std::vector<int64_t>& d);

}  // namespace agpu
