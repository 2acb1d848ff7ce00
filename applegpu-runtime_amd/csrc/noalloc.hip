// Device scratch of the allocation-free entry point
// (applegpu_eager_linear_noalloc): the split-K partial sums of its GEMM live
// in one file-scope device array instead of a pooled buffer, so the call
// makes no device allocation.  The loader places a copy of the array on
// every GPU the library's code object is loaded on, held until the process
// ends; the host reaches each copy only through the address
// hipGetSymbolAddress returns on that device (the array's name is a host
// stand-in that must never reach a kernel argument or a copy).
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "core.hpp"

namespace agpu {

namespace {

// Split-K partials of one GEMM: splits x M x N fp32.  The planner splits only
// a grid with fewer tiles than the GPU has CUs (256) and stops doubling the
// split count once tiles x splits reaches two per CU, so a 2-D product has
// fewer than 1024 tile-splits of at most 128 x 128 fp32 partials: under
// 64 MiB.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

}  // namespace

bool noalloc_setup(std::string* err) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    if (err) *err = "allocation-free scratch: no current device";
    return false;
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev]) return true;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) {
    (void)hipGetLastError();
    if (err)
      *err = std::string("allocation-free scratch: hipGetSymbolAddress failed: ") +
             (e != hipSuccess ? hipGetErrorString(e) : "null address");
    return false;
  }
  g_scratch_ptr[dev] = p;
  return true;
}

void* noalloc_scratch(size_t* cap) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    fail("allocation-free scratch: no current device");
  }
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    p = g_scratch_ptr[dev];
  }
  if (!p) {
    std::string err;
    if (!noalloc_setup(&err)) fail("%s", err.c_str());
    std::lock_guard<std::mutex> g(g_scratch_mu);
    p = g_scratch_ptr[dev];
  }
  *cap = kScratchBytes;
  return p;
}

}  // namespace agpu
