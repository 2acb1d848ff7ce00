// Device-side helpers shared by the gfx950 kernels: element types, float
// conversion, wavefront reductions and dtype dispatch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../kernels.hpp"

namespace agpu {
namespace dev {

typedef _Float16 half_t;
typedef __bf16 bf16_t;

template <typename T> __device__ __forceinline__ float to_f(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x) { return (T)x; }
template <> __device__ __forceinline__ bool from_f<bool>(float x) { return x != 0.f; }

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// GELU, tanh approximation (crates/core/src/kernel_templates.rs:272-307):
// 0.5 x (1 + tanh(u)), u = clamp(0.7978845608 (x + 0.044715 x^3), -10, 10).
// Evaluated through the identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)): one
// exp2 and one reciprocal instead of tanh, the same function to within a few
// fp32 ulp (no cancellation: the 1 + tanh sum is formed exactly).
__device__ __forceinline__ float gelu_tanh(float x) {
  float u = 0.7978845608f * (x + 0.044715f * x * x * x);
  u = fminf(fmaxf(u, -10.f), 10.f);
  // exp(-2u) as the hardware exp2 of -2u log2(e) and the division as the
  // hardware reciprocal (about 1 ulp each): with u clamped to +-10 the
  // exponent stays within +-28.9, so neither underflows nor overflows, and
  // the result stays within a few ulp of x / (1 + exp(-2u))
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(u * -2.8853900817779268f));
}

// Read-ahead blocks: a launch may carry extra blocks that read one dword of
// every 64-byte line of up to three ranges (the weights of the next GEMMs),
// so that those lines are in the memory-side Infinity Cache and the L2 when
// the GEMMs run; blocks from `first` on do this and return before anything
// else (no barrier is reached).  The loaded values feed an empty asm
// statement, so the loads are kept, and nothing is stored.
struct PfArgs {
  const char* p[3];
  int64_t lines[3];
  int n;
  int first;   // first read-ahead block (gridDim.x when there are none)
  int blocks;  // read-ahead blocks
};
// The reads of read-ahead block `b` (0 .. pf.blocks - 1).
__device__ __forceinline__ void prefetch_lines(const PfArgs& pf, int64_t b) {
  const int64_t stride = (int64_t)pf.blocks * blockDim.x;
  const int64_t t0 = b * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (int r = 0; r < pf.n; ++r) {
#pragma unroll 4
    for (int64_t l = t0; l < pf.lines[r]; l += stride) acc ^= *(const uint32_t*)(pf.p[r] + (l << 6));
  }
  asm volatile("" ::"v"(acc));
}
__device__ __forceinline__ bool prefetch_block(const PfArgs& pf) {
  if ((int)blockIdx.x < pf.first) return false;
  const int64_t stride = (int64_t)pf.blocks * blockDim.x;
  const int64_t t0 = (int64_t)(blockIdx.x - pf.first) * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (int r = 0; r < pf.n; ++r) {
#pragma unroll 4
    for (int64_t l = t0; l < pf.lines[r]; l += stride) acc ^= *(const uint32_t*)(pf.p[r] + (l << 6));
  }
  asm volatile("" ::"v"(acc));
  return true;
}

}  // namespace dev
namespace k {
// Read-ahead blocks for a launch of `main` blocks of `threads` threads: the
// pending ranges (take_prefetch, which clears them), one block per 32 KB of
// lines, at most 256; none when no range is pending.
dev::PfArgs make_prefetch(int main, int threads);
}  // namespace k
namespace dev {

// Launch geometry helpers
inline unsigned blocks_for(int64_t n, int per_block) {
  int64_t b = (n + per_block - 1) / per_block;
  return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace dev
}  // namespace agpu

// Dispatch on a float dtype (f32/f16/bf16); `T` is bound inside the body.
#define AGPU_FLOAT_SWITCH(dt, ...)                                              \
  switch (dt) {                                                                 \
    case ::agpu::DType::F32: { typedef float T; __VA_ARGS__; break; }          \
    case ::agpu::DType::F16: { typedef ::agpu::dev::half_t T; __VA_ARGS__; break; } \
    case ::agpu::DType::BF16: { typedef ::agpu::dev::bf16_t T; __VA_ARGS__; break; } \
    default: ::agpu::fail("dtype %s not supported by this kernel", ::agpu::dtype_name(dt)); \
  }

// Dispatch on every dtype the kernels compute in (no f64 on this path).
#define AGPU_ALL_SWITCH(dt, ...)                                                \
  switch (dt) {                                                                 \
    case ::agpu::DType::F32: { typedef float T; __VA_ARGS__; break; }          \
    case ::agpu::DType::F16: { typedef ::agpu::dev::half_t T; __VA_ARGS__; break; } \
    case ::agpu::DType::BF16: { typedef ::agpu::dev::bf16_t T; __VA_ARGS__; break; } \
    case ::agpu::DType::I8: { typedef int8_t T; __VA_ARGS__; break; }          \
    case ::agpu::DType::I16: { typedef int16_t T; __VA_ARGS__; break; }        \
    case ::agpu::DType::I32: { typedef int32_t T; __VA_ARGS__; break; }        \
    case ::agpu::DType::I64: { typedef int64_t T; __VA_ARGS__; break; }        \
    case ::agpu::DType::U8: { typedef uint8_t T; __VA_ARGS__; break; }         \
    case ::agpu::DType::U32: { typedef uint32_t T; __VA_ARGS__; break; }       \
    case ::agpu::DType::Bool: { typedef bool T; __VA_ARGS__; break; }          \
    default: ::agpu::fail("dtype %s not supported on this device path", ::agpu::dtype_name(dt)); \
  }

#define AGPU_INT_SWITCH(dt, ...)                                                \
  switch (dt) {                                                                 \
    case ::agpu::DType::I32: { typedef int32_t I; __VA_ARGS__; break; }        \
    case ::agpu::DType::I64: { typedef int64_t I; __VA_ARGS__; break; }        \
    default: ::agpu::fail("index dtype must be int32 or int64, got %s", ::agpu::dtype_name(dt)); \
  }
