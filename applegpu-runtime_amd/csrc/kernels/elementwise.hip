// Elementwise kernels: N-D strided binary/unary/where with broadcast, bias add,
// axpy (the SGD update), triangular masks.
//
// Reference semantics (crates/core/src/kernel_templates.rs):
//   binary ops over nd_index_to_offset          :41-88
//   float unary ops (relu = max(x,0), ...)       :119-168
//   gelu (tanh form, inner clamped to +-10)      :272-307
//   gelu_exact (erf)                             :311-360
//   add_bias (channel = (i / stride) % C)        :747-762
//   threshold_backward (g if x > thr else 0)     :1996-2020
//   quantize / dequantize (per-tensor)           :2193-2240
//   integer mod is C remainder `a % b`           :2446
// Differences on purpose: offsets and strides are 64-bit, every op honours
// view strides and byte offsets, and contiguous operands take a vectorised
// path (16-byte loads).
#include "device.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

template <typename T> struct Compute { typedef T type; };
template <> struct Compute<half_t> { typedef float type; };
template <> struct Compute<bf16_t> { typedef float type; };
template <> struct Compute<bool> { typedef bool type; };

template <typename T> __device__ __forceinline__ bool is_float_t() { return false; }
template <> __device__ __forceinline__ bool is_float_t<float>() { return true; }

// gelu with the tanh approximation; the reference clamps the inner term to
// +-10 before tanh (kernel_templates.rs:300-301), a no-op for fp32 tanh.
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }

// d/dx of gelu_tanh, with the forward's clamp of the inner term to +-10
// (kernel_templates.rs:2074-2096 and :2100-2122 compute the same):
// 0.5 (1 + t) + 0.5 x (1 - t^2) k (1 + 3 * 0.044715 x^2), t = tanh(k (x + 0.044715 x^3)).
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float k = 0.7978845608028654f;
  const float u = fminf(fmaxf(k * (x + 0.044715f * x * x * x), -10.f), 10.f);
  const float t = tanhf(u);
  return 0.5f * (1.f + t) + 0.5f * x * (1.f - t * t) * k * (1.f + 3.f * 0.044715f * x * x);
}

// d/dx of x * Phi(x): Phi(x) + x * phi(x) (kernel_templates.rs:2126-2152).
__device__ __forceinline__ float gelu_erf_grad(float x) {
  const float cdf = 0.5f * (1.f + erff(x * 0.70710678118654752f));
  const float pdf = 0.3989422804014327f * expf(-0.5f * x * x);
  return cdf + x * pdf;
}

template <typename C>
__device__ __forceinline__ C bin_apply(int op, C a, C b, float p0) {
  switch (op) {
    case kAdd: return a + b;
    case kSub: return a - b;
    case kMul: return a * b;
    case kDiv:
      if constexpr (std::is_integral<C>::value) return b == 0 ? C(0) : C(a / b);
      else return a / b;
    case kMin: return a < b ? a : b;
    case kMax: return a > b ? a : b;
    case kMod:
      if constexpr (std::is_integral<C>::value) return b == 0 ? C(0) : C(a % b);
      else return fmodf(a, b);
    case kAnd: if constexpr (std::is_integral<C>::value) return a & b; else return 0;
    case kOr: if constexpr (std::is_integral<C>::value) return a | b; else return 0;
    case kXor: if constexpr (std::is_integral<C>::value) return a ^ b; else return 0;
    case kLt: return a < b;
    case kGt: return a > b;
    case kLe: return a <= b;
    case kGe: return a >= b;
    case kEq: return a == b;
    case kNe: return a != b;
    case kThresholdBwd: return (float)b > p0 ? a : C(0);
    case kGeluBwd:
      if constexpr (std::is_floating_point<C>::value) return a * gelu_tanh_grad(b);
      else return C(0);
    case kGeluExactBwd:
      if constexpr (std::is_floating_point<C>::value) return a * gelu_erf_grad(b);
      else return C(0);
  }
  return C(0);
}

template <typename C>
__device__ __forceinline__ C un_apply(int op, C x, float p0, float p1) {
  if constexpr (std::is_same<C, float>::value) {
    switch (op) {
      case kNeg: return -x;
      case kRelu: return fmaxf(x, 0.f);
      case kExp: return expf(x);
      case kLog: return logf(x);
      case kSqrt: return sqrtf(x);
      case kAbs: return fabsf(x);
      case kSign: return (float)((x > 0.f) - (x < 0.f));
      case kTanh: return tanhf(x);
      case kSin: return sinf(x);
      case kCos: return cosf(x);
      case kSigmoid: return 1.f / (1.f + expf(-x));
      case kGelu: return gelu_tanh(x);
      case kGeluExact: return gelu_erf(x);
      case kScale: return x * p0;
      case kPow: return powf(x, p0);
      case kClamp: return fminf(fmaxf(x, p0), p1);
      case kLogicalNot: return x == 0.f ? 1.f : 0.f;
      case kCopy: return x;
      case kFill: return p0;
    }
    return x;
  } else {
    switch (op) {
      case kNeg: return (C)(-x);
      case kRelu: return x > 0 ? x : C(0);
      case kAbs: return x < 0 ? (C)(-x) : x;
      case kSign: return (C)((x > 0) - (x < 0));
      case kScale: return (C)((float)x * p0);
      case kClamp: return (C)fminf(fmaxf((float)x, p0), p1);
      case kBitNot:
        if constexpr (std::is_same<C, bool>::value) return !x;
        else return (C)(~x);
      case kLogicalNot: return x == 0 ? C(1) : C(0);
      case kShl: return (C)(x << (int)p0);
      case kShr: return (C)(x >> (int)p0);
      case kCopy: return x;
      case kFill: return (C)p0;
    }
    return x;
  }
}

// Decode a flat index of the contiguous output into an operand offset.
template <typename I>
__device__ __forceinline__ I nd_offset(I flat, const ND& shape, const ND& s) {
  I off = 0;
  for (int d = shape.ndim - 1; d >= 0; --d) {
    I sz = (I)shape.shape[d];
    I i = flat % sz;
    flat /= sz;
    off += i * (I)s.stride[d];
  }
  return off;
}

template <typename I, typename TI, typename TO>
__global__ void __launch_bounds__(256) binary_nd(int op, const TI* __restrict__ a, ND sa,
                                                 const TI* __restrict__ b, ND sb,
                                                 TO* __restrict__ o, ND so, I n, float p0) {
  typedef typename Compute<TI>::type C;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    C x = (C)a[nd_offset<I>(i, so, sa)];
    C y = (C)b[nd_offset<I>(i, so, sb)];
    o[i] = (TO)bin_apply<C>(op, x, y, p0);
  }
}

// Contiguous, same-shape operands: 4 elements per thread.
template <typename TI, typename TO>
__global__ void __launch_bounds__(256) binary_flat(int op, const TI* __restrict__ a,
                                                   const TI* __restrict__ b, TO* __restrict__ o,
                                                   int64_t n, float p0) {
  typedef typename Compute<TI>::type C;
  int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (base + 4 <= n) {
    TI av[4], bv[4];
    TO ov[4];
    if constexpr (sizeof(TI) == 4) {
      *(float4*)av = *(const float4*)(a + base);
      *(float4*)bv = *(const float4*)(b + base);
    } else if constexpr (sizeof(TI) == 2) {
      *(float2*)av = *(const float2*)(a + base);
      *(float2*)bv = *(const float2*)(b + base);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) { av[j] = a[base + j]; bv[j] = b[base + j]; }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) ov[j] = (TO)bin_apply<C>(op, (C)av[j], (C)bv[j], p0);
    if constexpr (sizeof(TO) == 4) *(float4*)(o + base) = *(float4*)ov;
    else if constexpr (sizeof(TO) == 2) *(float2*)(o + base) = *(float2*)ov;
    else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[base + j] = ov[j];
    }
  } else {
    for (int64_t i = base; i < n; ++i) o[i] = (TO)bin_apply<C>(op, (C)a[i], (C)b[i], p0);
  }
}

template <typename I, typename TI, typename TO>
__global__ void __launch_bounds__(256) unary_nd(int op, const TI* __restrict__ x, ND sx,
                                                TO* __restrict__ o, ND so, I n, float p0, float p1) {
  typedef typename Compute<TI>::type C;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    C v = (C)x[nd_offset<I>(i, so, sx)];
    o[i] = (TO)un_apply<C>(op, v, p0, p1);  // float -> int casts truncate (C semantics)
  }
}

template <typename TI, typename TO>
__global__ void __launch_bounds__(256) unary_flat(int op, const TI* __restrict__ x,
                                                  TO* __restrict__ o, int64_t n, float p0, float p1) {
  typedef typename Compute<TI>::type C;
  int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (base + 4 <= n) {
    TI xv[4];
    TO ov[4];
    if constexpr (sizeof(TI) == 4) *(float4*)xv = *(const float4*)(x + base);
    else if constexpr (sizeof(TI) == 2) *(float2*)xv = *(const float2*)(x + base);
    else {
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[j] = x[base + j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) ov[j] = (TO)un_apply<C>(op, (C)xv[j], p0, p1);
    if constexpr (sizeof(TO) == 4) *(float4*)(o + base) = *(float4*)ov;
    else if constexpr (sizeof(TO) == 2) *(float2*)(o + base) = *(float2*)ov;
    else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[base + j] = ov[j];
    }
  } else {
    for (int64_t i = base; i < n; ++i) o[i] = (TO)un_apply<C>(op, (C)x[i], p0, p1);
  }
}

// Per-tensor quantize with MSL-style round (half away from zero) and the
// zero point added after rounding (kernel_templates.rs:2207-2212).
template <typename I, typename TI, typename TO>
__global__ void __launch_bounds__(256) quantize_nd(const TI* __restrict__ x, ND sx, TO* __restrict__ o,
                                                   ND so, I n, float scale, float zp, float lo, float hi) {
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    float v = roundf((float)x[nd_offset<I>(i, so, sx)] / scale) + zp;
    v = fminf(fmaxf(v, lo), hi);
    o[i] = (TO)(int)v;
  }
}

template <typename I, typename TI, typename TO>
__global__ void __launch_bounds__(256) dequantize_nd(const TI* __restrict__ x, ND sx, TO* __restrict__ o,
                                                     ND so, I n, float scale, int zp) {
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    int q = (int)x[nd_offset<I>(i, so, sx)];
    o[i] = (TO)((float)(q - zp) * scale);
  }
}

template <typename I, typename TC, typename T>
__global__ void __launch_bounds__(256) where_nd(const TC* __restrict__ c, ND sc, const T* __restrict__ x, ND sx,
                                                const T* __restrict__ y, ND sy, T* __restrict__ o, ND so, I n) {
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    bool take = c[nd_offset<I>(i, so, sc)] != TC(0);
    o[i] = take ? x[nd_offset<I>(i, so, sx)] : y[nd_offset<I>(i, so, sy)];
  }
}

template <typename T>
__global__ void __launch_bounds__(256) tri_kernel(const T* __restrict__ x, T* __restrict__ o, int64_t n,
                                                  int64_t rows, int64_t cols, int64_t diag, bool upper) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t c = i % cols;
    int64_t r = (i / cols) % rows;
    bool keep = upper ? (c - r >= diag) : (c - r <= diag);
    o[i] = keep ? x[i] : T(0);
  }
}

template <typename I, typename T>
__global__ void __launch_bounds__(256) axpy_nd(T* __restrict__ y, const T* __restrict__ x, ND sx, ND sy,
                                               I n, float alpha) {
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    float v = (float)y[i] + alpha * (float)x[nd_offset<I>(i, sy, sx)];
    y[i] = (T)v;
  }
}

// y += alpha * x over contiguous float32 data, 4 per thread.
__global__ void __launch_bounds__(256) axpy_flat_f32(float* __restrict__ y, const float* __restrict__ x,
                                                     int64_t n, float alpha) {
  int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (base + 4 <= n) {
    float4 a = *(const float4*)(x + base);
    float4 b = *(float4*)(y + base);
    b.x += alpha * a.x; b.y += alpha * a.y; b.z += alpha * a.z; b.w += alpha * a.w;
    *(float4*)(y + base) = b;
  } else {
    for (int64_t i = base; i < n; ++i) y[i] += alpha * x[i];
  }
}

template <typename T>
__global__ void __launch_bounds__(256) add_bias_kernel(const T* __restrict__ in, const T* __restrict__ bias,
                                                       T* __restrict__ out, int64_t n, int64_t C, int64_t cs) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t ch = (i / cs) % C;
    out[i] = (T)((float)in[i] + (float)bias[ch]);
  }
}

// ── fused elementwise chains ────────────────────────────────────────────────
// Every step computes in fp32 through bin_apply/un_apply, the functions the
// unfused kernels use, and rounds to T as the unfused node's store would.
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (std::is_same<T, float>::value) return v;
  else return (float)(T)v;
}

template <typename T>
__device__ __forceinline__ float chain_step(const ChainStep& st, float acc, float v) {
  float r;
  if (st.leaf < 0) r = un_apply<float>(st.op, acc, st.p0, st.p1);
  else r = st.acc_rhs ? bin_apply<float>(st.op, v, acc, 0.f) : bin_apply<float>(st.op, acc, v, 0.f);
  return round_to<T>(r);
}

// Four consecutive elements [base, base + 4) of leaf j in the flat layout:
// element i reads leaf[i % period] (period == n: the whole output; 1: a
// scalar; otherwise a multiple of 4 that divides n, so the four are
// contiguous in the leaf).
template <typename T>
__device__ __forceinline__ void chain_load4(const ChainLeaves& L, int j, int64_t base, int64_t n, float (&v)[4]) {
  const T* p = (const T*)L.ptr[j];
  const int64_t period = L.period[j];
  if (period == 1) {
    const float s = (float)p[0];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = s;
    return;
  }
  const int64_t off = period == n ? base : base % period;
  T raw[4];
  if constexpr (sizeof(T) == 4) *(float4*)raw = *(const float4*)(p + off);
  else *(float2*)raw = *(const float2*)(p + off);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (float)raw[e];
}

// Contiguous, scalar and suffix-broadcast leaves: 4 elements per thread,
// 16-byte (fp32) or 8-byte (16-bit) loads and stores.
template <typename T>
__global__ void __launch_bounds__(256) chain_flat(ChainProgram p, ChainLeaves L, T* __restrict__ o, int64_t n) {
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (base >= n) return;
  if (base + 4 <= n) {
    float acc[4];
    chain_load4<T>(L, p.first, base, n, acc);
    for (int s = 0; s < p.n_steps; ++s) {
      const ChainStep st = p.step[s];
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (st.leaf >= 0) chain_load4<T>(L, st.leaf, base, n, v);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = chain_step<T>(st, acc[e], v[e]);
    }
    T out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (T)acc[e];
    if constexpr (sizeof(T) == 4) *(float4*)(o + base) = *(float4*)out;
    else *(float2*)(o + base) = *(float2*)out;
  } else {
    for (int64_t i = base; i < n; ++i) {
      auto at = [&](int j) { return (float)((const T*)L.ptr[j])[L.period[j] == 1 ? 0 : i % L.period[j]]; };
      float acc = at(p.first);
      for (int s = 0; s < p.n_steps; ++s) {
        const ChainStep st = p.step[s];
        acc = chain_step<T>(st, acc, st.leaf >= 0 ? at(st.leaf) : 0.f);
      }
      o[i] = (T)acc;
    }
  }
}

// Any leaf layout: each leaf read through its own strides over the output.
template <typename I, typename T>
__global__ void __launch_bounds__(256) chain_nd(ChainProgram p, ChainLeaves L, T* __restrict__ o, ND so, I n) {
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x) {
    auto at = [&](int j) { return (float)((const T*)L.ptr[j])[nd_offset<I>(i, so, L.nd[j])]; };
    float acc = at(p.first);
    for (int s = 0; s < p.n_steps; ++s) {
      const ChainStep st = p.step[s];
      acc = chain_step<T>(st, acc, st.leaf >= 0 ? at(st.leaf) : 0.f);
    }
    o[i] = (T)acc;
  }
}

bool fits32(int64_t n, const ND& a, const ND& b) {
  if (n >= (int64_t(1) << 31)) return false;
  int64_t ea = 0, eb = 0;
  for (int d = 0; d < a.ndim; ++d) ea += (a.shape[d] - 1) * a.stride[d];
  for (int d = 0; d < b.ndim; ++d) eb += (b.shape[d] - 1) * b.stride[d];
  return ea < (int64_t(1) << 31) && eb < (int64_t(1) << 31);
}

bool is_flat(const ND& s, const ND& shape) {
  int64_t expect = 1;
  for (int d = shape.ndim - 1; d >= 0; --d) {
    if (shape.shape[d] != 1 && s.stride[d] != expect) return false;
    expect *= shape.shape[d];
  }
  return true;
}

int64_t numel_of(const ND& s) {
  int64_t n = 1;
  for (int d = 0; d < s.ndim; ++d) n *= s.shape[d];
  return n;
}

unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;  // grid-stride loops cover the rest
  return (unsigned)(b < 1 ? 1 : b);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename TI, typename TO>
void launch_binary(int op, const void* a, const ND& sa, const void* b, const ND& sb, void* o,
                   const ND& so, float p0, hipStream_t s) {
  int64_t n = numel_of(so);
  if (n == 0) return;
  if (is_flat(sa, so) && is_flat(sb, so) && aligned16(a) && aligned16(b) && aligned16(o)) {
    unsigned g = (unsigned)((n + 1023) / 1024);
    hipLaunchKernelGGL((binary_flat<TI, TO>), dim3(g), dim3(256), 0, s, op, (const TI*)a,
                       (const TI*)b, (TO*)o, n, p0);
  } else if (fits32(n, sa, sb)) {
    hipLaunchKernelGGL((binary_nd<uint32_t, TI, TO>), dim3(grid_for(n)), dim3(256), 0, s, op,
                       (const TI*)a, sa, (const TI*)b, sb, (TO*)o, so, (uint32_t)n, p0);
  } else {
    hipLaunchKernelGGL((binary_nd<uint64_t, TI, TO>), dim3(grid_for(n)), dim3(256), 0, s, op,
                       (const TI*)a, sa, (const TI*)b, sb, (TO*)o, so, (uint64_t)n, p0);
  }
  check_launch("binary");
}

template <typename TI, typename TO>
void launch_unary(int op, const void* x, const ND& sx, void* o, const ND& so, float p0, float p1,
                  hipStream_t s) {
  int64_t n = numel_of(so);
  if (n == 0) return;
  if (is_flat(sx, so) && aligned16(x) && aligned16(o)) {
    unsigned g = (unsigned)((n + 1023) / 1024);
    hipLaunchKernelGGL((unary_flat<TI, TO>), dim3(g), dim3(256), 0, s, op, (const TI*)x, (TO*)o, n,
                       p0, p1);
  } else if (fits32(n, sx, sx)) {
    hipLaunchKernelGGL((unary_nd<uint32_t, TI, TO>), dim3(grid_for(n)), dim3(256), 0, s, op,
                       (const TI*)x, sx, (TO*)o, so, (uint32_t)n, p0, p1);
  } else {
    hipLaunchKernelGGL((unary_nd<uint64_t, TI, TO>), dim3(grid_for(n)), dim3(256), 0, s, op,
                       (const TI*)x, sx, (TO*)o, so, (uint64_t)n, p0, p1);
  }
  check_launch("unary");
}

// o[offset(i) through so's strides] = x[offset(i) through sx's strides]
template <typename I, typename TI, typename TO>
__global__ void __launch_bounds__(256) copy_nd_strided(const TI* __restrict__ x, ND sx, TO* __restrict__ o,
                                                       ND so, I n) {
  typedef typename Compute<TI>::type C;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (I)gridDim.x * blockDim.x)
    o[nd_offset<I>(i, so, so)] = (TO)(C)x[nd_offset<I>(i, so, sx)];
}

template <typename TI, typename TO>
void launch_copy_strided(const void* x, const ND& sx, void* o, const ND& so, hipStream_t s) {
  int64_t n = numel_of(so);
  if (n == 0) return;
  if (fits32(n, sx, so))
    hipLaunchKernelGGL((copy_nd_strided<uint32_t, TI, TO>), dim3(grid_for(n)), dim3(256), 0, s, (const TI*)x, sx,
                       (TO*)o, so, (uint32_t)n);
  else
    hipLaunchKernelGGL((copy_nd_strided<uint64_t, TI, TO>), dim3(grid_for(n)), dim3(256), 0, s, (const TI*)x, sx,
                       (TO*)o, so, (uint64_t)n);
  check_launch("copy_strided");
}

template <typename TI>
void copy_strided_to(DType out, const void* x, const ND& sx, void* o, const ND& so, hipStream_t s) {
  switch (out) {
    case DType::F32: launch_copy_strided<TI, float>(x, sx, o, so, s); break;
    case DType::F16: launch_copy_strided<TI, half_t>(x, sx, o, so, s); break;
    case DType::BF16: launch_copy_strided<TI, bf16_t>(x, sx, o, so, s); break;
    case DType::I8: launch_copy_strided<TI, int8_t>(x, sx, o, so, s); break;
    case DType::I16: launch_copy_strided<TI, int16_t>(x, sx, o, so, s); break;
    case DType::I32: launch_copy_strided<TI, int32_t>(x, sx, o, so, s); break;
    case DType::I64: launch_copy_strided<TI, int64_t>(x, sx, o, so, s); break;
    case DType::U8: launch_copy_strided<TI, uint8_t>(x, sx, o, so, s); break;
    case DType::U32: launch_copy_strided<TI, uint32_t>(x, sx, o, so, s); break;
    case DType::Bool: launch_copy_strided<TI, bool>(x, sx, o, so, s); break;
    default: fail("copy: unsupported destination dtype %s", dtype_name(out));
  }
}

}  // namespace

void copy_strided(DType in, DType out, const void* x, const ND& sx, void* o, const ND& so, hipStream_t s) {
  AGPU_ALL_SWITCH(in, copy_strided_to<T>(out, x, sx, o, so, s));
}

void binary(int op, DType in, DType out, const void* a, const ND& sa, const void* b, const ND& sb,
            void* o, const ND& so, float p0, hipStream_t s) {
  if (out == in) {
    AGPU_ALL_SWITCH(in, launch_binary<T, T>(op, a, sa, b, sb, o, so, p0, s));
  } else if (out == DType::Bool) {
    AGPU_ALL_SWITCH(in, launch_binary<T, bool>(op, a, sa, b, sb, o, so, p0, s));
  } else {
    fail("binary op: unsupported output dtype %s for input %s", dtype_name(out), dtype_name(in));
  }
}

template <typename TI>
static void unary_to(int op, DType out, const void* x, const ND& sx, void* o, const ND& so, float p0,
                     float p1, hipStream_t s) {
  switch (out) {
    case DType::F32: launch_unary<TI, float>(op, x, sx, o, so, p0, p1, s); break;
    case DType::F16: launch_unary<TI, half_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::BF16: launch_unary<TI, bf16_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::I8: launch_unary<TI, int8_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::I16: launch_unary<TI, int16_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::I32: launch_unary<TI, int32_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::I64: launch_unary<TI, int64_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::U8: launch_unary<TI, uint8_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::U32: launch_unary<TI, uint32_t>(op, x, sx, o, so, p0, p1, s); break;
    case DType::Bool: launch_unary<TI, bool>(op, x, sx, o, so, p0, p1, s); break;
    default: fail("unary op: unsupported output dtype %s", dtype_name(out));
  }
}

void unary(int op, DType in, DType out, const void* x, const ND& sx, void* o, const ND& so, float p0,
           float p1, hipStream_t s) {
  int64_t n = numel_of(so);
  if (n == 0) return;
  if (op == kQuantize) {
    float lo = out == DType::I8 ? -128.f : 0.f, hi = out == DType::I8 ? 127.f : 255.f;
    if (out != DType::I8 && out != DType::U8) fail("quantize target must be int8 or uint8");
    AGPU_FLOAT_SWITCH(in, {
      if (out == DType::I8)
        hipLaunchKernelGGL((quantize_nd<uint64_t, T, int8_t>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const T*)x, sx, (int8_t*)o, so, (uint64_t)n, p0, p1, lo, hi);
      else
        hipLaunchKernelGGL((quantize_nd<uint64_t, T, uint8_t>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const T*)x, sx, (uint8_t*)o, so, (uint64_t)n, p0, p1, lo, hi);
    });
    check_launch("quantize");
    return;
  }
  if (op == kDequantize) {
    if (in != DType::I8 && in != DType::U8) fail("dequantize input must be int8 or uint8");
    AGPU_FLOAT_SWITCH(out, {
      if (in == DType::I8)
        hipLaunchKernelGGL((dequantize_nd<uint64_t, int8_t, T>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const int8_t*)x, sx, (T*)o, so, (uint64_t)n, p0, (int)p1);
      else
        hipLaunchKernelGGL((dequantize_nd<uint64_t, uint8_t, T>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const uint8_t*)x, sx, (T*)o, so, (uint64_t)n, p0, (int)p1);
    });
    check_launch("dequantize");
    return;
  }
  AGPU_ALL_SWITCH(in, unary_to<T>(op, out, x, sx, o, so, p0, p1, s));
}

void where(DType cdt, DType dt, const void* c, const ND& sc, const void* x, const ND& sx,
           const void* y, const ND& sy, void* o, const ND& so, hipStream_t s) {
  int64_t n = numel_of(so);
  if (n == 0) return;
  AGPU_ALL_SWITCH(dt, {
    typedef T TV;
    switch (cdt) {
      case DType::Bool:
      case DType::U8:
        hipLaunchKernelGGL((where_nd<uint64_t, uint8_t, TV>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const uint8_t*)c, sc, (const TV*)x, sx, (const TV*)y, sy, (TV*)o, so,
                           (uint64_t)n);
        break;
      case DType::I32:
        hipLaunchKernelGGL((where_nd<uint64_t, int32_t, TV>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const int32_t*)c, sc, (const TV*)x, sx, (const TV*)y, sy, (TV*)o, so,
                           (uint64_t)n);
        break;
      case DType::F32:
        hipLaunchKernelGGL((where_nd<uint64_t, float, TV>), dim3(grid_for(n)), dim3(256), 0, s,
                           (const float*)c, sc, (const TV*)x, sx, (const TV*)y, sy, (TV*)o, so,
                           (uint64_t)n);
        break;
      default: fail("where: condition dtype %s not supported", dtype_name(cdt));
    }
  });
  check_launch("where");
}

void tri(DType dt, bool upper, int64_t diag, const void* x, void* o, int64_t batch, int64_t rows,
         int64_t cols, hipStream_t s) {
  int64_t n = batch * rows * cols;
  if (n == 0) return;
  AGPU_ALL_SWITCH(dt, hipLaunchKernelGGL((tri_kernel<T>), dim3(grid_for(n)), dim3(256), 0, s,
                                         (const T*)x, (T*)o, n, rows, cols, diag, upper));
  check_launch("tri");
}

void axpy(DType dt, void* y, const ND& sy, const void* x, const ND& sx, float alpha, hipStream_t s) {
  int64_t n = numel_of(sy);
  if (n == 0) return;
  if (dt == DType::F32 && is_flat(sx, sy) && aligned16(x) && aligned16(y)) {
    hipLaunchKernelGGL(axpy_flat_f32, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, s, (float*)y,
                       (const float*)x, n, alpha);
  } else {
    AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((axpy_nd<uint64_t, T>), dim3(grid_for(n)), dim3(256), 0, s,
                                             (T*)y, (const T*)x, sx, sy, (uint64_t)n, alpha));
  }
  check_launch("axpy");
}

// The flat-path period of a leaf over the contiguous output `so`: n when it
// is laid out like the output, 1 for a single broadcast value, the element
// count of the output's trailing dims when it is contiguous over those and
// broadcast over the leading ones; 0 when none applies.
static int64_t chain_period(const ND& l, const ND& so, int64_t n) {
  if (is_flat(l, so)) return n;
  int d = so.ndim;
  int64_t expect = 1;
  while (d > 0 && (so.shape[d - 1] == 1 || l.stride[d - 1] == expect)) {
    expect *= so.shape[d - 1];
    --d;
  }
  for (int i = 0; i < d; ++i)
    if (l.stride[i] != 0 && so.shape[i] != 1) return 0;
  return expect;
}

void fused_chain(DType dt, const ChainProgram& prog, ChainLeaves L, void* out, const ND& so, hipStream_t s) {
  const int64_t n = numel_of(so);
  if (n == 0) return;
  if (prog.n_leaves < 1 || prog.n_leaves > kChainMaxLeaves || prog.n_steps < 1 || prog.n_steps > kChainMaxSteps ||
      prog.first < 0 || prog.first >= prog.n_leaves)
    fail("fused_chain: malformed program");
  for (int i = 0; i < prog.n_steps; ++i)
    if (prog.step[i].leaf >= prog.n_leaves) fail("fused_chain: step %d names leaf %d", i, prog.step[i].leaf);
  const size_t es = dt == DType::F32 ? 4 : 2;
  bool flat = aligned16(out) || (es == 2 && ((uintptr_t)out & 7) == 0);
  for (int j = 0; j < prog.n_leaves && flat; ++j) {
    const int64_t per = chain_period(L.nd[j], so, n);
    const bool vec_ok = ((uintptr_t)L.ptr[j] & (4 * es - 1)) == 0;
    if (per == 1) L.period[j] = 1;
    else if (per == n && vec_ok) L.period[j] = n;
    else if (per > 1 && per % 4 == 0 && n % per == 0 && vec_ok) L.period[j] = per;
    else flat = false;
  }
  if (flat) {
    const unsigned g = (unsigned)((n + 1023) / 1024);
    AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((chain_flat<T>), dim3(g), dim3(256), 0, s, prog, L, (T*)out, n));
  } else {
    bool small = n < (int64_t(1) << 31);
    for (int j = 0; j < prog.n_leaves && small; ++j) small = fits32(n, L.nd[j], L.nd[j]);
    if (small) {
      AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((chain_nd<uint32_t, T>), dim3(grid_for(n)), dim3(256), 0, s, prog, L,
                                               (T*)out, so, (uint32_t)n));
    } else {
      AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((chain_nd<uint64_t, T>), dim3(grid_for(n)), dim3(256), 0, s, prog, L,
                                               (T*)out, so, (uint64_t)n));
    }
  }
  check_launch("fused_chain");
}

void add_bias(DType dt, const void* in, const void* bias, void* out, int64_t numel, int64_t channels,
              int64_t channel_stride, hipStream_t s) {
  if (numel == 0) return;
  AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((add_bias_kernel<T>), dim3(grid_for(numel)), dim3(256), 0, s,
                                           (const T*)in, (const T*)bias, (T*)out, numel, channels,
                                           channel_stride));
  check_launch("add_bias");
}

}  // namespace k
}  // namespace agpu
