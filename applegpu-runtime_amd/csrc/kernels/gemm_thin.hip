// GEMMs with a unit extent, where MFMA tiles would be almost all padding:
//   N == 1: matrix-vector, C[b, m] = sum_k A[b, m, k] B[b, k]  (one wavefront
//           per output row, a shuffle reduction);
//   M == 1: vector-matrix with B rows contiguous along n, C[b, n] =
//           sum_k A[b, k] B[b, k, n]  (a 1024-thread block per 64 columns,
//           16 k slices reduced through LDS in slice order; optionally also
//           an SGD bias step from A's sum, GArgs::rowsum_acc);
//   K == 1: outer product, C[b, m, n] = A[b, m] B[b, n]  (elementwise).
// Same arithmetic as the reference's matmul/linear (fp32 accumulation,
// crates/core/src/kernel_templates.rs:987-1072) and the same fused epilogue
// as the tiled kernels (alpha, bias, activation, residual, mask).  In the
// C3 MLP step these are the forward and both backward products of the
// 4096 -> 1 output layer.
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

template <typename T>
__global__ void __launch_bounds__(256) gemv_n1(GArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  if (m >= p.M) return;  // a whole wavefront; the kernel has no barrier
  const T* A = (const T*)p.A + b * p.a_sb + m * p.a_sm;
  const T* B = (const T*)p.B + b * p.b_sb;
  float acc = 0.f;
#pragma unroll 8
  for (int64_t k = lane; k < p.K; k += 64) acc += to_f(A[k * p.a_sk]) * to_f(B[k * p.b_sk]);
  acc = wave_sum(acc);
  if (lane == 0) epilogue_store<T>(p, b, m, 0, acc);
}

template <typename T>
__global__ void __launch_bounds__(1024) gevm_m1(GArgs p) {
  __shared__ float sh[16][64];
  const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  const int64_t b = blockIdx.y;
  const T* A = (const T*)p.A + b * p.a_sb;
  const T* B = (const T*)p.B + b * p.b_sb;
  float s = 0.f;
  if (n < p.N) {
#pragma unroll 8
    for (int64_t k = slice; k < p.K; k += 16) s += to_f(A[k * p.a_sk]) * to_f(B[k * p.b_sk + n]);
  }
  sh[slice][lane] = s;
  __syncthreads();
  if (slice == 0 && n < p.N) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += sh[i][lane];
    epilogue_store<T>(p, b, 0, n, t);
  }
  // rowsum_acc[0] += alpha * sum_k A[k] (one batch): block 0 alone, its 16
  // wavefront sums added in order
  if (p.rowsum_acc && blockIdx.x == 0 && blockIdx.y == 0) {
    __syncthreads();  // slice 0 is done reading sh
    float r = 0.f;
    for (int64_t k = threadIdx.x; k < p.K; k += 1024) r += to_f(A[k * p.a_sk]);
    r = wave_sum(r);
    if (lane == 0) sh[0][slice] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) t += sh[0][i];
      p.rowsum_acc[0] += p.alpha * t;
    }
  }
}

// The backward of a Linear layer with one output (w [1, N]) and its SGD
// step, in one pass over the layer input h [R, N]: for each column j
//   g_in[r, j] = h[r, j] > 0 ? dz[r] * w[j] : 0   (with w before the update)
//   w[j]      += alpha * sum_r dz[r] * h[r, j]
// and b[0] += alpha * sum_r dz[r] (block 0).  It replaces outer_k1 (with
// the mask) followed by gevm_m1 (with the residual and rowsum_acc).  A block
// owns 16 columns over all rows (64 row slices of 16 lanes, so every CU
// gets a block at N = 4096); a column's 64 slice sums meet in LDS in slice
// order, so results repeat exactly.
template <typename T>
__global__ void __launch_bounds__(1024) linear1_bwd_sgd(Lin1Bwd p) {
  __shared__ float sh[64][17];
  const int c = threadIdx.x & 15, slice = threadIdx.x >> 4;
  const int64_t j = (int64_t)blockIdx.x * 16 + c;
  const T* h = (const T*)p.h;
  const T* dz = (const T*)p.dz;
  T* w = (T*)p.w;
  float s = 0.f;
  if (j < p.N) {
    const float wj = to_f(w[j]);
#pragma unroll 4
    for (int64_t r = slice; r < p.R; r += 64) {
      const float hv = to_f(h[r * p.h_sm + j]);
      const float d = to_f(dz[r * p.dz_s]);
      if (p.gin) ((T*)p.gin)[r * p.N + j] = from_f<T>(hv > 0.f ? d * wj : 0.f);
      s += d * hv;
    }
  }
  sh[slice][c] = s;
  __syncthreads();
  if (slice == 0 && j < p.N) {
    float t = 0.f;
#pragma unroll 8
    for (int i = 0; i < 64; ++i) t += sh[i][c];
    w[j] = from_f<T>(p.alpha * t + to_f(w[j]));
  }
  if (p.b && blockIdx.x == 0) {
    __syncthreads();  // slice 0 is done reading sh
    float r = 0.f, q = 0.f;
    for (int64_t k = threadIdx.x; k < p.R; k += 1024) {
      r += to_f(dz[k * p.dz_s]);
      if (p.loss) {
        const float d = to_f(((const T*)p.z)[k]) - to_f(((const T*)p.y)[k]);
        q += d * d;
      }
    }
    r = wave_sum(r);
    q = wave_sum(q);
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sh[0][wv] = r; sh[1][wv] = q; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f, u = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { t += sh[0][i]; u += sh[1][i]; }
      T* b = (T*)p.b;
      b[0] = from_f<T>(to_f(b[0]) + p.alpha * t);
      if (p.loss) ((T*)p.loss)[0] = from_f<T>(u * p.inv_n);
    }
  }
}

// z[r] = h[r, :] . w + b[0] and the MSE gradient dz[r] = (z[r] - y[r]) *
// 2/n, one 256-thread block per row (16-byte loads when the rows allow);
// the wavefront sums meet in LDS in order.
template <typename T>
__global__ void __launch_bounds__(256) linear1_fwd_mse(Lin1Fwd p) {
  __shared__ float sh[4];
  const int64_t r = blockIdx.x;
  const T* h = (const T*)p.h + r * p.h_sm;
  const T* w = (const T*)p.w;
  float s = 0.f;
  const bool vec = sizeof(T) == 4 && (p.N & 3) == 0 && (((uintptr_t)h | (uintptr_t)w) & 15) == 0;
  if (vec) {
    for (int64_t k = threadIdx.x; k < p.N / 4; k += 256) {
      const float4 a = ((const float4*)h)[k], c = ((const float4*)w)[k];
      s += a.x * c.x;
      s += a.y * c.y;
      s += a.z * c.z;
      s += a.w * c.w;
    }
  } else {
    for (int64_t k = threadIdx.x; k < p.N; k += 256) s += to_f(h[k]) * to_f(w[k]);
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float z = ((sh[0] + sh[1]) + (sh[2] + sh[3])) + to_f(((const T*)p.b)[0]);
    const T zt = from_f<T>(z);
    ((T*)p.z)[r] = zt;
    const float d = to_f(zt) - to_f(((const T*)p.y)[r]);
    ((T*)p.dz)[r] = from_f<T>(d * p.two_over_n);
  }
}

// linear1_fwd_mse with the input row formed from split-K partials (the
// previous layer's GEMM left them unreduced): one 1024-thread block per row;
// each thread sums the splits of its 4-column groups in split order, adds
// the bias, applies the ReLU (the split-K reduction's arithmetic, so h is
// the same bits), stores h and accumulates its dot with w.
__global__ void __launch_bounds__(1024) linear1_fwd_mse_parts(Lin1FwdParts p) {
  __shared__ float sh[16];
  const int64_t r = blockIdx.x;
  const float* pr = p.part + r * p.N;
  float s = 0.f;
  for (int64_t k = threadIdx.x; k < p.N / 4; k += 1024) {
    float4 parts[8];
#pragma unroll
    for (int sp = 0; sp < 8; ++sp)
      if (sp < p.splits) parts[sp] = ((const float4*)(pr + sp * p.plane))[k];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int sp = 0; sp < 8; ++sp)
      if (sp < p.splits) {
        acc.x += parts[sp].x; acc.y += parts[sp].y; acc.z += parts[sp].z; acc.w += parts[sp].w;
      }
    const float4 bb = ((const float4*)p.hb)[k];
    float4 h;
    h.x = fmaxf(acc.x + bb.x, 0.f); h.y = fmaxf(acc.y + bb.y, 0.f);
    h.z = fmaxf(acc.z + bb.z, 0.f); h.w = fmaxf(acc.w + bb.w, 0.f);
    ((float4*)(p.h_out + r * p.N))[k] = h;
    const float4 c = ((const float4*)p.w)[k];
    s += h.x * c.x;
    s += h.y * c.y;
    s += h.z * c.z;
    s += h.w * c.w;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += sh[i];
    const float z = t + p.b[0];
    p.z[r] = z;
    p.dz[r] = (z - p.y[r]) * p.two_over_n;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) outer_k1(GArgs p) {
  const int64_t b = blockIdx.y;
  const int64_t total = p.M * p.N;
  const T* A = (const T*)p.A + b * p.a_sb;
  const T* B = (const T*)p.B + b * p.b_sb;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / p.N, n = i % p.N;
    epilogue_store<T>(p, b, m, n, to_f(A[m * p.a_sm]) * to_f(B[n * p.b_sn]));
  }
}

}  // namespace

void linear1_backward_sgd(DType dt, const Lin1Bwd& a, hipStream_t s) {
  if (a.N == 0) return;
  if (dt != DType::F32) fail("linear1_backward_sgd: fp32 only");
  hipLaunchKernelGGL((linear1_bwd_sgd<float>), dim3((unsigned)((a.N + 15) / 16)), dim3(1024), 0, s, a);
  check_launch("linear1_backward_sgd");
}

void linear1_forward_mse_parts(const Lin1FwdParts& a, hipStream_t s) {
  if (a.R == 0) return;
  if (a.R > 0x7fffffffLL || a.splits < 1 || a.splits > 8 || a.N % 4 != 0 ||
      (((uintptr_t)a.part | (uintptr_t)a.hb | (uintptr_t)a.h_out | (uintptr_t)a.w) & 15) || a.plane % 4 != 0)
    fail("linear1_forward_mse_parts: 1-8 splits, N %% 4 == 0 and 16-byte aligned operands needed");
  hipLaunchKernelGGL(linear1_fwd_mse_parts, dim3((unsigned)a.R), dim3(1024), 0, s, a);
  check_launch("linear1_forward_mse_parts");
}

void linear1_forward_mse(DType dt, const Lin1Fwd& a, hipStream_t s) {
  if (a.R == 0) return;
  if (dt != DType::F32) fail("linear1_forward_mse: fp32 only");
  if (a.R > 0x7fffffffLL) fail("linear1_forward_mse: too many rows");
  hipLaunchKernelGGL((linear1_fwd_mse<float>), dim3((unsigned)a.R), dim3(256), 0, s, a);
  check_launch("linear1_forward_mse");
}

int thin_kind(const Gemm& g) {
  const bool fl = g.dt == DType::F32 || g.dt == DType::F16 || g.dt == DType::BF16;
  if (!fl || g.b_dt != g.dt || g.b_scale || g.ln_gamma || g.b_packed || g.b_x3 || g.batch > 65535) return kThinNone;
  if (g.K == 1) return kThinK1;
  if (g.N == 1) return kThinN1;
  if (g.M == 1 && g.dt == DType::F32 && g.b_sn == 1) return kThinM1;
  return kThinNone;
}

void gemm_thin(int kind, DType dt, const GArgs& p, hipStream_t s) {
  const unsigned nb = (unsigned)p.batch;
  switch (kind) {
    case kThinN1: {
      dim3 grid((unsigned)((p.M + 3) / 4), nb);
      AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((gemv_n1<T>), grid, dim3(256), 0, s, p));
      break;
    }
    case kThinM1: {
      dim3 grid((unsigned)((p.N + 63) / 64), nb);
      AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((gevm_m1<T>), grid, dim3(1024), 0, s, p));
      break;
    }
    case kThinK1: {
      int64_t blocks = (p.M * p.N + 255) / 256;
      if (blocks > 4096) blocks = 4096;
      dim3 grid((unsigned)blocks, nb);
      AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((outer_k1<T>), grid, dim3(256), 0, s, p));
      break;
    }
    default: fail("gemm_thin: not a thin shape");
  }
  check_launch("gemm_thin");
}

}  // namespace k
}  // namespace agpu
