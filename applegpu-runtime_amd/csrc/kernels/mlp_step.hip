// One SGD step of a small two-layer MLP in a single workgroup.
//
// Linear(N0 -> N1) -> ReLU -> Linear(N1 -> N2), MSE loss over all R x N2
// outputs, SGD w += alpha * grad (alpha = -lr) for both layers: the step the
// reference trains through autograd and torch.optim.SGD
// (python/tests/bench_comparison.py:11-38; aten sequence of
// backend_cpp/applegpu_backend.cpp:533-566, 584-620, 678-686, 801-895).  At
// the sizes of config C1 (batch 32, 64 -> 128 -> 10) the whole step is
// 0.65 M multiply-adds over 38 KB of parameters: as separate GEMM, loss and
// reduction launches it is bound by launch latency (eight launches), while
// one 1024-thread workgroup holds every activation in LDS and finishes it in
// one launch.
//
//   h  = relu(x W1^T + b1)                       [R, N1]
//   z  = h W2^T + b2,  dz = 2 (z - y) / (R N2)   [R, N2]
//   dh = (dz W2) * (h > 0)                       [R, N1]  (W2 before its step)
//   W2 += alpha dz^T h,  b2 += alpha sum_r dz
//   W1 += alpha dh^T x,  b1 += alpha sum_r dh
//   loss = sum (z - y)^2 / (R N2)
//
// Every sum runs in a fixed order in fp32 (fmaf), so repeated steps give
// identical bits.  Threads that share an operand read it from LDS as a
// float4 broadcast and own four outputs each; the output layer's dot products
// (length N1) are split over eight lanes and reduced by fixed xor steps.
#include "device.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kMlpThreads = 1024, kMlpWaves = kMlpThreads / 64;

// n floats rounded up to a whole number of float4
__host__ __device__ constexpr int64_t al4(int64_t n) { return (n + 3) & ~(int64_t)3; }

__global__ void __launch_bounds__(kMlpThreads) mlp2_step_kernel(Mlp2Step p) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int R = p.R, N0 = p.N0, N1 = p.N1, N2 = p.N2, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // h and W2 rows have an odd pitch (N1 + 1): the output layer's lanes read
  // them eight rows at a time (with pitch N1, a multiple of 32, all eight
  // rows fall on one bank)
  // (every region starts on 16 bytes: x and dh are read as float4)
  const int P1 = N1 + 1;
  float* xs = sm;                      // [R][N0]
  float* hs = xs + R * N0;             // [R][P1]
  float* dhs = hs + al4(R * P1);       // [R][N1]
  float* w2s = dhs + R * N1;           // [N2][P1]
  float* dzs = w2s + al4(N2 * P1);     // [R][N2]
  float* ys = dzs + al4(R * N2);       // [R][N2]
  float* b1s = ys + al4(R * N2);       // [N1]
  float* b2s = b1s + N1;               // [N2]
  float* red = b2s + al4(N2);          // [kMlpWaves]

  // 1. x, W2, y and the biases into LDS (N0 % 4 == 0, N1 % 4 == 0): no
  //    phase below then waits on a global load inside its loops
  for (int i = tid; i < R * N0 / 4; i += kMlpThreads) ((float4*)xs)[i] = ((const float4*)p.x)[i];
  for (int i = tid; i < N2 * N1 / 4; i += kMlpThreads) {
    const float4 v = ((const float4*)p.w2)[i];
    float* d = w2s + (4 * i / N1) * P1 + 4 * i % N1;
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
  }
  for (int i = tid; i < R * N2; i += kMlpThreads) ys[i] = p.y[i];
  for (int i = tid; i < N1; i += kMlpThreads) b1s[i] = p.b1[i];
  for (int i = tid; i < N2; i += kMlpThreads) b2s[i] = p.b2[i];
  __syncthreads();

  // 2. h = relu(x W1^T + b1): thread (g, j) owns rows 4g .. 4g+3 of column j
  //    and reads W1's row j from global memory in chunks of 64 columns, the
  //    16 loads of a chunk issued before the first is used.  Columns past N0
  //    re-read the row's last four and are not added.
  const int RG = (R + 3) / 4;
  for (int o = tid; o < RG * N1; o += kMlpThreads) {
    const int g = o / N1, j = o % N1;
    const float* wr = p.w1 + (int64_t)j * N0;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < N0; k0 += 64) {
      float4 wv[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) wv[q] = *(const float4*)(wr + (k0 + 4 * q < N0 ? k0 + 4 * q : N0 - 4));
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        if (k0 + 4 * q >= N0) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * g + i < R ? 4 * g + i : R - 1;
          const float4 xv = *(const float4*)(xs + r * N0 + k0 + 4 * q);
          acc[i] = fmaf(xv.x, wv[q].x, acc[i]);
          acc[i] = fmaf(xv.y, wv[q].y, acc[i]);
          acc[i] = fmaf(xv.z, wv[q].z, acc[i]);
          acc[i] = fmaf(xv.w, wv[q].w, acc[i]);
        }
      }
    }
    const float bj = b1s[j];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * g + i < R) hs[(4 * g + i) * P1 + j] = fmaxf(acc[i] + bj, 0.f);
  }
  __syncthreads();

  // 3. z = h W2^T + b2 and the MSE gradient: eight lanes per (row, output)
  //    pair, lane e of the eight taking columns e, e + 8, ... of the N1
  //    products, then three xor steps over the eight; the lane with e = 0
  //    writes dz and adds its squared error.
  const float inv_n = 1.f / (float)(R * N2);
  float se = 0.f;
  const int e8 = tid & 7;
  for (int o0 = tid >> 3; o0 < ((R * N2 + 127) / 128) * 128; o0 += kMlpThreads / 8) {
    const int o = o0 < R * N2 ? o0 : R * N2 - 1;  // (every lane of the loop reaches the xor steps)
    const int r = o / N2, c = o % N2;
    const float* hr = hs + r * P1;
    const float* wr = w2s + c * P1;
    float part = 0.f;
#pragma unroll 4
    for (int j = e8; j < N1; j += 8) part = fmaf(hr[j], wr[j], part);
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    part += __shfl_xor(part, 4, 64);
    if (e8 == 0 && o0 < R * N2) {
      const float d = (part + b2s[c]) - ys[o];
      dzs[o] = 2.f * d * inv_n;
      se = fmaf(d, d, se);
    }
  }
  se += __shfl_xor(se, 8, 64);
  se += __shfl_xor(se, 16, 64);
  se += __shfl_xor(se, 32, 64);
  if (lane == 0) red[wave] = se;
  __syncthreads();

  // 4. dh = (dz W2) * (h > 0) with W2 before its step; W2's and b2's steps
  //    (dz^T h: thread (c, j) over the rows); the loss
  for (int o = tid; o < R * N1; o += kMlpThreads) {
    const int r = o / N1, j = o % N1;
    float acc = 0.f;
    for (int c = 0; c < N2; ++c) acc = fmaf(dzs[r * N2 + c], w2s[c * P1 + j], acc);
    dhs[o] = hs[r * P1 + j] > 0.f ? acc : 0.f;
  }
  for (int o = tid; o < N2 * N1; o += kMlpThreads) {
    const int c = o / N1, j = o % N1;
    float acc = 0.f;
#pragma unroll 8
    for (int r = 0; r < R; ++r) acc = fmaf(dzs[r * N2 + c], hs[r * P1 + j], acc);
    p.w2[o] = fmaf(p.alpha, acc, w2s[c * P1 + j]);
  }
  for (int c = tid; c < N2; c += kMlpThreads) {
    float acc = 0.f;
#pragma unroll 8
    for (int r = 0; r < R; ++r) acc += dzs[r * N2 + c];
    p.b2[c] = fmaf(p.alpha, acc, b2s[c]);
  }
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < kMlpWaves; ++w) t += red[w];
    p.loss[0] = t * inv_n;
  }
  __syncthreads();

  // 5. W1's and b1's steps: thread (g, k) owns rows 4g .. 4g+3 of W1's
  //    column k (dh^T x over the batch rows; dh read as a float4 broadcast)
  const int JG = N1 / 4;
  for (int o = tid; o < JG * N0; o += kMlpThreads) {
    const int g = o / N0, k = o % N0;
    // the four weights first: their loads overlap the sums below
    float* w = p.w1 + (int64_t)(4 * g) * N0 + k;
    const float w0 = w[0], w1 = w[N0], w2 = w[2 * N0], w3 = w[3 * N0];
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int r = 0; r < R; ++r) {
      const float xv = xs[r * N0 + k];
      const float4 dv = *(const float4*)(dhs + r * N1 + 4 * g);
      acc[0] = fmaf(dv.x, xv, acc[0]);
      acc[1] = fmaf(dv.y, xv, acc[1]);
      acc[2] = fmaf(dv.z, xv, acc[2]);
      acc[3] = fmaf(dv.w, xv, acc[3]);
    }
    w[0] = fmaf(p.alpha, acc[0], w0);
    w[N0] = fmaf(p.alpha, acc[1], w1);
    w[2 * N0] = fmaf(p.alpha, acc[2], w2);
    w[3 * N0] = fmaf(p.alpha, acc[3], w3);
  }
  for (int j = tid; j < N1; j += kMlpThreads) {
    float acc = 0.f;
#pragma unroll 8
    for (int r = 0; r < R; ++r) acc += dhs[r * N1 + j];
    p.b1[j] = fmaf(p.alpha, acc, b1s[j]);
  }
}

size_t mlp2_lds_bytes(int64_t R, int64_t N0, int64_t N1, int64_t N2) {
  return (size_t)(R * N0 + al4(R * (N1 + 1)) + R * N1 + al4(N2 * (N1 + 1)) + 2 * al4(R * N2) + N1 + al4(N2) +
                  kMlpWaves) * sizeof(float);
}

}  // namespace

bool mlp2_step_ok(int64_t R, int64_t N0, int64_t N1, int64_t N2) {
  return R >= 1 && N0 >= 4 && N1 >= 4 && N2 >= 1 && N0 % 4 == 0 && N1 % 4 == 0 && R <= 256 && N0 <= 1024 &&
         N1 <= 1024 && N2 <= 64 && mlp2_lds_bytes(R, N0, N1, N2) <= 64 * 1024;
}

void mlp2_step(const Mlp2Step& a, hipStream_t s) {
  if (!mlp2_step_ok(a.R, a.N0, a.N1, a.N2)) fail("mlp2_step: shape outside the one-workgroup step");
  if ((((uintptr_t)a.x | (uintptr_t)a.w1 | (uintptr_t)a.w2) & 15) != 0)
    fail("mlp2_step: x, W1 and W2 must be 16-byte aligned");
  hipLaunchKernelGGL(mlp2_step_kernel, dim3(1), dim3(kMlpThreads), mlp2_lds_bytes(a.R, a.N0, a.N1, a.N2), s, a);
  check_launch("mlp2_step");
}

}  // namespace k
}  // namespace agpu
