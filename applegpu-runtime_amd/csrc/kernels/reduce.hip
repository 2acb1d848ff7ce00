// Reductions (sum over one dim, whole-tensor sum / squared-error sum, MSE
// backward) and index kernels (embedding, index_select, gather).
//
// Reference semantics:
//   sum_dim output shape, keepdim                 crates/core/src/eager.rs:827-855
//   mean_all -> one element                       crates/core/src/eager.rs:710-769
//   mse_loss = mean((a-b)^2), grad = (a-b)*2/n*g  backend_cpp/applegpu_backend.cpp:801-867
//   embedding out[i,:] = W[idx[i],:]              crates/core/src/kernel_templates.rs:1119-1143
//   gather / index_select                         crates/core/src/kernel_templates.rs:870-975
// The reference's mean_all chains thread-per-row mean kernels; here a
// two-stage tree reduction with a fixed order (deterministic, no atomics).
#include "device.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

// [outer, red, inner] -> [outer, inner]; inner == 1 uses a wavefront per row.
template <typename T>
__global__ void __launch_bounds__(256) sum_last(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                int64_t red, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * red;
  float s = 0.f;
  for (int64_t c = lane; c < red; c += 64) s += to_f(xr[c]);
  s = wave_sum(s);
  if (lane == 0) y[row] = from_f<T>(s * scale);
}

// Column sums: a 1024-thread block covers 64 columns x 16 row slices (each
// thread's loads are independent, so they are all in flight), then the 16
// partial sums meet in LDS and are added in slice order.  acc != 0 adds the
// scaled sum to y instead of storing it (y += scale * sum: the bias update
// of an SGD step fused with its gradient).
template <typename T>
__global__ void __launch_bounds__(1024) sum_cols(const T* __restrict__ x, T* __restrict__ y, int64_t outer,
                                                 int64_t red, int64_t inner, float scale, int acc) {
  __shared__ float sh[16][64];
  const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t o = blockIdx.y;
  float s = 0.f;
  if (col < inner) {
    const T* base = x + o * red * inner + col;
#pragma unroll 8
    for (int64_t r = slice; r < red; r += 16) s += to_f(base[r * inner]);
  }
  sh[slice][lane] = s;
  __syncthreads();
  if (slice == 0 && col < inner) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += sh[i][lane];
    float v = t * scale;
    if (acc) v += to_f(y[o * inner + col]);
    y[o * inner + col] = from_f<T>(v);
  }
}

template <typename T>
__global__ void __launch_bounds__(256) sum_int_dim(const T* __restrict__ x, T* __restrict__ y, int64_t outer,
                                                   int64_t red, int64_t inner) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= outer * inner) return;
  int64_t o = i / inner, c = i % inner;
  long long s = 0;
  for (int64_t r = 0; r < red; ++r) s += (long long)x[(o * red + r) * inner + c];
  y[i] = (T)s;
}

constexpr int kPartials = 512;

// Stage 1: each block writes one fp32 partial.
template <typename T>
__global__ void __launch_bounds__(256) reduce_stage1(int kind, const T* __restrict__ a, const T* __restrict__ b,
                                                     int64_t n, float* __restrict__ part) {
  __shared__ float sh[4];
  float s = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float v = to_f(a[i]);
    if (kind == 1) {
      v -= to_f(b[i]);
      v *= v;
    }
    s += v;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = sh[0] + sh[1] + sh[2] + sh[3];
}

template <typename T>
__global__ void __launch_bounds__(256) reduce_stage2(const float* __restrict__ part, int nparts, float scale,
                                                     T* __restrict__ out) {
  __shared__ float sh[4];
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 256) s += part[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = from_f<T>((sh[0] + sh[1] + sh[2] + sh[3]) * scale);
}

template <typename T>
__global__ void __launch_bounds__(256) mse_bwd_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                      const T* __restrict__ g, T* __restrict__ dx, int64_t n,
                                                      float two_over_n) {
  const float gs = to_f(g[0]);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    dx[i] = from_f<T>((to_f(a[i]) - to_f(b[i])) * two_over_n * gs);
}

// MSE loss and its gradient (upstream gradient 1) in one single-block
// launch, for the small outputs of a training step: loss = sum((a-b)^2) / n
// (the 1024 per-thread partial sums are reduced in a fixed order) and
// grad = (a - b) * 2/n, the expressions of reduce_stage1/2 and
// mse_bwd_kernel.
constexpr int kMseFusedMax = 1 << 16;
template <typename T>
__global__ void __launch_bounds__(1024) mse_fused_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                         T* __restrict__ loss, T* __restrict__ grad, int64_t n,
                                                         float inv_n, float two_over_n) {
  __shared__ float sh[16];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) {
    const float d = to_f(a[i]) - to_f(b[i]);
    s += d * d;
    grad[i] = from_f<T>(d * two_over_n * 1.f);
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += sh[i];
    loss[0] = from_f<T>(t * inv_n);
  }
}

// Rows with an index outside [0, vocab) come out as zeros.
template <typename T, typename I>
__global__ void __launch_bounds__(256) embedding_kernel(const T* __restrict__ w, int64_t vocab, int64_t dim,
                                                        const I* __restrict__ idx, int64_t n,
                                                        T* __restrict__ out) {
  const int64_t row = blockIdx.y;
  for (int64_t r = row; r < n; r += gridDim.y) {
    const int64_t id = (int64_t)idx[r];
    const bool ok = id >= 0 && id < vocab;
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < dim; c += (int64_t)gridDim.x * 256)
      out[r * dim + c] = ok ? w[id * dim + c] : T(0);
  }
}

// ── embedding backward ────────────────────────────────────────────────────
// dw[w, :] = sum of dy[i, :] over the tokens i with idx[i] == w, added in
// token order; rows no token names are zero (filled first).  One 256-thread
// block per token: the first token naming w collects every token naming w,
// in ascending order, into an LDS list (wavefront ballots keep the order)
// and writes the row, so each row has one writer and one summation order.
// The reference scatters with float atomics (kernel_templates.rs:1867-1913),
// whose order varies from run to run.  Tokens whose index is outside
// [0, nw) add nothing.
constexpr int kEbList = 1024;  // tokens gathered per round
constexpr int kEbCols = 4;     // columns per thread: a pass covers 1024 columns

template <typename T>
__global__ void __launch_bounds__(256) fill_zero_kernel(T* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = T(0);
}

template <typename T, typename I>
__global__ void __launch_bounds__(256) embedding_bwd_kernel(const T* __restrict__ dy, const I* __restrict__ idx,
                                                            T* __restrict__ dw, int64_t n, int64_t dim,
                                                            int64_t nw) {
  __shared__ int64_t list[kEbList];
  __shared__ int wave_cnt[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t i = blockIdx.x;
  const int64_t w = (int64_t)idx[i];
  if (w < 0 || w >= nw) return;  // uniform over the block
  int dup = 0;
#pragma unroll 8
  for (int64_t j = tid; j < i; j += 256) dup |= (int64_t)idx[j] == w;
  if (__syncthreads_or(dup)) return;  // an earlier token's block writes row w

  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int64_t c0 = 0; c0 < dim; c0 += 256 * kEbCols) {
    float acc[kEbCols];
#pragma unroll
    for (int k = 0; k < kEbCols; ++k) acc[k] = 0.f;
    int64_t t0 = i;
    while (t0 < n) {
      // gather the next round of matching tokens (ascending) into the list
      int cnt = 0;
      while (t0 < n && cnt <= kEbList - 256) {
        const int64_t j = t0 + tid;
        const bool m = j < n && (int64_t)idx[j] == w;
        const uint64_t mask = __ballot(m);
        if (lane == 0) wave_cnt[wv] = __popcll(mask);
        __syncthreads();
        int off = cnt;
        for (int x = 0; x < wv; ++x) off += wave_cnt[x];
        if (m) list[off + __popcll(mask & below)] = j;
        cnt += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
        __syncthreads();
        t0 += 256;
      }
      for (int e = 0; e < cnt; ++e) {
        const T* row = dy + list[e] * dim;
#pragma unroll
        for (int k = 0; k < kEbCols; ++k) {
          const int64_t c = c0 + k * 256 + tid;
          if (c < dim) acc[k] += to_f(row[c]);
        }
      }
      __syncthreads();  // the list is refilled next round
    }
#pragma unroll
    for (int k = 0; k < kEbCols; ++k) {
      const int64_t c = c0 + k * 256 + tid;
      if (c < dim) dw[w * dim + c] = from_f<T>(acc[k]);
    }
  }
}

template <typename T, typename I>
__global__ void __launch_bounds__(256) index_select_kernel(const T* __restrict__ x, int64_t outer, int64_t size,
                                                           int64_t inner, const I* __restrict__ idx, int64_t m,
                                                           T* __restrict__ out) {
  const int64_t n = outer * m * inner;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t c = i % inner, j = (i / inner) % m, o = i / (inner * m);
    int64_t id = (int64_t)idx[j];
    out[i] = (id >= 0 && id < size) ? x[(o * size + id) * inner + c] : T(0);
  }
}

template <typename T, typename I>
__global__ void __launch_bounds__(256) gather_kernel(const T* __restrict__ x, int64_t outer, int64_t size,
                                                     int64_t inner, const I* __restrict__ idx, int64_t m,
                                                     T* __restrict__ out) {
  const int64_t n = outer * m * inner;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t c = i % inner, o = i / (inner * m);
    int64_t id = (int64_t)idx[i];
    out[i] = (id >= 0 && id < size) ? x[(o * size + id) * inner + c] : T(0);
  }
}

unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

void sum_dim(DType dt, const void* x, void* y, int64_t outer, int64_t red, int64_t inner, float scale,
             hipStream_t s) {
  if (outer * inner == 0) return;
  if (!dtype_is_float(dt)) {
    AGPU_ALL_SWITCH(dt, hipLaunchKernelGGL((sum_int_dim<T>), dim3(grid_for(outer * inner)), dim3(256), 0, s,
                                           (const T*)x, (T*)y, outer, red, inner));
  } else if (inner == 1) {
    AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((sum_last<T>), dim3((unsigned)((outer + 3) / 4)), dim3(256), 0, s,
                                             (const T*)x, (T*)y, outer, red, scale));
  } else {
    if (outer > 65535) fail("sum_dim: outer extent %lld too large", (long long)outer);
    dim3 grid((unsigned)((inner + 63) / 64), (unsigned)outer);
    AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((sum_cols<T>), grid, dim3(1024), 0, s, (const T*)x, (T*)y, outer,
                                             red, inner, scale, 0));
  }
  check_launch("sum_dim");
}

size_t reduce_all_ws_bytes() { return kPartials * sizeof(float); }

void reduce_all(int kind, DType dt, const void* a, const void* b, int64_t n, float scale, void* out, void* ws,
                hipStream_t s) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > kPartials) blocks = kPartials;
  if (blocks < 1) blocks = 1;
  AGPU_FLOAT_SWITCH(dt, {
    hipLaunchKernelGGL((reduce_stage1<T>), dim3((unsigned)blocks), dim3(256), 0, s, kind, (const T*)a,
                       (const T*)b, n, (float*)ws);
    hipLaunchKernelGGL((reduce_stage2<T>), dim3(1), dim3(256), 0, s, (const float*)ws, (int)blocks, scale,
                       (T*)out);
  });
  check_launch("reduce_all");
}

void mse_backward(DType dt, const void* a, const void* b, const void* g, void* dx, int64_t n, hipStream_t s) {
  if (n == 0) return;
  float two_over_n = 2.f / (float)n;
  AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((mse_bwd_kernel<T>), dim3(grid_for(n)), dim3(256), 0, s, (const T*)a,
                                           (const T*)b, (const T*)g, (T*)dx, n, two_over_n));
  check_launch("mse_backward");
}

void sum_rows_axpy(DType dt, const void* x, void* y, int64_t rows, int64_t cols, float alpha, hipStream_t s) {
  if (cols == 0) return;
  dim3 grid((unsigned)((cols + 63) / 64), 1);
  AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((sum_cols<T>), grid, dim3(1024), 0, s, (const T*)x, (T*)y, (int64_t)1,
                                           rows, cols, alpha, 1));
  check_launch("sum_rows_axpy");
}

bool mse_fused_ok(int64_t n) { return n > 0 && n <= kMseFusedMax; }

void mse_loss_grad(DType dt, const void* a, const void* b, void* loss, void* grad, int64_t n, hipStream_t s) {
  if (!mse_fused_ok(n)) fail("mse_loss_grad: %lld elements (one block handles at most %d)", (long long)n,
                             kMseFusedMax);
  AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((mse_fused_kernel<T>), dim3(1), dim3(1024), 0, s, (const T*)a,
                                           (const T*)b, (T*)loss, (T*)grad, n, 1.f / (float)n, 2.f / (float)n));
  check_launch("mse_loss_grad");
}

void embedding(DType dt, const void* w, int64_t vocab, int64_t dim, DType idx_dt, const void* idx, int64_t n,
               void* out, hipStream_t s) {
  if (n == 0 || dim == 0) return;
  dim3 grid((unsigned)((dim + 255) / 256), (unsigned)(n < 65535 ? n : 65535));
  AGPU_ALL_SWITCH(dt, {
    typedef T TV;
    AGPU_INT_SWITCH(idx_dt, hipLaunchKernelGGL((embedding_kernel<TV, I>), grid, dim3(256), 0, s, (const TV*)w,
                                               vocab, dim, (const I*)idx, n, (TV*)out));
  });
  check_launch("embedding");
}

void embedding_backward(DType dt, const void* dy, DType idx_dt, const void* idx, int64_t n, int64_t dim,
                        int64_t nw, void* dw, hipStream_t s) {
  if (nw == 0 || dim == 0) return;
  if (n > 0x7fffffffLL) fail("embedding_backward: %lld tokens exceed the grid", (long long)n);
  AGPU_FLOAT_SWITCH(dt, {
    typedef T TV;
    const int64_t total = nw * dim;
    const int64_t fb = (total + 255) / 256;
    hipLaunchKernelGGL((fill_zero_kernel<TV>), dim3((unsigned)(fb < 8192 ? fb : 8192)), dim3(256), 0, s, (TV*)dw,
                       total);
    if (n > 0)
      AGPU_INT_SWITCH(idx_dt, hipLaunchKernelGGL((embedding_bwd_kernel<TV, I>), dim3((unsigned)n), dim3(256), 0, s,
                                                 (const TV*)dy, (const I*)idx, (TV*)dw, n, dim, nw));
  });
  check_launch("embedding_backward");
}

void index_select(DType dt, const void* x, int64_t outer, int64_t size, int64_t inner, DType idx_dt,
                  const void* idx, int64_t m, void* out, hipStream_t s) {
  int64_t n = outer * m * inner;
  if (n == 0) return;
  AGPU_ALL_SWITCH(dt, {
    typedef T TV;
    AGPU_INT_SWITCH(idx_dt, hipLaunchKernelGGL((index_select_kernel<TV, I>), dim3(grid_for(n)), dim3(256), 0, s,
                                               (const TV*)x, outer, size, inner, (const I*)idx, m, (TV*)out));
  });
  check_launch("index_select");
}

void gather(DType dt, const void* x, int64_t outer, int64_t size, int64_t inner, DType idx_dt, const void* idx,
            int64_t m, void* out, hipStream_t s) {
  int64_t n = outer * m * inner;
  if (n == 0) return;
  AGPU_ALL_SWITCH(dt, {
    typedef T TV;
    AGPU_INT_SWITCH(idx_dt, hipLaunchKernelGGL((gather_kernel<TV, I>), dim3(grid_for(n)), dim3(256), 0, s,
                                               (const TV*)x, outer, size, inner, (const I*)idx, m, (TV*)out));
  });
  check_launch("gather");
}

}  // namespace k
}  // namespace agpu
