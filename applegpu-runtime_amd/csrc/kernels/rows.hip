// Row kernels over the last dimension: softmax, log_softmax, softmax_causal,
// layer_norm, row reductions (sum/mean/amax/argmax/var), softmax backward and
// the symmetric per-row int8 quantize / dequantize pair.
//
// Reference semantics (crates/core/src/kernel_templates.rs):
//   softmax: m = max, e = exp(x-m), out = e / sum(e)           :398-430
//   log_softmax: x - m - log(sum(exp(x-m)))                    :434-465
//   softmax_causal: columns j <= row only, zeros above          :468-497
//   argmax: strict > so the first maximum wins, int32 output    :500-520
//   layer_norm: two-pass mean, population variance,
//               y = gamma*(x-mean)*inv_std + beta              :1075-1116
// The reference runs one thread per row; here one 64-lane wavefront owns a
// row (rows up to 2048 columns stay in registers: a single HBM read and a
// single write), and a 256-thread workgroup owns longer rows.
#include "device.hpp"
#include "gemm_kernels.hpp"  // x3_store4: packed x3 rows of the layer_norm output

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kRowsPerBlock = 4;  // one wavefront per row

// Loads 4 consecutive elements at column c (c % 4 == 0) as float, with a
// per-element guard against `limit`; masked lanes get `fill`.  FULL: the
// row is an exact multiple of the wavefront's vectors and 16-byte aligned,
// so every lane loads unconditionally (no per-lane branch around the load,
// which would make each load wait as it issues).
template <typename T, bool FULL = false>
__device__ __forceinline__ void load4(const T* __restrict__ row, int64_t c, int64_t limit, bool vec,
                                      float fill, float out[4]) {
  if (FULL || (vec && c + 4 <= limit)) {
    if constexpr (sizeof(T) == 4) {
      float4 v = *(const float4*)(row + c);
      out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
      T tmp[4];
      *(float2*)tmp = *(const float2*)(row + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) out[j] = to_f(tmp[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = (c + j < limit) ? to_f(row[c + j]) : fill;
  }
}

template <typename T, bool FULL = false>
__device__ __forceinline__ void store4(T* __restrict__ row, int64_t c, int64_t limit, bool vec,
                                       const float v[4]) {
  if (FULL || (vec && c + 4 <= limit)) {
    if constexpr (sizeof(T) == 4) {
      *(float4*)(row + c) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      T tmp[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) tmp[j] = from_f<T>(v[j]);
      *(float2*)(row + c) = *(float2*)tmp;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c + j < limit) row[c + j] = from_f<T>(v[j]);
  }
}

// Register-resident rows: group i of a lane holds 4 consecutive columns.
// fp32: lane l's group i starts at column 4 (64 i + l) (one 16-byte load).
// 16-bit: groups 2p and 2p + 1 are 8 consecutive columns starting at
// 512 p + 8 l, so that one 16-byte load fills both; with an odd group count
// the last group alone covers columns 256 (NV - 1) + 4 l.  Either way a
// wavefront covers columns [0, 256 NV), each exactly once.
template <typename T, int NV>
__device__ __forceinline__ int64_t gcol(int i, int lane) {
  if constexpr (sizeof(T) == 4) {
    return ((int64_t)i * 64 + lane) * 4;
  } else {
    if (NV % 2 == 1 && i == NV - 1) return (int64_t)256 * (NV - 1) + 4 * lane;
    return ((int64_t)(i >> 1) * 64 + lane) * 8 + (i & 1) * 4;
  }
}
// The 16-bit wide loads need 16-byte aligned rows: the base 16-byte aligned
// and the leading dimension a multiple of 16 bytes.
inline bool vec16_ok(const void* p, int64_t ld, size_t esz) {
  return ((uintptr_t)p % 16) == 0 && ((ld * (int64_t)esz) % 16) == 0;
}
template <typename T, int NV, bool FULL>
__device__ __forceinline__ void load_groups(const T* __restrict__ row, int lane, int64_t limit, bool vec, float fill,
                                            float (&v)[NV][4]) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = gcol<T, NV>(i, lane);
    if constexpr (sizeof(T) == 2) {
      if (i % 2 == 0 && i + 1 < NV && (FULL || (vec && c + 8 <= limit))) {
        T tmp[8];
        *(uint4*)tmp = *(const uint4*)(row + c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[i][j] = to_f(tmp[j]);
          v[i + 1][j] = to_f(tmp[4 + j]);
        }
        continue;
      }
      if (i % 2 == 1 && (FULL || (vec && c + 4 <= limit))) continue;  // filled with group i - 1
    }
    load4<T, FULL>(row, c, limit, vec, fill, v[i]);
  }
}
template <typename T, int NV, bool FULL>
__device__ __forceinline__ void store_groups(T* __restrict__ row, int lane, int64_t limit, bool vec,
                                             const float (&v)[NV][4]) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = gcol<T, NV>(i, lane);
    if constexpr (sizeof(T) == 2) {
      if (i % 2 == 0 && i + 1 < NV && (FULL || (vec && c + 8 <= limit))) {
        T tmp[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          tmp[j] = from_f<T>(v[i][j]);
          tmp[4 + j] = from_f<T>(v[i + 1][j]);
        }
        *(uint4*)(row + c) = *(const uint4*)tmp;
        continue;
      }
      if (i % 2 == 1 && (FULL || (vec && c + 4 <= limit))) continue;  // stored with group i - 1
    }
    store4<T, FULL>(row, c, limit, vec, v[i]);
  }
}

// ── softmax family, register-resident (cols <= 256 * NV) ─────────────────
template <typename T, int NV, bool FULL>
__global__ void __launch_bounds__(256) softmax_wave(int op, const T* __restrict__ x, int64_t ldx,
                                                    T* __restrict__ y, int64_t ldy, int64_t rows,
                                                    int64_t cols, int64_t causal_rows, bool vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  T* yr = y + row * ldy;
  int64_t valid = cols;
  if (op == kSoftmaxCausal) {
    int64_t r = row % causal_rows;
    valid = r + 1 < cols ? r + 1 : cols;
  }
  float v[NV][4];
  float mx = -INFINITY;
  // Columns at or past `valid` hold -inf from here on (the guarded loads
  // fill them, the full-row path masks them), so exp gives them 0.
  load_groups<T, NV, FULL>(xr, lane, FULL ? cols : valid, vec, -INFINITY, v);
  if (FULL && op == kSoftmaxCausal) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = gcol<T, NV>(i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j >= valid) v[i][j] = -INFINITY;
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, v[i][j]);
  mx = wave_max(mx);
  // 16-bit outputs round to 2^-11 or coarser: exp(v - mx) as 2^(v log2 e -
  // mx log2 e) on the hardware exp2 (about 1 ulp of fp32) is well inside
  // that; fp32 rows keep the correctly range-reduced expf.
  constexpr float kLog2e = 1.4426950408889634f;
  const float mxl = mx * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float e;
      if constexpr (sizeof(T) == 2) e = __builtin_amdgcn_exp2f(fmaf(v[i][j], kLog2e, -mxl));
      else e = expf(v[i][j] - mx);
      sum += e;
      if (op != kLogSoftmax) v[i][j] = e;
    }
  }
  sum = wave_sum(sum);
  if (op == kLogSoftmax) {
    const float ls = logf(sum);
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = v[i][j] - mx - ls;
  } else {
    const float inv = 1.f / sum;  // one division per row, then products
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] *= inv;
  }
  store_groups<T, NV, FULL>(yr, lane, cols, vec, v);
}

// Block-wide reductions for 256 threads.
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  return sh[0] + sh[1] + sh[2] + sh[3];
}
__device__ __forceinline__ float block_max(float v, float* sh) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}

// ── softmax family, long rows: one 256-thread block per row, online max/sum ─
template <typename T>
__global__ void __launch_bounds__(256) softmax_block(int op, const T* __restrict__ x, int64_t ldx,
                                                     T* __restrict__ y, int64_t ldy, int64_t cols,
                                                     int64_t causal_rows) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  T* yr = y + row * ldy;
  int64_t valid = cols;
  if (op == kSoftmaxCausal) {
    int64_t r = row % causal_rows;
    valid = r + 1 < cols ? r + 1 : cols;
  }
  float m = -INFINITY, s = 0.f;
  for (int64_t c = threadIdx.x; c < valid; c += 256) {
    float v = to_f(xr[c]);
    if (v > m) { s = s * expf(m - v) + 1.f; m = v; }
    else s += expf(v - m);
  }
  float gm = block_max(m, sh);
  float part = (m == -INFINITY) ? 0.f : s * expf(m - gm);
  float gs = block_sum(part, sh);
  const float ls = logf(gs);
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float out;
    if (c >= valid) out = 0.f;
    else if (op == kLogSoftmax) out = to_f(xr[c]) - gm - ls;
    else out = expf(to_f(xr[c]) - gm) / gs;
    yr[c] = from_f<T>(out);
  }
}

// ── layer_norm ────────────────────────────────────────────────────────────
template <typename T, int NV, bool FULL>
__global__ void __launch_bounds__(256) layer_norm_wave(const T* __restrict__ x, int64_t ldx,
                                                       const T* __restrict__ g, const T* __restrict__ b,
                                                       T* __restrict__ y, int64_t rows, int64_t cols,
                                                       float eps, bool vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  T* yr = y + row * cols;
  float v[NV][4];
  float s = 0.f;
  load_groups<T, NV, FULL>(xr, lane, cols, vec, 0.f, v);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += v[i][j];
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = gcol<T, NV>(i, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float d = (c + j < cols) ? v[i][j] - mean : 0.f;
      q += d * d;
    }
  }
  const float var = wave_sum(q) / (float)cols;
  const float inv = 1.f / sqrtf(var + eps);
  float gv[NV][4], bv[NV][4];
  load_groups<T, NV, FULL>(g, lane, cols, vec, 0.f, gv);
  load_groups<T, NV, FULL>(b, lane, cols, vec, 0.f, bv);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) v[i][j] = gv[i][j] * (v[i][j] - mean) * inv + bv[i][j];
  store_groups<T, NV, FULL>(yr, lane, cols, vec, v);
}

template <typename T>
__global__ void __launch_bounds__(256) layer_norm_block(const T* __restrict__ x, int64_t ldx,
                                                        const T* __restrict__ g, const T* __restrict__ b,
                                                        T* __restrict__ y, int64_t cols, float eps) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  T* yr = y + row * cols;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) s += to_f(xr[c]);
  const float mean = block_sum(s, sh) / (float)cols;
  float q = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float d = to_f(xr[c]) - mean;
    q += d * d;
  }
  const float var = block_sum(q, sh) / (float)cols;
  const float inv = 1.f / sqrtf(var + eps);
  for (int64_t c = threadIdx.x; c < cols; c += 256)
    yr[c] = from_f<T>(to_f(g[c]) * (to_f(xr[c]) - mean) * inv + to_f(b[c]));
}

// ── layer_norm backward ───────────────────────────────────────────────────
// dx = inv * (dy*g - mean_j(dy*g) - xhat * mean_j(dy*g * xhat)) with the
// row's mean and inv = 1/sqrt(var + eps) recomputed from x by the forward
// kernel's own two-pass arithmetic (kernel_templates.rs:1601-1659).  stats
// (optional) receives [rows][2] = (mean, inv) for the parameter gradients.
// mean_in/rstd_in (optional, [rows]): the forward's saved statistics, used
// instead of recomputing them (torch's layer_norm backward carries no eps).
template <typename T, int NV, bool FULL>
__global__ void __launch_bounds__(256) layer_norm_bwd_wave(const T* __restrict__ dy, const T* __restrict__ x,
                                                           const T* __restrict__ g, T* __restrict__ dx,
                                                           float* __restrict__ stats, const T* __restrict__ mean_in,
                                                           const T* __restrict__ rstd_in, int64_t rows,
                                                           int64_t cols, float eps, bool vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  const T* dr = dy + row * cols;
  float v[NV][4], d[NV][4];
  float s = 0.f;
  load_groups<T, NV, FULL>(xr, lane, cols, vec, 0.f, v);
  load_groups<T, NV, FULL>(dr, lane, cols, vec, 0.f, d);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += v[i][j];
  float mean, inv;
  if (mean_in) {
    mean = to_f(mean_in[row]);
    inv = to_f(rstd_in[row]);
  } else {
    mean = wave_sum(s) / (float)cols;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = gcol<T, NV>(i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = (c + j < cols) ? v[i][j] - mean : 0.f;
        q += e * e;
      }
    }
    inv = 1.f / sqrtf(wave_sum(q) / (float)cols + eps);
  }
  float s1 = 0.f, s2 = 0.f;
  {
    float gv[NV][4];
    load_groups<T, NV, FULL>(g, lane, cols, vec, 0.f, gv);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = gcol<T, NV>(i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float xh = (c + j < cols) ? (v[i][j] - mean) * inv : 0.f;
        const float dg = d[i][j] * gv[i][j];  // 0 past the row (both loads fill 0)
        v[i][j] = xh;
        d[i][j] = dg;
        s1 += dg;
        s2 += dg * xh;
      }
    }
  }
  const float m1 = wave_sum(s1) / (float)cols, m2 = wave_sum(s2) / (float)cols;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) v[i][j] = inv * (d[i][j] - m1 - v[i][j] * m2);
  store_groups<T, NV, FULL>(dx + row * cols, lane, cols, vec, v);
  if (stats && lane == 0) {
    stats[2 * row] = mean;
    stats[2 * row + 1] = inv;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) layer_norm_bwd_block(const T* __restrict__ dy, const T* __restrict__ x,
                                                            const T* __restrict__ g, T* __restrict__ dx,
                                                            float* __restrict__ stats, const T* __restrict__ mean_in,
                                                            const T* __restrict__ rstd_in, int64_t cols, float eps) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  const T* dr = dy + row * cols;
  float mean, inv;
  if (mean_in) {
    mean = to_f(mean_in[row]);
    inv = to_f(rstd_in[row]);
  } else {
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) s += to_f(xr[c]);
    mean = block_sum(s, sh) / (float)cols;
    float q = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const float e = to_f(xr[c]) - mean;
      q += e * e;
    }
    inv = 1.f / sqrtf(block_sum(q, sh) / (float)cols + eps);
  }
  float s1 = 0.f, s2 = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float dg = to_f(dr[c]) * to_f(g[c]);
    s1 += dg;
    s2 += dg * (to_f(xr[c]) - mean) * inv;
  }
  const float m1 = block_sum(s1, sh) / (float)cols;
  const float m2 = block_sum(s2, sh) / (float)cols;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float xh = (to_f(xr[c]) - mean) * inv;
    dx[row * cols + c] = from_f<T>(inv * (to_f(dr[c]) * to_f(g[c]) - m1 - xh * m2));
  }
  if (stats && threadIdx.x == 0) {
    stats[2 * row] = mean;
    stats[2 * row + 1] = inv;
  }
}

// dgamma[c] = sum_r dy[r,c] * (x[r,c] - mean_r) * inv_r, dbeta[c] = sum_r dy[r,c].
// Stage 1: a 1024-thread block owns 64 columns of a chunk of kLnChunk rows
// (16 row slices, merged through LDS) and writes fp32 partials
// part[chunk][2][cols]; stage 2 adds the chunks in order (deterministic).
constexpr int kLnChunk = 256;

template <typename T>
__global__ void __launch_bounds__(1024) ln_param_partials(const T* __restrict__ dy, const T* __restrict__ x,
                                                          const float* __restrict__ stats, float* __restrict__ part,
                                                          int64_t rows, int64_t cols) {
  __shared__ float shg[16][64], shb[16][64];
  const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t chunk = blockIdx.y;
  const int64_t r1 = (chunk + 1) * kLnChunk < rows ? (chunk + 1) * kLnChunk : rows;
  float sg = 0.f, sb = 0.f;
  if (col < cols) {
#pragma unroll 4
    for (int64_t r = chunk * kLnChunk + slice; r < r1; r += 16) {
      const float d = to_f(dy[r * cols + col]);
      sb += d;
      sg += d * (to_f(x[r * cols + col]) - stats[2 * r]) * stats[2 * r + 1];
    }
  }
  shg[slice][lane] = sg;
  shb[slice][lane] = sb;
  __syncthreads();
  if (slice == 0 && col < cols) {
    float tg = 0.f, tb = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      tg += shg[i][lane];
      tb += shb[i][lane];
    }
    part[(chunk * 2) * cols + col] = tg;
    part[(chunk * 2 + 1) * cols + col] = tb;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) ln_param_final(const float* __restrict__ part, T* __restrict__ dg,
                                                      T* __restrict__ db, int64_t chunks, int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  float sg = 0.f, sb = 0.f;
  for (int64_t k = 0; k < chunks; ++k) {
    sg += part[(k * 2) * cols + c];
    sb += part[(k * 2 + 1) * cols + c];
  }
  dg[c] = from_f<T>(sg);
  db[c] = from_f<T>(sb);
}

// ── token + position embedding, optionally with the layer_norm after it ───
// x[r] = w1[i1[r]] + w2[i2[r]] (fp32 sum, rounded once, as embedding +
// embedding + add store it; an index outside its table gives a zero row, as
// the embedding kernel does), and with LN also y[r] = layer_norm(x[r]) from
// the stored (rounded) x by layer_norm_wave's own arithmetic.  GPT-2's
// wte[ids] + wpe[pos] -> ln_1 (python/applegpu_runtime/models/gpt2.py:84-178)
// in one launch instead of four.
template <typename T, typename I, int NV, bool LN>
__global__ void __launch_bounds__(256) embed_add_wave(const T* __restrict__ w1, const I* __restrict__ i1, int64_t v1,
                                                      const T* __restrict__ w2, const I* __restrict__ i2, int64_t v2,
                                                      T* __restrict__ x, const T* __restrict__ g,
                                                      const T* __restrict__ b, T* __restrict__ y,
                                                      bf16_t* __restrict__ ypk, int64_t rows, int64_t cols, float eps,
                                                      bool vec, PfArgs pf) {
  if (prefetch_block(pf)) return;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // one wavefront per row
  if (row >= rows) return;
  const int64_t a = (int64_t)i1[row], c = (int64_t)i2[row];
  const bool oka = a >= 0 && a < v1, okc = c >= 0 && c < v2;
  const T* ra = w1 + (oka ? a : 0) * cols;
  const T* rc = w2 + (okc ? c : 0) * cols;
  float v[NV][4];
  float s = 0.f;
  {
    float q[NV][4];
    load_groups<T, NV, false>(ra, lane, cols, vec, 0.f, v);
    load_groups<T, NV, false>(rc, lane, cols, vec, 0.f, q);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t col = gcol<T, NV>(i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // the sum as stored (rounded to T), which is what layer_norm reads
        v[i][j] = to_f(from_f<T>((oka ? v[i][j] : 0.f) + (okc ? q[i][j] : 0.f)));
        s += col + j < cols ? v[i][j] : 0.f;
      }
    }
  }
  store_groups<T, NV, false>(x + row * cols, lane, cols, vec, v);
  if constexpr (LN) {
    const float mean = wave_sum(s) / (float)cols;
    float qs = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t col = gcol<T, NV>(i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d = col + j < cols ? v[i][j] - mean : 0.f;
        qs += d * d;
      }
    }
    const float inv = 1.f / sqrtf(wave_sum(qs) / (float)cols + eps);
    float gv[NV][4], bv[NV][4];
    load_groups<T, NV, false>(g, lane, cols, vec, 0.f, gv);
    load_groups<T, NV, false>(b, lane, cols, vec, 0.f, bv);
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = gv[i][j] * (v[i][j] - mean) * inv + bv[i][j];
    if (y) store_groups<T, NV, false>(y + row * cols, lane, cols, vec, v);
    if constexpr (sizeof(T) == 4) {
      if (ypk) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int64_t col = gcol<T, NV>(i, lane);
          if (col < cols) x3_store4(ypk, cols / 16, row, col, v[i]);
        }
      }
    }
  }
}

// ── row reductions (one wavefront per row) ───────────────────────────────
template <typename TI, typename TO>
__global__ void __launch_bounds__(256) row_reduce_wave(int op, const TI* __restrict__ x, int64_t ldx,
                                                       TO* __restrict__ y, int64_t rows, int64_t cols,
                                                       int correction) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TI* xr = x + row * ldx;
  if (op == kRArgmax) {
    // First occurrence of the maximum; NaN counts as the maximum (the first
    // NaN wins), as torch.argmax on the CPU does.
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t c = lane; c < cols; c += 64) {
      float v = to_f(xr[c]);
      bool better = bi < 0 || (isnan(v) && !isnan(best)) || (!isnan(best) && v > best);
      if (better) { best = v; bi = c; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      float ob = __shfl_xor(best, m, 64);
      int64_t oi = __shfl_xor(bi, m, 64);
      bool take;
      if (oi < 0) take = false;
      else if (bi < 0) take = true;
      else if (isnan(ob) != isnan(best)) take = isnan(ob);
      else if (isnan(ob)) take = oi < bi;
      else take = ob > best || (ob == best && oi < bi);
      if (take) { best = ob; bi = oi; }
    }
    if (lane == 0) y[row] = (TO)(bi < 0 ? 0 : bi);
    return;
  }
  if (op == kRAmax) {
    float m = -INFINITY;
    for (int64_t c = lane; c < cols; c += 64) {
      float v = to_f(xr[c]);
      m = (isnan(v) || isnan(m)) ? NAN : fmaxf(m, v);
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
      float o = __shfl_xor(m, s, 64);
      m = (isnan(o) || isnan(m)) ? NAN : fmaxf(m, o);
    }
    if (lane == 0) y[row] = (TO)m;
    return;
  }
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += to_f(xr[c]);
  s = wave_sum(s);
  if (op == kRSum) { if (lane == 0) y[row] = (TO)s; return; }
  float mean = s / (float)cols;
  if (op == kRMean) { if (lane == 0) y[row] = (TO)mean; return; }
  float q = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    float d = to_f(xr[c]) - mean;
    q += d * d;
  }
  q = wave_sum(q);
  if (lane == 0) y[row] = (TO)(q / (float)(cols - correction));
}

// (value, index) candidate of an argmax: the first occurrence of the maximum,
// NaN counting as the maximum (the first NaN wins), as torch.argmax on the
// CPU does.  `bi` < 0 marks an empty candidate.
__device__ __forceinline__ void argmax_take(float& best, int64_t& bi, float ob, int64_t oi) {
  bool take;
  if (oi < 0) take = false;
  else if (bi < 0) take = true;
  else if (isnan(ob) != isnan(best)) take = isnan(ob);
  else if (isnan(ob)) take = oi < bi;
  else take = ob > best || (ob == best && oi < bi);
  if (take) { best = ob; bi = oi; }
}

// One thread's scan over its own elements, whose indices arrive in
// increasing order: a later value wins only if strictly larger, a NaN
// replaces only a non-NaN (so the first NaN wins), and -inf is never taken
// (bi stays -1, an empty candidate, which argmax_take ranks last).  Float
// compares and 32-bit indices: argmax_take's int64 branches per element had
// made the [8, 50257] argmax 24 us.
__device__ __forceinline__ void argmax_scan(float& best, int& bi, float v, int idx) {
  const bool take = v > best || (v != v && best == best);
  best = take ? v : best;
  bi = take ? idx : bi;
}

// Argmax of long rows (e.g. [batch, vocab] logits): one 1024-thread block per
// row, 16-byte loads over the aligned body of the row (rows of an odd length
// start unaligned: a scalar head and tail cover the rest); cols < 2^31.
template <typename TI>
__global__ void __launch_bounds__(1024) argmax_row_block(const TI* __restrict__ x, int64_t ldx,
                                                         int32_t* __restrict__ y, int64_t cols) {
  constexpr int VE = 16 / sizeof(TI);
  __shared__ float sb[16];
  __shared__ int64_t si[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row = blockIdx.x;
  const TI* xr = x + row * ldx;
  int64_t head = (int64_t)(((16 - ((uintptr_t)xr & 15)) & 15) / sizeof(TI));
  if (head > cols) head = cols;
  const int64_t nvec = (cols - head) / VE;
  const int64_t tail0 = head + nvec * VE;
  float best = -INFINITY;
  int b32 = -1;
  if (tid < head) argmax_scan(best, b32, to_f(xr[tid]), tid);
  const uint4* xv = (const uint4*)(xr + head);
  const int nv = (int)nvec, hd = (int)head;
  for (int v = tid; v < nv; v += 1024) {
    const uint4 u = xv[v];
    TI e[VE];
    __builtin_memcpy(e, &u, 16);
#pragma unroll
    for (int k = 0; k < VE; ++k) argmax_scan(best, b32, to_f(e[k]), hd + v * VE + k);
  }
  if (tail0 + tid < cols) argmax_scan(best, b32, to_f(xr[tail0 + tid]), (int)(tail0 + tid));
  int64_t bi = b32;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(best, m, 64);
    const int64_t oi = __shfl_xor(bi, m, 64);
    argmax_take(best, bi, ob, oi);
  }
  if (lane == 0) { sb[w] = best; si[w] = bi; }
  __syncthreads();
  if (w != 0) return;
  best = lane < 16 ? sb[lane] : -INFINITY;
  bi = lane < 16 ? si[lane] : -1;
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(best, m, 64);
    const int64_t oi = __shfl_xor(bi, m, 64);
    argmax_take(best, bi, ob, oi);
  }
  if (lane == 0) y[row] = (int32_t)(bi < 0 ? 0 : bi);
}

// Integer sums stay exact in 64-bit.
template <typename TI, typename TO>
__global__ void __launch_bounds__(256) row_sum_int(const TI* __restrict__ x, int64_t ldx, TO* __restrict__ y,
                                                   int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TI* xr = x + row * ldx;
  long long s = 0;
  for (int64_t c = lane; c < cols; c += 64) s += (long long)xr[c];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (lane == 0) y[row] = (TO)s;
}

template <typename T>
__global__ void __launch_bounds__(256) softmax_bwd_wave(const T* __restrict__ dy, const T* __restrict__ yv,
                                                        T* __restrict__ dx, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* a = dy + row * cols;
  const T* b = yv + row * cols;
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += to_f(a[c]) * to_f(b[c]);
  s = wave_sum(s);
  for (int64_t c = lane; c < cols; c += 64) dx[row * cols + c] = from_f<T>(to_f(b[c]) * (to_f(a[c]) - s));
}

// ── per-row int8 quantize: one 256-thread block per row ───────────────────
// scale = absmax/127 (fp32), q = clamp(rint(x / scale), -128, 127); x / scale
// is IEEE division and rint rounds half to even, as torch.round does.  A row
// of zeros gets scale 0 and codes 0.
template <typename T, int NV, bool FULL>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const T* __restrict__ x, int8_t* __restrict__ q,
                                                            float* __restrict__ scale, int64_t cols, bool vec) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  int8_t* qr = q + row * cols;
  float v[NV][4];
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    int64_t c = ((int64_t)i * 256 + threadIdx.x) * 4;
    load4<T, FULL>(xr, c, cols, vec, 0.f, v[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fabsf(v[i][j]));
  }
  const float amax = block_max(m, sh);
  const float sc = amax / 127.f;
  if (threadIdx.x == 0) scale[row] = sc;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    int64_t c = ((int64_t)i * 256 + threadIdx.x) * 4;
    int8_t b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float r = sc == 0.f ? 0.f : rintf(v[i][j] / sc);
      r = fminf(fmaxf(r, -128.f), 127.f);
      b[j] = (int8_t)(int)r;
    }
    if (FULL || (vec && c + 4 <= cols)) {
      *(int32_t*)(qr + c) = *(int32_t*)b;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < cols) qr[c + j] = b[j];
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) quantize_rows_loop(const T* __restrict__ x, int8_t* __restrict__ q,
                                                          float* __restrict__ scale, int64_t cols) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float m = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) m = fmaxf(m, fabsf(to_f(xr[c])));
  const float sc = block_max(m, sh) / 127.f;
  if (threadIdx.x == 0) scale[row] = sc;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float r = sc == 0.f ? 0.f : rintf(to_f(xr[c]) / sc);
    q[row * cols + c] = (int8_t)(int)fminf(fmaxf(r, -128.f), 127.f);
  }
}

// y[r, c] = q[r, c] * scale[r]; grid.y walks rows, 4 codes per thread (one
// 4-byte load, one 16-byte fp32 store).  VEC: cols % 4 == 0 and both sides
// aligned, so every thread in range takes the vector path.
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) dequantize_rows_kernel(const int8_t* __restrict__ q,
                                                              const float* __restrict__ scale,
                                                              T* __restrict__ y, int64_t rows, int64_t cols) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= cols) return;
  for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {
    const float sc = scale[row];
    const int8_t* qr = q + row * cols;
    T* yr = y + row * cols;
    float v[4];
    if constexpr (VEC) {
      const int32_t w = *(const int32_t*)(qr + c);
      const int8_t* b = (const int8_t*)&w;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (float)b[j] * sc;
      store4<T, true>(yr, c, cols, true, v);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = c + j < cols ? (float)qr[c + j] * sc : 0.f;
      store4(yr, c, cols, false, v);
    }
  }
}

// ── 16-values-per-thread quantize (C5's [8192, 8192]) ─────────────────────
// A thread owns groups of 16 consecutive values: 64 bytes of fp32 in (four
// 16-byte loads), 16 bytes of codes out (one store).  C5: 60 us, 0.69 of HBM
// peak, against 65 us with four values per thread and 4-byte code stores.
// (The same layout for dequantize measured 96 us: its 64-byte-per-lane
// stores are not coalesced within an instruction; dequantize_rows_4x4 keeps
// every access coalesced instead.  Nontemporal loads and stores made both
// far slower.)
typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ void load16(const T* __restrict__ p, float (&v)[16]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4_v a = ((const f32x4_v*)p)[i];
      v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4_v a = ((const u32x4_v*)p)[i];
      const T* h = (const T*)&a;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[8 * i + j] = to_f(h[j]);
    }
  }
}
// Per-row int8 quantize, one 256-thread block per row of 4096 NG values
// (cols % 4096 == 0, 16-byte aligned rows); the arithmetic of
// quantize_rows_kernel.  NT: the codes are written with nontemporal stores
// (for outputs too large to stay cached for a consumer: C5's 64 MiB of codes
// 59.9 -> 57.5 us, measured over three rotating 256 MiB inputs).
template <typename T, int NG, bool NT>
__global__ void __launch_bounds__(256) quantize_rows_v16(const T* __restrict__ x, int8_t* __restrict__ q,
                                                         float* __restrict__ scale, int64_t cols) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  int8_t* qr = q + row * cols;
  float v[NG][16];
#pragma unroll
  for (int g = 0; g < NG; ++g) load16<T>(xr + ((int64_t)g * 256 + threadIdx.x) * 16, v[g]);
  float m = 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(v[g][j]));
  const float sc = block_max(m, sh) / 127.f;
  if (threadIdx.x == 0) scale[row] = sc;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    u32x4_v out;
    int8_t* b = (int8_t*)&out;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float r = sc == 0.f ? 0.f : rintf(v[g][j] / sc);
      r = fminf(fmaxf(r, -128.f), 127.f);
      b[j] = (int8_t)(int)r;
    }
    u32x4_v* dst = (u32x4_v*)(qr + ((int64_t)g * 256 + threadIdx.x) * 16);
    if constexpr (NT) __builtin_nontemporal_store(out, dst);
    else *dst = out;
  }
}

// y = codes * scale[row] for a block of 4096 columns of one row.  The codes
// come in with one 16-byte load per thread and are staged through LDS; then
// thread t writes columns 4 (t + 256 i) .. + 3 for i = 0..3, so each of its
// four stores (16 bytes of fp32) is one coalesced wavefront access.
// cols % 4096 == 0, 16-byte aligned rows.  NT: nontemporal stores, for
// outputs too large to stay cached for a consumer.  C5 ([8192, 8192] fp32,
// codes rotating over 6 copies so that they come from HBM): 57.8 us with NT
// stores against 60.1 us for 4-byte code loads and plain stores (and 68 us
// with one group per thread).
template <typename T, bool NT>
__global__ void __launch_bounds__(256) dequantize_rows_lds(const int8_t* __restrict__ q,
                                                           const float* __restrict__ scale, T* __restrict__ y,
                                                           int64_t cols) {
  __shared__ __attribute__((aligned(16))) int8_t codes[4096];
  const int64_t row = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * 4096;
  const float sc = scale[row];
  *(u32x4_v*)&codes[threadIdx.x * 16] = *(const u32x4_v*)(q + row * cols + base + threadIdx.x * 16);
  __syncthreads();
  T* yr = y + row * cols + base;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x * 4 + 1024 * i;
    const int32_t w = *(const int32_t*)&codes[c];
    const int8_t* b = (const int8_t*)&w;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (float)b[j] * sc;
    if constexpr (NT && sizeof(T) == 4) {
      f32x4_v o = {v[0], v[1], v[2], v[3]};
      __builtin_nontemporal_store(o, (f32x4_v*)(yr + c));
    } else if constexpr (NT) {
      T h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = from_f<T>(v[j]);
      typedef unsigned int u32x2_v __attribute__((ext_vector_type(2)));
      __builtin_nontemporal_store(*(const u32x2_v*)h, (u32x2_v*)(yr + c));
    } else {
      store4<T, true>(yr, c, 4096, true, v);
    }
  }
}

// Outputs at least this large are written with nontemporal stores by the
// quantize / dequantize kernels: they cannot all stay in the 256 MB Infinity
// Cache for a consumer, and bypassing it measured 4-5 % faster.
constexpr int64_t kNtStoreBytes = (int64_t)64 << 20;

// Per-row int8 quantize with one wavefront per row for rows of up to 2048
// columns: the row stays in registers, the absmax is a wave reduction (no
// block barrier), then the codes are written 4 per lane.  Longer rows take
// one 256-thread block each (quantize_rows_kernel), measured faster there.
template <typename T, int NV, bool FULL>
__global__ void __launch_bounds__(256) quantize_rows_wave(const T* __restrict__ x, int8_t* __restrict__ q,
                                                          float* __restrict__ scale, int64_t rows, int64_t cols,
                                                          bool vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  int8_t* qr = q + row * cols;
  float v[NV][4];
  float m = 0.f;
  load_groups<T, NV, FULL>(xr, lane, cols, vec, 0.f, v);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fabsf(v[i][j]));
  const float sc = wave_max(m) / 127.f;
  if (lane == 0) scale[row] = sc;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = gcol<T, NV>(i, lane);
    int8_t b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float r = sc == 0.f ? 0.f : rintf(v[i][j] / sc);
      r = fminf(fmaxf(r, -128.f), 127.f);
      b[j] = (int8_t)(int)r;
    }
    if (FULL || (vec && c + 4 <= cols)) {
      *(int32_t*)(qr + c) = *(int32_t*)b;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < cols) qr[c + j] = b[j];
    }
  }
}

bool vec_ok(const void* p, int64_t ld, size_t esz) {
  return (((uintptr_t)p) % (4 * esz)) == 0 && (ld % 4) == 0;
}

unsigned rows_grid(int64_t rows) { return (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock); }

template <typename T, int NV>
void sm_nv(int op, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t cols, int64_t crow,
           bool vec, hipStream_t s) {
  if (vec && cols == NV * 256)
    hipLaunchKernelGGL((softmax_wave<T, NV, true>), dim3(rows_grid(rows)), dim3(256), 0, s, op, (const T*)x, ldx,
                       (T*)y, ldy, rows, cols, crow, vec);
  else
    hipLaunchKernelGGL((softmax_wave<T, NV, false>), dim3(rows_grid(rows)), dim3(256), 0, s, op, (const T*)x, ldx,
                       (T*)y, ldy, rows, cols, crow, vec);
}

template <typename T>
void sm_launch(int op, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t cols, int64_t crow,
               hipStream_t s) {
  bool vec = vec16_ok(x, ldx, sizeof(T)) && vec16_ok(y, ldy, sizeof(T));
  switch ((cols + 255) / 256) {
    case 1: sm_nv<T, 1>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 2: sm_nv<T, 2>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 3: sm_nv<T, 3>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 4: sm_nv<T, 4>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 5: sm_nv<T, 5>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 6: sm_nv<T, 6>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 7: sm_nv<T, 7>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    case 8: sm_nv<T, 8>(op, x, ldx, y, ldy, rows, cols, crow, vec, s); break;
    default:
      hipLaunchKernelGGL((softmax_block<T>), dim3((unsigned)rows), dim3(256), 0, s, op, (const T*)x, ldx, (T*)y, ldy,
                         cols, crow);
  }
}

template <typename T, int NV>
void ln_nv(const void* x, int64_t ldx, const void* g, const void* b, void* y, int64_t rows, int64_t cols, float eps,
           bool vec, hipStream_t s) {
  if (vec && cols == NV * 256)
    hipLaunchKernelGGL((layer_norm_wave<T, NV, true>), dim3(rows_grid(rows)), dim3(256), 0, s, (const T*)x, ldx,
                       (const T*)g, (const T*)b, (T*)y, rows, cols, eps, vec);
  else
    hipLaunchKernelGGL((layer_norm_wave<T, NV, false>), dim3(rows_grid(rows)), dim3(256), 0, s, (const T*)x, ldx,
                       (const T*)g, (const T*)b, (T*)y, rows, cols, eps, vec);
}

template <typename T>
void ln_launch(const void* x, int64_t ldx, const void* g, const void* b, void* y, int64_t rows, int64_t cols,
               float eps, hipStream_t s) {
  bool vec = vec16_ok(x, ldx, sizeof(T)) && vec16_ok(y, cols, sizeof(T)) && vec16_ok(g, 0, sizeof(T)) &&
             vec16_ok(b, 0, sizeof(T));
  switch ((cols + 255) / 256) {
    case 1: ln_nv<T, 1>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 2: ln_nv<T, 2>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 3: ln_nv<T, 3>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 4: ln_nv<T, 4>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 5: ln_nv<T, 5>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 6: ln_nv<T, 6>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 7: ln_nv<T, 7>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    case 8: ln_nv<T, 8>(x, ldx, g, b, y, rows, cols, eps, vec, s); break;
    default:
      hipLaunchKernelGGL((layer_norm_block<T>), dim3((unsigned)rows), dim3(256), 0, s, (const T*)x, ldx, (const T*)g,
                         (const T*)b, (T*)y, cols, eps);
  }
}

struct LnbArgs {
  const void *dy, *x, *g, *mean_in, *rstd_in;
  void* dx;
  float* stats;
  int64_t rows, cols;
  float eps;
};

template <typename T, int NV>
void lnb_nv(const LnbArgs& a, bool vec, hipStream_t s) {
  if (vec && a.cols == NV * 256)
    hipLaunchKernelGGL((layer_norm_bwd_wave<T, NV, true>), dim3(rows_grid(a.rows)), dim3(256), 0, s, (const T*)a.dy,
                       (const T*)a.x, (const T*)a.g, (T*)a.dx, a.stats, (const T*)a.mean_in, (const T*)a.rstd_in,
                       a.rows, a.cols, a.eps, vec);
  else
    hipLaunchKernelGGL((layer_norm_bwd_wave<T, NV, false>), dim3(rows_grid(a.rows)), dim3(256), 0, s,
                       (const T*)a.dy, (const T*)a.x, (const T*)a.g, (T*)a.dx, a.stats, (const T*)a.mean_in,
                       (const T*)a.rstd_in, a.rows, a.cols, a.eps, vec);
}

template <typename T>
void lnb_launch(const LnbArgs& a, hipStream_t s) {
  const bool vec = vec16_ok(a.x, a.cols, sizeof(T)) && vec16_ok(a.dy, a.cols, sizeof(T)) &&
                   vec16_ok(a.dx, a.cols, sizeof(T)) && vec16_ok(a.g, 0, sizeof(T));
  switch ((a.cols + 255) / 256) {
    case 1: lnb_nv<T, 1>(a, vec, s); break;
    case 2: lnb_nv<T, 2>(a, vec, s); break;
    case 3: lnb_nv<T, 3>(a, vec, s); break;
    case 4: lnb_nv<T, 4>(a, vec, s); break;
    case 5: lnb_nv<T, 5>(a, vec, s); break;
    case 6: lnb_nv<T, 6>(a, vec, s); break;
    case 7: lnb_nv<T, 7>(a, vec, s); break;
    case 8: lnb_nv<T, 8>(a, vec, s); break;
    default:
      hipLaunchKernelGGL((layer_norm_bwd_block<T>), dim3((unsigned)a.rows), dim3(256), 0, s, (const T*)a.dy,
                         (const T*)a.x, (const T*)a.g, (T*)a.dx, a.stats, (const T*)a.mean_in, (const T*)a.rstd_in,
                         a.cols, a.eps);
  }
}

template <typename T>
void q_launch(const void* x, int8_t* q, float* scale, int64_t rows, int64_t cols, hipStream_t s) {
  bool vec = vec16_ok(x, cols, sizeof(T)) && vec_ok(q, cols, 1);
  if (cols <= 2048) {
    const int64_t nw = (cols + 255) / 256;  // float4 groups per lane
    dim3 gw(rows_grid(rows));
#define AGPU_QW(NV)                                                                                     \
  if (vec && cols == NV * 256)                                                                          \
    hipLaunchKernelGGL((quantize_rows_wave<T, NV, true>), gw, dim3(256), 0, s, (const T*)x, q, scale, rows, cols, vec); \
  else                                                                                                  \
    hipLaunchKernelGGL((quantize_rows_wave<T, NV, false>), gw, dim3(256), 0, s, (const T*)x, q, scale, rows, cols, vec);
    if (nw <= 4) { AGPU_QW(4) }
    else { AGPU_QW(8) }
#undef AGPU_QW
    return;
  }
  int64_t nv = (cols + 1023) / 1024;
  dim3 g((unsigned)rows);
  if (vec && cols % 4096 == 0 && cols <= 4096 * 4 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 15) == 0 &&
      (cols * (int64_t)sizeof(T)) % 16 == 0) {
    const bool nt = rows * cols >= kNtStoreBytes;
#define AGPU_QV(NG)                                                                                        \
  if (nt) hipLaunchKernelGGL((quantize_rows_v16<T, NG, true>), g, dim3(256), 0, s, (const T*)x, q, scale, cols); \
  else hipLaunchKernelGGL((quantize_rows_v16<T, NG, false>), g, dim3(256), 0, s, (const T*)x, q, scale, cols);
    switch (cols / 4096) {
      case 1: AGPU_QV(1) return;
      case 2: AGPU_QV(2) return;
      case 3: AGPU_QV(3) return;
      default: AGPU_QV(4) return;
    }
#undef AGPU_QV
  }
#define AGPU_Q(NV)                                                                                   \
  if (vec && cols == NV * 1024)                                                                      \
    hipLaunchKernelGGL((quantize_rows_kernel<T, NV, true>), g, dim3(256), 0, s, (const T*)x, q, scale, cols, vec); \
  else                                                                                               \
    hipLaunchKernelGGL((quantize_rows_kernel<T, NV, false>), g, dim3(256), 0, s, (const T*)x, q, scale, cols, vec);
  if (nv <= 1) { AGPU_Q(1) }
  else if (nv <= 2) { AGPU_Q(2) }
  else if (nv <= 4) { AGPU_Q(4) }
  else if (nv <= 8) { AGPU_Q(8) }
#undef AGPU_Q
  else hipLaunchKernelGGL((quantize_rows_loop<T>), g, dim3(256), 0, s, (const T*)x, q, scale, cols);
}

}  // namespace

void softmax_rows(int op, DType dt, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                  int64_t cols, int64_t causal_rows, hipStream_t s) {
  if (rows == 0 || cols == 0) return;
  if (causal_rows <= 0) causal_rows = rows;
  AGPU_FLOAT_SWITCH(dt, sm_launch<T>(op, x, ldx, y, ldy, rows, cols, causal_rows, s));
  check_launch("softmax_rows");
}

void layer_norm(DType dt, const void* x, int64_t ldx, const void* gamma, const void* beta, void* y,
                int64_t rows, int64_t cols, float eps, hipStream_t s) {
  if (rows == 0 || cols == 0) return;
  AGPU_FLOAT_SWITCH(dt, ln_launch<T>(x, ldx, gamma, beta, y, rows, cols, eps, s));
  check_launch("layer_norm");
}

void row_reduce(int op, DType in, DType out, const void* x, int64_t ldx, void* y, int64_t rows,
                int64_t cols, int correction, hipStream_t s) {
  if (rows == 0) return;
  if (op == kRArgmax) {
    if (out != DType::I32) fail("argmax output must be int32");
    if (rows > 0x7fffffffLL) fail("argmax: too many rows");
    AGPU_ALL_SWITCH(in, {
      if constexpr (std::is_same<T, int64_t>::value)
        fail("argmax over int64 is not supported");
      else if (cols >= 4096 && cols < 0x7fffffffLL)
        hipLaunchKernelGGL((argmax_row_block<T>), dim3((unsigned)rows), dim3(1024), 0, s, (const T*)x, ldx,
                           (int32_t*)y, cols);
      else
        hipLaunchKernelGGL((row_reduce_wave<T, int32_t>), dim3(rows_grid(rows)), dim3(256), 0, s, op,
                           (const T*)x, ldx, (int32_t*)y, rows, cols, correction);
    });
  } else if (dtype_is_float(in)) {
    if (out != in) fail("row reduction output dtype must match input");
    AGPU_FLOAT_SWITCH(in, hipLaunchKernelGGL((row_reduce_wave<T, T>), dim3(rows_grid(rows)), dim3(256), 0, s,
                                             op, (const T*)x, ldx, (T*)y, rows, cols, correction));
  } else if (op == kRSum) {
    AGPU_ALL_SWITCH(in, {
      typedef T TI;
      AGPU_ALL_SWITCH(out, hipLaunchKernelGGL((row_sum_int<TI, T>), dim3(rows_grid(rows)), dim3(256), 0, s,
                                              (const TI*)x, ldx, (T*)y, rows, cols));
    });
  } else if (op == kRAmax) {
    AGPU_ALL_SWITCH(in, hipLaunchKernelGGL((row_reduce_wave<T, T>), dim3(rows_grid(rows)), dim3(256), 0, s,
                                           op, (const T*)x, ldx, (T*)y, rows, cols, correction));
  } else {
    fail("row reduction %d needs a float dtype", op);
  }
  check_launch("row_reduce");
}

void softmax_backward(DType dt, const void* dy, const void* y, void* dx, int64_t rows, int64_t cols,
                      hipStream_t s) {
  if (rows == 0) return;
  AGPU_FLOAT_SWITCH(dt, hipLaunchKernelGGL((softmax_bwd_wave<T>), dim3(rows_grid(rows)), dim3(256), 0, s,
                                           (const T*)dy, (const T*)y, (T*)dx, rows, cols));
  check_launch("softmax_backward");
}

void layer_norm_backward(DType dt, const void* dy, const void* x, const void* gamma, void* dx, float* stats,
                         const void* mean_in, const void* rstd_in, int64_t rows, int64_t cols, float eps,
                         hipStream_t s) {
  if (rows == 0 || cols == 0) return;
  if (rows > 0x7fffffffLL) fail("layer_norm_backward: too many rows");
  if ((mean_in == nullptr) != (rstd_in == nullptr)) fail("layer_norm_backward: saved mean without rstd");
  const LnbArgs a{dy, x, gamma, mean_in, rstd_in, dx, stats, rows, cols, eps};
  AGPU_FLOAT_SWITCH(dt, lnb_launch<T>(a, s));
  check_launch("layer_norm_backward");
}

size_t layer_norm_param_ws_bytes(int64_t rows, int64_t cols) {
  return (size_t)((rows + kLnChunk - 1) / kLnChunk) * 2 * (size_t)cols * sizeof(float);
}

void layer_norm_param_grads(DType dt, const void* dy, const void* x, const float* stats, void* dgamma, void* dbeta,
                            float* ws, int64_t rows, int64_t cols, hipStream_t s) {
  if (cols == 0) return;
  const int64_t chunks = (rows + kLnChunk - 1) / kLnChunk;
  if (chunks > 65535) fail("layer_norm_backward: %lld rows exceed the parameter-gradient grid", (long long)rows);
  AGPU_FLOAT_SWITCH(dt, {
    if (chunks > 0)
      hipLaunchKernelGGL((ln_param_partials<T>), dim3((unsigned)((cols + 63) / 64), (unsigned)chunks), dim3(1024), 0,
                         s, (const T*)dy, (const T*)x, stats, ws, rows, cols);
    hipLaunchKernelGGL((ln_param_final<T>), dim3((unsigned)((cols + 255) / 256)), dim3(256), 0, s, (const float*)ws,
                       (T*)dgamma, (T*)dbeta, chunks, cols);
  });
  check_launch("layer_norm_param_grads");
}

bool embedding_add_ok(int64_t cols) { return cols > 0 && cols <= 2048; }

namespace {
struct EaArgs {
  const void *w1, *i1, *w2, *i2, *g, *b;
  void *x, *y, *ypk;
  int64_t v1, v2, rows, cols;
  float eps;
  bool vec;
};

template <typename T, typename I, int NV>
void ea_nv(const EaArgs& a, hipStream_t s) {
  // up to 1024 rows, one row per block: the rows reach as many CUs
  const int rpb = a.rows <= 1024 ? 1 : kRowsPerBlock;
  const unsigned main = (unsigned)((a.rows + rpb - 1) / rpb);
  const PfArgs pf = make_prefetch((int)main, 64 * rpb);
  const dim3 grid(main + (unsigned)pf.blocks), block(64 * rpb);
  if (a.g)
    hipLaunchKernelGGL((embed_add_wave<T, I, NV, true>), grid, block, 0, s, (const T*)a.w1,
                       (const I*)a.i1, a.v1, (const T*)a.w2, (const I*)a.i2, a.v2, (T*)a.x, (const T*)a.g,
                       (const T*)a.b, (T*)a.y, (bf16_t*)a.ypk, a.rows, a.cols, a.eps, a.vec, pf);
  else
    hipLaunchKernelGGL((embed_add_wave<T, I, NV, false>), grid, block, 0, s, (const T*)a.w1,
                       (const I*)a.i1, a.v1, (const T*)a.w2, (const I*)a.i2, a.v2, (T*)a.x, (const T*)nullptr,
                       (const T*)nullptr, (T*)nullptr, (bf16_t*)nullptr, a.rows, a.cols, a.eps, a.vec, pf);
}

template <typename T, typename I>
void ea_launch(const EaArgs& a, hipStream_t s) {
  switch ((a.cols + 255) / 256) {
    case 1: ea_nv<T, I, 1>(a, s); break;
    case 2: ea_nv<T, I, 2>(a, s); break;
    case 3: ea_nv<T, I, 3>(a, s); break;
    case 4: ea_nv<T, I, 4>(a, s); break;
    case 5: ea_nv<T, I, 5>(a, s); break;
    case 6: ea_nv<T, I, 6>(a, s); break;
    default: ea_nv<T, I, 8>(a, s);
  }
}
}  // namespace

void embedding_add(DType dt, const void* w1, DType i1_dt, const void* i1, int64_t v1, const void* w2, DType i2_dt,
                   const void* i2, int64_t v2, void* x, const void* gamma, const void* beta, void* y, void* ypk,
                   int64_t rows, int64_t cols, float eps, hipStream_t s) {
  if (rows == 0) return;
  if (!embedding_add_ok(cols)) fail("embedding_add: %lld columns (at most 2048)", (long long)cols);
  if (i1_dt != i2_dt) fail("embedding_add: index dtypes differ");
  if (rows > 0x7fffffffLL) fail("embedding_add: too many rows");
  if (ypk && (dt != DType::F32 || cols % 16 != 0 || ((uintptr_t)ypk & 15)))
    fail("embedding_add: packed layer_norm rows need fp32, 16-aligned columns");
  const size_t es = dtype_size(dt);
  const bool ln = gamma != nullptr;
  EaArgs a{w1, i1, w2, i2, gamma, beta, x, y, ypk, v1, v2, rows, cols, eps, false};
  a.vec = vec16_ok(w1, cols, es) && vec16_ok(w2, cols, es) && vec16_ok(x, cols, es) &&
          (!ln || ((y == nullptr || vec16_ok(y, cols, es)) && vec16_ok(gamma, 0, es) && vec16_ok(beta, 0, es)));
  AGPU_FLOAT_SWITCH(dt, {
    typedef T TV;
    AGPU_INT_SWITCH(i1_dt, ea_launch<TV, I>(a, s));
  });
  check_launch("embedding_add");
}

void quantize_rows(DType in, const void* x, int8_t* q, float* scale, int64_t rows, int64_t cols,
                   hipStream_t s) {
  if (rows == 0) return;
  AGPU_FLOAT_SWITCH(in, q_launch<T>(x, q, scale, rows, cols, s));
  check_launch("quantize_rows");
}

void dequantize_rows(DType out, const int8_t* q, const float* scale, void* y, int64_t rows, int64_t cols,
                     hipStream_t s) {
  if (rows == 0 || cols == 0) return;
  AGPU_FLOAT_SWITCH(out, {
    if (cols % 4096 == 0 && rows <= 65535 && ((uintptr_t)q % 16) == 0 && ((uintptr_t)y % 16) == 0) {
      const dim3 g((unsigned)(cols / 4096), (unsigned)rows);
      if (rows * cols * (int64_t)sizeof(T) >= kNtStoreBytes)
        hipLaunchKernelGGL((dequantize_rows_lds<T, true>), g, dim3(256), 0, s, q, scale, (T*)y, cols);
      else
        hipLaunchKernelGGL((dequantize_rows_lds<T, false>), g, dim3(256), 0, s, q, scale, (T*)y, cols);
      check_launch("dequantize_rows");
      return;
    }
    const bool vec = ((uintptr_t)q % 4) == 0 && ((uintptr_t)y % (4 * sizeof(T))) == 0 && cols % 4 == 0;
    dim3 grid((unsigned)((cols + 1023) / 1024), (unsigned)(rows < 65535 ? rows : 65535));
    if (vec) hipLaunchKernelGGL((dequantize_rows_kernel<T, true>), grid, dim3(256), 0, s, q, scale, (T*)y, rows, cols);
    else hipLaunchKernelGGL((dequantize_rows_kernel<T, false>), grid, dim3(256), 0, s, q, scale, (T*)y, rows, cols);
  });
  check_launch("dequantize_rows");
}

}  // namespace k
}  // namespace agpu
