// fp32 GEMM against weights packed once as bf16 hi/lo MFMA fragments, for
// activations of few rows (GPT-2's M = 128 projections).
//
// A (fp32 activations) x B (fp32 weights, static) with B split ahead of time:
// hi = bf16(b), lo = bf16(b - hi), stored in the B-operand order of
// v_mfma_f32_32x32x16_bf16.  For column strip s (32 columns from 32 s) and
// k step t (16 k values from 16 t), lane l holds B(16 t + 8 (l / 32) + j,
// 32 s + l % 32), j = 0..7, as 8 bf16: element ((s T + t) 2 + h) 512 + 8 l + j
// of the packed array (h = 0 hi, 1 lo; T = ceil(K / 16); zero past K and N).
// One wavefront's fragment is then one contiguous 1 KB read, and the weights
// need no conversion at run time.
//
// One block (4 wavefronts in a WR x WC grid, each owning FR x FC 32x32
// output blocks) covers BM = 32 FR WR rows and BN = 32 FC WC columns over
// KT k steps (16 KT k values) of the block's split: it issues every global
// load of its range first (each wave's B fragments, then the block's A tile),
// splits A into hi/lo bf16 in LDS once, and runs 3 KT FR FC MFMAs per wave
// (lo*hi, hi*lo, hi*hi per fragment pair, fp32 accumulation; Henry, Tang,
// Heinecke 2019).  With one memory round trip per block and no loop-carried
// loads, the launch costs one load latency plus its MFMAs; the K range is
// split across blocks so that the grid fills the GPU, and the partial sums
// go through the same split-K reductions (and epilogues) as the tiled GEMM.
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {

namespace {

// One lane-fragment of the packed layout: thread gid of S T 64 (S column
// strips, T k steps).  Every load is issued unconditionally from a clamped
// in-range address (the padding past K and N is zeroed after the load): a
// per-lane branch around the loads would make each of them wait as it
// issues.
struct PackSrc {
  const float* B;
  int64_t b_sk, b_sn, K, N, T;
  bf16_t* out;
};
__device__ __forceinline__ void pack_x3_one(const PackSrc& a, int64_t gid) {
  const int64_t S = (a.N + 31) / 32;
  if (gid >= S * a.T * 64) return;
  const int l = (int)(gid & 63);
  const int64_t st = gid >> 6;
  const int64_t t = st % a.T, s = st / a.T;
  const int64_t n = 32 * s + (l & 31);
  const int64_t k0 = 16 * t + 8 * (l >> 5);
  const bool nin = n < a.N;
  const int64_t nc = nin ? n : a.N - 1;
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t k = k0 + j;
    x[j] = a.B[(k < a.K ? k : a.K - 1) * a.b_sk + nc * a.b_sn];
  }
  bf16x8_t h, lo;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bf16_t hj, lj;
    split_bf16(nin && k0 + j < a.K ? x[j] : 0.f, hj, lj);
    h[j] = hj;
    lo[j] = lj;
  }
  bf16_t* dst = a.out + (st * 2) * 512 + l * 8;
  *(bf16x8_t*)dst = h;
  *(bf16x8_t*)(dst + 512) = lo;
}

__global__ void __launch_bounds__(256) pack_x3_kernel(PackSrc a) {
  pack_x3_one(a, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// Two operands in one launch: blocks [0, nb0) pack a, the rest b.
__global__ void __launch_bounds__(256) pack_x3_pair_kernel(PackSrc a, PackSrc b, int64_t nb0) {
  if ((int64_t)blockIdx.x < nb0) pack_x3_one(a, (int64_t)blockIdx.x * 256 + threadIdx.x);
  else pack_x3_one(b, ((int64_t)blockIdx.x - nb0) * 256 + threadIdx.x);
}

// As pack_x3_pair_kernel, and acc[n] += alpha * sum_k a(k, n) for a's
// columns (an SGD bias step folded into the packing of the gradient).
// Blocks [0, nb0) take one 32-column strip of a each: wave w packs k steps
// t = w, w + 4, ... (the fragments pack_x3_one writes for them) while
// summing its lanes' values; the four waves' and two half-waves' sums are
// then added in a fixed order, so results repeat exactly.
__device__ __forceinline__ void pack_pair_sum_block(const PackSrc& a, const PackSrc& b, int64_t nb0,
                                                    float* __restrict__ acc, float alpha, int64_t bid,
                                                    float (&red)[4][64]) {
  if (bid >= nb0) {
    pack_x3_one(b, (bid - nb0) * 256 + threadIdx.x);
    return;
  }
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t s = bid;
  const int64_t n = 32 * s + (l & 31);
  const bool nin = n < a.N;
  const int64_t nc = nin ? n : a.N - 1;
  float sum = 0.f;
  for (int64_t t = w; t < a.T; t += 4) {
    const int64_t k0 = 16 * t + 8 * (l >> 5);
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = k0 + j;
      x[j] = nin && k < a.K ? a.B[k * a.b_sk + nc * a.b_sn] : 0.f;
    }
    bf16x8_t h, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bf16_t hj, lj;
      split_bf16(x[j], hj, lj);
      h[j] = hj;
      lo[j] = lj;
      sum += x[j];
    }
    bf16_t* dst = a.out + ((s * a.T + t) * 2) * 512 + l * 8;
    *(bf16x8_t*)dst = h;
    *(bf16x8_t*)(dst + 512) = lo;
  }
  red[w][l] = sum;
  __syncthreads();
  if (threadIdx.x < 32 && nin) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) t += red[q][threadIdx.x] + red[q][threadIdx.x + 32];
    acc[n] += alpha * t;
  }
}

__global__ void __launch_bounds__(256) pack_x3_pair_sum_kernel(PackSrc a, PackSrc b, int64_t nb0,
                                                               float* __restrict__ acc, float alpha) {
  __shared__ float red[4][64];
  pack_pair_sum_block(a, b, nb0, acc, alpha, blockIdx.x, red);
}

// Two products' operands in one launch (two SGD weight updates): blocks
// [0, n0) are the first product's pack_x3_pair_sum_kernel, the rest the
// second's.
__global__ void __launch_bounds__(256) pack_x3_2pair_sum_kernel(PackSrc a0, PackSrc b0, int64_t nb0, int64_t n0,
                                                                float* __restrict__ acc0, PackSrc a1, PackSrc b1,
                                                                int64_t nb1, float* __restrict__ acc1, float alpha) {
  __shared__ float red[4][64];
  if ((int64_t)blockIdx.x < n0) pack_pair_sum_block(a0, b0, nb0, acc0, alpha, blockIdx.x, red);
  else pack_pair_sum_block(a1, b1, nb1, acc1, alpha, (int64_t)blockIdx.x - n0, red);
}

template <int FR, int FC, int WR, int WC, int KT, bool APK>
__global__ void __launch_bounds__(256) gemm_x3p(GArgs p, int64_t T) {
  static_assert(WR * WC == 4, "four wavefronts per block");
  constexpr int BM = 32 * FR * WR, BN = 32 * FC * WC, KB = 16 * KT;
  constexpr int LDA = KB + 8;             // bf16 row pitch: 16-byte operand reads without bank conflicts
  constexpr int F4R = KB / 4;             // float4 per A row
  constexpr int NQ = BM * F4R / 256;      // float4 per thread
  static_assert(BM * F4R % 256 == 0, "A tile split over 256 threads");
  __shared__ __attribute__((aligned(16))) bf16_t sA[2][APK ? 8 : BM * LDA];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave / WC, wc = wave % WC;
  const int tn = (int)(blockIdx.x % p.tiles_n), tm = (int)(blockIdx.x / p.tiles_n);
  const int split = blockIdx.y;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t t0 = (int64_t)split * KT;
  const int64_t S = (p.N + 31) / 32;

  // 1. This wave's B fragments for all KT k steps (strips past N read the
  //    last strip: legal addresses, outputs never stored).
  bf16x8_t bh[FC][KT], bl[FC][KT];
  const bf16_t* Bp = (const bf16_t*)p.B;
#pragma unroll
  for (int j = 0; j < FC; ++j) {
    int64_t s = (n0 >> 5) + wc * FC + j;
    s = s < S ? s : S - 1;
    const bf16_t* src = Bp + ((s * T + t0) * 2) * 512 + lane * 8;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      bh[j][t] = *(const bf16x8_t*)(src + t * 1024);
      bl[j][t] = *(const bf16x8_t*)(src + t * 1024 + 512);
    }
  }
  // 2. A.  Packed (APK): this wave's fragments of its FR row strips, like
  //    B's (strips past M read the last strip; never stored).  fp32: the
  //    block's BM x KB tile (rows past M read row M - 1), split into hi/lo
  //    in LDS, [row][k] with k contiguous.
  [[maybe_unused]] bf16x8_t ah_r[APK ? FR : 1][APK ? KT : 1], al_r[APK ? FR : 1][APK ? KT : 1];
  if constexpr (APK) {
    const int64_t Sm = (p.M + 31) / 32;
    const bf16_t* Ap = (const bf16_t*)p.A;
#pragma unroll
    for (int i = 0; i < FR; ++i) {
      int64_t s = (m0 >> 5) + wr * FR + i;
      s = s < Sm ? s : Sm - 1;
      const bf16_t* src = Ap + ((s * T + t0) * 2) * 512 + lane * 8;
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        ah_r[i][t] = *(const bf16x8_t*)(src + t * 1024);
        al_r[i][t] = *(const bf16x8_t*)(src + t * 1024 + 512);
      }
    }
  } else {
    const float* A = (const float*)p.A;
    const int64_t kbeg = t0 * 16;
    float4 av[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int r = q / F4R, c4 = q % F4R;
      const int64_t row = m0 + r < p.M ? m0 + r : p.M - 1;
      av[i] = *(const float4*)(A + row * p.a_sm + kbeg + 4 * c4);
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int q = threadIdx.x + 256 * i;
      const int r = q / F4R, c4 = q % F4R;
      bf16x2_t h0, l0, h1, l1;
      split_bf16x2(av[i].x, av[i].y, h0, l0);
      split_bf16x2(av[i].z, av[i].w, h1, l1);
      typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
      const bf16x4_t hv = {h0.x, h0.y, h1.x, h1.y};
      const bf16x4_t lv = {l0.x, l0.y, l1.x, l1.y};
      *(bf16x4_t*)&sA[0][r * LDA + 4 * c4] = hv;
      *(bf16x4_t*)&sA[1][r * LDA + 4 * c4] = lv;
    }
    __syncthreads();
  }

  // 4. The products.
  f32x16 acc[FR][FC];
#pragma unroll
  for (int i = 0; i < FR; ++i)
#pragma unroll
    for (int j = 0; j < FC; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const int ko = 16 * t + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < FR; ++i) {
      const int r = (wr * FR + i) * 32 + (lane & 31);
      bf16x8_t ah, al;
      if constexpr (APK) {
        ah = ah_r[i][t];
        al = al_r[i][t];
      } else {
        ah = *(const bf16x8_t*)&sA[0][r * LDA + ko];
        al = *(const bf16x8_t*)&sA[1][r * LDA + ko];
      }
#pragma unroll
      for (int j = 0; j < FC; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[j][t], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[j][t], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[j][t], acc[i][j], 0, 0, 0);
      }
    }
  }

  // 5. Output block (i, j): lane l, register r -> row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
  if (p.splits == 1) {
#pragma unroll
    for (int i = 0; i < FR; ++i)
#pragma unroll
      for (int j = 0; j < FC; ++j) {
        const int64_t col = n0 + (wc * FC + j) * 32 + (lane & 31);
        const int64_t cc = col < p.N ? col : p.N - 1;
        const int64_t r0 = m0 + (wr * FR + i) * 32 + 4 * (lane >> 5);
        const float bias = p.bias ? ((const float*)p.bias)[cc] : 0.f;
        float res[16], msk[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = r0 + 8 * (r >> 2) + (r & 3);
          const int64_t rc = row < p.M ? row : p.M - 1;
          res[r] = p.res ? ((const float*)p.res)[rc * p.r_sm + cc] : 0.f;
          msk[r] = p.mask ? ((const float*)p.mask)[rc * p.k_sm + cc] : 1.f;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = r0 + 8 * (r >> 2) + (r & 3);
          float v = p.alpha * acc[i][j][r] + bias;
          if (p.act == kActRelu) v = fmaxf(v, 0.f);
          else if (p.act == kActGelu) v = gelu_tanh(v);
          else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
          v += res[r];
          if (p.mask) v = msk[r] > 0.f ? v : 0.f;
          if (row < p.M && col < p.N) ((float*)p.C)[row * p.c_sm + col] = v;
        }
      }
    return;
  }
  // Split K: the partial tile, for the split-K reduction to sum in split order.
  float* ws = p.ws + (int64_t)split * p.M * p.N;
#pragma unroll
  for (int i = 0; i < FR; ++i)
#pragma unroll
    for (int j = 0; j < FC; ++j) {
      const int64_t col = n0 + (wc * FC + j) * 32 + (lane & 31);
      const int64_t r0 = m0 + (wr * FR + i) * 32 + 4 * (lane >> 5);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = r0 + 8 * (r >> 2) + (r & 3);
        if (row < p.M && col < p.N) ws[row * p.N + col] = acc[i][j][r];
      }
    }
}

// ── the row-major finish of a 32 x 32 row-panel block ────────────────────
// Thread t < 256 owns row t / 8 of the block and columns 4 (t % 8) .. + 3;
// the eight threads of a row are consecutive lanes of one wavefront.

// A row's tile statistics (rs_in) as lane q of the row's eight holds them:
// tiles q, q + 8, ..., at most kRsPerLane (48 tiles: K <= 1536), loaded
// together.
constexpr int kRsPerLane = 6;
struct RowStats {
  float2 v[kRsPerLane];
};
// Tiles past the end read the row's last tile (not merged): a load under a
// per-lane condition would be waited for on its own.  Call with rs_in set.
__device__ __forceinline__ void row_norm_load(const GArgs& p, int64_t row, int q, RowStats& rs) {
  const float* st = p.rs_in + row * (int64_t)p.rs_tiles * 2;
#pragma unroll
  for (int i = 0; i < kRsPerLane; ++i) {
    const int j = q + 8 * i < p.rs_tiles ? q + 8 * i : p.rs_tiles - 1;
    rs.v[i] = *(const float2*)(st + 2 * j);
  }
}

// mean and 1 / sqrt(var + eps) of the row from its tile statistics (each
// tile 32 values: sum s_t, squared deviations D_t from its mean): mean =
// sum of s_t / n, then var = sum over tiles of (D_t + 32 (s_t / 32 - mean)^2)
// / n (Chan, Golub and LeVeque's combination of partial variances, through
// the overall mean).  Each lane adds its tiles in order and the eight lanes
// combine by an xor butterfly, which gives all eight the same bits.
// Population variance, as layer_norm's.
__device__ __forceinline__ void row_norm_stats(const GArgs& p, int q, const RowStats& rs, float& mean, float& inv) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kRsPerLane; ++i)
    if (q + 8 * i < p.rs_tiles) s += rs.v[i].x;
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  const float rn = 1.f / (float)p.rs_n;
  mean = s * rn;
  float m2 = 0.f;
#pragma unroll
  for (int i = 0; i < kRsPerLane; ++i) {
    const float d = rs.v[i].x * (1.f / 32.f) - mean;
    if (q + 8 * i < p.rs_tiles) m2 += rs.v[i].y + 32.f * d * d;
  }
  m2 += __shfl_xor(m2, 1, 64);
  m2 += __shfl_xor(m2, 2, 64);
  m2 += __shfl_xor(m2, 4, 64);
  inv = 1.f / sqrtf(m2 * rn + p.rs_eps);
}

struct RowEpi {
  float bias[4], res[4], msk[4], cs[4];
};

// Epilogue operands of the thread's four outputs (row clamped to M - 1 and
// columns to N - 1: legal addresses; such outputs are not stored).  Absent
// operands (uniform tests) are not loaded.
__device__ __forceinline__ void row_epi_load(const GArgs& p, int64_t row, int64_t col, RowEpi& e) {
  const int64_t rc = row < p.M ? row : p.M - 1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t cc = col + j < p.N ? col + j : p.N - 1;
    e.bias[j] = p.bias ? ((const float*)p.bias)[cc] : 0.f;
    e.res[j] = p.res ? ((const float*)p.res)[rc * p.r_sm + cc] : 0.f;
    e.msk[j] = p.mask ? ((const float*)p.mask)[rc * p.k_sm + cc] : 1.f;
    e.cs[j] = p.rs_in ? p.rs_cs[cc] : 0.f;
  }
}

// v (the summed products) -> epilogue -> C, packed rows (c_pk) and this
// block's tile statistics (rs_out: sum and squared deviations from the tile
// mean over the 32 stored values of the row).  The eight threads of the row
// all call it (row < M).
__device__ __forceinline__ void row_epi_store(const GArgs& p, int64_t row, int64_t col, int q, int tn, float (&v)[4],
                                              const RowEpi& e, float mean, float inv) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float y = v[j];
    if (p.rs_in) y = inv * (y - mean * e.cs[j]);
    y = p.alpha * y + e.bias[j];
    if (p.act == kActRelu) y = fmaxf(y, 0.f);
    else if (p.act == kActGelu) y = gelu_tanh(y);
    else if (p.act == kActGeluExact) y = 0.5f * y * (1.f + erff(y * 0.70710678118654752f));
    y += e.res[j];
    if (p.mask) y = e.msk[j] > 0.f ? y : 0.f;
    v[j] = y;
  }
  // Outputs go out with agent-scope stores, which write through the XCD's L2:
  // the next launch reads them from other XCDs, and the kernel's end has
  // fewer dirty lines to write back (GPT-2 forward 0.6228 -> 0.6215 ms).
  if (p.C) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (col + j < p.N)
        __hip_atomic_store((float*)p.C + row * p.c_sm + col + j, v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (p.c_pk && col < p.N) {
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    bf16x2_t h0, l0, h1, l1;
    split_bf16x2(v[0], v[1], h0, l0);
    split_bf16x2(v[2], v[3], h1, l1);
    bf16_t* d = p.c_pk + x3_row_offset(row, col, p.N / 16);
    __hip_atomic_store((uint64_t*)d, __builtin_bit_cast(uint64_t, bf16x4_t{h0.x, h0.y, h1.x, h1.y}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store((uint64_t*)(d + 512), __builtin_bit_cast(uint64_t, bf16x4_t{l0.x, l0.y, l1.x, l1.y}),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (p.rs_out) {
    float sm = (v[0] + v[1]) + (v[2] + v[3]);
    sm += __shfl_xor(sm, 1, 64);
    sm += __shfl_xor(sm, 2, 64);
    sm += __shfl_xor(sm, 4, 64);
    const float mt = sm * (1.f / 32.f);
    float d2 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) d2 += (v[j] - mt) * (v[j] - mt);
    d2 += __shfl_xor(d2, 1, 64);
    d2 += __shfl_xor(d2, 2, 64);
    d2 += __shfl_xor(d2, 4, 64);
    if (q == 0)
      __hip_atomic_store((uint64_t*)(p.rs_out + (row * (int64_t)p.tiles_n + tn) * 2),
                         __builtin_bit_cast(uint64_t, make_float2(sm, d2)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Row panel: one block owns 32 rows x 32 columns over the whole K (K = 64
// KPW), so no split-K reduction launch follows it, and a layer_norm of the A
// rows can run in its prologue (the block holds whole rows).  The four
// wavefronts split the K steps (wave w takes steps [w KPW, (w + 1) KPW)) and
// meet in LDS: each output is the sum of the four partials in wave order,
// then the epilogue.  Every global load is issued first: each wave's B
// fragments, then the block's 32 x K rows of A (thread t holds row t / 8,
// float4 columns t % 8 + 8 i), and, with the layer_norm, gamma and beta
// into LDS.  Blocks of one 32-column strip are dealt to one XCD (their ids
// are equal mod 8) so that the strip's weights come from HBM once per XCD.
// layer_norm: two-pass mean and population variance over the row in fp32,
// y = (x - mean) / sqrt(var + eps) * gamma + beta (crates/core/src/
// kernel_templates.rs:1075-1116), then y is split into hi/lo.
template <int KPW, bool LN>
__global__ void __launch_bounds__(256) gemm_x3_rows(GArgs p) {
  constexpr int K = 64 * KPW, NQ = K / 32, LDA = K + 8;
  __shared__ __attribute__((aligned(16))) bf16_t sA[2][32 * LDA];
  __shared__ __attribute__((aligned(16))) float sGB[LN ? 2 * K : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tm = (int)blockIdx.x / p.tiles_n, tn = (int)blockIdx.x % p.tiles_n;
  const int64_t m0 = (int64_t)tm * 32, n0 = (int64_t)tn * 32;
  const int64_t S = (p.N + 31) / 32;
  constexpr int64_t T = K / 16;

  // 1. B: this wave's KPW fragments of the strip.
  bf16x8_t bh[KPW], bl[KPW];
  {
    const int64_t s = n0 >> 5 < S ? n0 >> 5 : S - 1;
    const bf16_t* src = (const bf16_t*)p.B + ((s * T + (int64_t)wave * KPW) * 2) * 512 + lane * 8;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      bh[i] = *(const bf16x8_t*)(src + i * 1024);
      bl[i] = *(const bf16x8_t*)(src + i * 1024 + 512);
    }
  }
  // 2. A: 32 rows x K (rows past M read row M - 1; never stored).
  const int r = threadIdx.x >> 3, j = threadIdx.x & 7;
  const int64_t row = m0 + r < p.M ? m0 + r : p.M - 1;
  const float* arow = (const float*)p.A + row * p.a_sm;
  float4 av[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) av[i] = *(const float4*)(arow + 4 * (j + 8 * i));
  // the epilogue's operands (thread t finishes row t / 8, columns 4 (t % 8) .. + 3)
  RowEpi ep;
  row_epi_load(p, m0 + r, n0 + 4 * j, ep);
  if constexpr (LN) {
    for (int e = threadIdx.x; e < K; e += 256) {
      sGB[e] = ((const float*)p.ln_g)[e];
      sGB[K + e] = ((const float*)p.ln_b)[e];
    }
  }
  // 3. (layer_norm), hi/lo split, LDS.
  if constexpr (LN) {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) sum += (av[i].x + av[i].y) + (av[i].z + av[i].w);
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    const float mean = sum / (float)K;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const float a = av[i].x - mean, b = av[i].y - mean, c = av[i].z - mean, d = av[i].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
    q += __shfl_xor(q, 1, 64);
    q += __shfl_xor(q, 2, 64);
    q += __shfl_xor(q, 4, 64);
    const float inv = 1.f / sqrtf(q / (float)K + p.ln_eps);
    __syncthreads();  // gamma and beta are in LDS
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int k = 4 * (j + 8 * i);
      const float4 g = *(const float4*)&sGB[k];
      const float4 b = *(const float4*)&sGB[K + k];
      av[i].x = (av[i].x - mean) * inv * g.x + b.x;
      av[i].y = (av[i].y - mean) * inv * g.y + b.y;
      av[i].z = (av[i].z - mean) * inv * g.z + b.z;
      av[i].w = (av[i].w - mean) * inv * g.w + b.w;
    }
  }
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int k = 4 * (j + 8 * i);
    bf16x2_t h0, l0, h1, l1;
    split_bf16x2(av[i].x, av[i].y, h0, l0);
    split_bf16x2(av[i].z, av[i].w, h1, l1);
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    const bf16x4_t hv = {h0.x, h0.y, h1.x, h1.y};
    const bf16x4_t lv = {l0.x, l0.y, l1.x, l1.y};
    *(bf16x4_t*)&sA[0][r * LDA + k] = hv;
    *(bf16x4_t*)&sA[1][r * LDA + k] = lv;
  }
  __syncthreads();

  // 4. This wave's K steps of the 32 x 32 block.
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int ko = 16 * (wave * KPW + i) + 8 * (lane >> 5);
    const bf16x8_t ah = *(const bf16x8_t*)&sA[0][(lane & 31) * LDA + ko];
    const bf16x8_t al = *(const bf16x8_t*)&sA[1][(lane & 31) * LDA + ko];
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[i], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[i], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[i], acc, 0, 0, 0);
  }

  // 5. The four partials meet in LDS (the A tiles are no longer read): row
  //    r, columns 4q..4q+3 are register 4 (r / 8) + r % 4 of lanes
  //    32 ((r / 4) % 2) + 4q + 0..3 in every wave, summed in wave order.
  __syncthreads();
  float* red = (float*)&sA[0][0];
#pragma unroll
  for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[e];
  __syncthreads();
  if (m0 + r >= p.M) return;
  const int e = 4 * (r >> 3) + (r & 3);
  const int lb = 32 * ((r >> 2) & 1) + 4 * j;
  float v[4];
  {
    const float4 w0 = *(const float4*)&red[e * 64 + lb];
    v[0] = w0.x; v[1] = w0.y; v[2] = w0.z; v[3] = w0.w;
  }
#pragma unroll
  for (int x = 1; x < 4; ++x) {
    const float4 w = *(const float4*)&red[(x * 16 + e) * 64 + lb];
    v[0] += w.x; v[1] += w.y; v[2] += w.z; v[3] += w.w;
  }
  row_epi_store(p, m0 + r, n0 + 4 * j, j, tn, v, ep, 0.f, 1.f);
}

// Row panel over packed A: the block (8 wavefronts) owns 32 rows x 32
// columns over a K range of 8 KPW k steps (block id = split x tiles + tile;
// the whole K when splits == 1); wave w multiplies k steps [w KPW, (w + 1) KPW) of the range
// with its A and B fragments loaded straight from global memory into
// registers (both operands are stored in MFMA order), so the product needs
// no LDS, no barrier and no conversion.  The eight partial 32 x 32 blocks
// meet in LDS; threads 0..255 then finish row t / 8, columns 4 (t % 8) .. + 3,
// adding the partials in wave order (fixed: repeated launches give identical
// bits).  Without a split they apply the epilogue, whose operands they load
// while the products run, and write C (fp32) and/or, as packed x3 rows,
// c_pk (N % 16 == 0) for the next packed-A GEMM; with one, the split's sums
// go to the workspace, and either a split-K reduction launch follows
// (tile_cnt null) or the tile is finished in this launch by whichever of its
// splits arrives last (tile_cnt: one counter per tile).  Then every split
// writes its sums with agent-scope (L2-bypassing) stores, waits until they
// have completed and counts itself in with an atomic add on the tile's
// counter; the block that brings the count to `splits` resets the counter
// for the next launch, reads the other splits' sums with agent-scope loads,
// adds all of them in split order (0 + s0 + s1 + ..., the reduction
// launch's order, so the bits are the same) and runs the epilogue.  No
// block waits for another (a split-owner that waited for its tile's other
// splits measured 20 us slower per GPT-2 forward: the polls add latency).
// Blocks past tiles x splits read ahead the next GEMMs' weights
// (prefetch_block).  Tile ids run along the columns (tm = tile / tiles_n):
// with cold weights this measured faster than dealing the row tiles of one
// column strip to one XCD back to back (qkv's weight loads 8.7 vs 10.5 us),
// whose simultaneous misses on the same lines are not merged.  Up to 6 k
// steps per wave the kernel is held to 128 VGPRs (the epilogue operands are
// loaded after the products), so two blocks share a CU and a 288- or
// 384-block grid runs in one round (GPT-2 forward 0.6305 -> 0.6215 ms
// against 144 VGPRs, one block per CU).
template <int KPW>
__global__ void __launch_bounds__(512, KPW <= 6 ? 2 : 1) gemm_x3_rows_pk(GArgs p) {
  constexpr int W = 8;
  if (prefetch_block(p.pf)) return;
  const int64_t T = p.K >> 4;
  __shared__ __attribute__((aligned(16))) float red[W * 16 * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tiles = p.tiles_m * p.tiles_n;
  const int tile = (int)blockIdx.x % tiles, split = (int)blockIdx.x / tiles;
  const int tm = tile / p.tiles_n, tn = tile % p.tiles_n;
  const int64_t m0 = (int64_t)tm * 32, n0 = (int64_t)tn * 32;
  const int64_t t0 = (int64_t)split * (W * KPW) + (int64_t)wave * KPW;

  // 1. Fragments: tiles_m and tiles_n equal the strip counts, so tm and tn
  //    name existing strips.
  bf16x8_t ah[KPW], al[KPW], bh[KPW], bl[KPW];
  {
    const bf16_t* as = (const bf16_t*)p.A + (((int64_t)tm * T + t0) * 2) * 512 + lane * 8;
    const bf16_t* bs = (const bf16_t*)p.B + (((int64_t)tn * T + t0) * 2) * 512 + lane * 8;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      bh[i] = *(const bf16x8_t*)(bs + i * 1024);
      bl[i] = *(const bf16x8_t*)(bs + i * 1024 + 512);
      ah[i] = *(const bf16x8_t*)(as + i * 1024);
      al[i] = *(const bf16x8_t*)(as + i * 1024 + 512);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every fragment load goes out before the first product
  // 2. This wave's k steps.
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[i], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[i], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[i], acc, 0, 0, 0);
  }
  // 3. Epilogue operands of this thread's four outputs (waves 0..3), and
  //    with a folded layer_norm the statistics of its row of A, loaded once
  //    the fragments' registers are free (their latency then overlaps the
  //    partial tiles' meeting in LDS), so that two blocks fit on a CU.
  const int r = (threadIdx.x >> 3) & 31, q = threadIdx.x & 7;
  const int64_t row = m0 + r, rc = row < p.M ? row : p.M - 1;
  RowEpi ep;
  RowStats rs;
  if (wave < 4 && (p.splits == 1 || p.tile_cnt)) {
    row_epi_load(p, row, n0 + 4 * q, ep);
    if (p.rs_in) row_norm_load(p, rc, q, rs);
  }
  // 4. Partials to LDS: register e of lane l is row 8 (e / 4) + 4 (l / 32) +
  //    e % 4, column l % 32.
#pragma unroll
  for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[e];
  __syncthreads();
  const bool fin = wave < 4 && row < p.M;  // this thread finishes row r, columns 4q..4q+3
  if (!fin && !(p.splits > 1 && p.tile_cnt)) return;
  // 5. Row r, columns 4q..4q+3: register 4 (r / 8) + r % 4 of lanes
  //    32 ((r / 4) % 2) + 4q + 0..3 in every wave.
  const int e = 4 * (r >> 3) + (r & 3);
  const int lb = 32 * ((r >> 2) & 1) + 4 * q;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (fin) {
    const float4 w0 = *(const float4*)&red[e * 64 + lb];
    v[0] = w0.x; v[1] = w0.y; v[2] = w0.z; v[3] = w0.w;
#pragma unroll
    for (int x = 1; x < W; ++x) {
      const float4 w = *(const float4*)&red[(x * 16 + e) * 64 + lb];
      v[0] += w.x; v[1] += w.y; v[2] += w.z; v[3] += w.w;
    }
  }
  const int64_t col = n0 + 4 * q;
  if (p.splits > 1) {
    const int64_t plane = p.M * p.N;
    float* ws = p.ws + (int64_t)split * plane + row * p.N;
    if (!p.tile_cnt) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (col + j < p.N) ws[col + j] = v[j];
      return;
    }
    // the tile is finished by whichever split arrives last: sums out, wait
    // until they have completed, count in (all 512 threads reach both
    // barriers)
    if (fin) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (col + j < p.N) __hip_atomic_store(ws + col + j, v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __shared__ unsigned last;
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned before =
          __hip_atomic_fetch_add(p.tile_cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = before == (unsigned)(p.splits - 1);
      if (last) __hip_atomic_store(p.tile_cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last || !fin) return;
    float sum[4] = {0.f, 0.f, 0.f, 0.f};
    const float* wr = p.ws + row * p.N;
    for (int sp = 0; sp < p.splits; ++sp) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t cj = col + j < p.N ? col + j : p.N - 1;
        sum[j] += sp == split ? v[j]
                              : __hip_atomic_load(wr + sp * plane + cj, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = sum[j];
  }
  float mean = 0.f, inv = 1.f;
  if (p.rs_in) row_norm_stats(p, q, rs, mean, inv);
  row_epi_store(p, row, col, q, tn, v, ep, mean, inv);
}

// Tile statistics of an fp32 matrix [M, N] (N % 32 == 0): per row and
// 32-column tile, the sum and the sum of squared deviations from the tile
// mean, formed in row_epi_store's order (four-column groups, then the
// pairwise tree over the eight groups), so that they equal the statistics a
// row-panel GEMM writes for the same values.  One thread per (row, tile).
__global__ void __launch_bounds__(256) row_tile_stats_kernel(const float* __restrict__ x, int64_t sm, int64_t M,
                                                             int64_t tiles, float* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= M * tiles) return;
  const int64_t row = gid / tiles, t = gid % tiles;
  const float* src = x + row * sm + t * 32;
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 a = *(const float4*)(src + 4 * i);
    v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
  }
  float g[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) g[i] = (v[4 * i] + v[4 * i + 1]) + (v[4 * i + 2] + v[4 * i + 3]);
  const float sm_ = ((g[0] + g[1]) + (g[2] + g[3])) + ((g[4] + g[5]) + (g[6] + g[7]));
  const float mt = sm_ * (1.f / 32.f);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) d += (v[4 * i + j] - mt) * (v[4 * i + j] - mt);
    g[i] = d;
  }
  const float d2 = ((g[0] + g[1]) + (g[2] + g[3])) + ((g[4] + g[5]) + (g[6] + g[7]));
  *(float2*)(out + gid * 2) = make_float2(sm_, d2);
}

// Vocabulary head, one column strip per wavefront: 128 rows of packed A times
// many 32-column weight strips (GPT-2's head: 128 x 768 x 50257, 1571
// strips).  The grid has one 8-wavefront block per CU (256 per row tile);
// block b owns the strips [b Sn / G, (b + 1) Sn / G) (6 or 7 for the head),
// so every CU streams the same share of the weights, and wavefront w takes
// strip w of the block's range, loading its weight fragments straight into
// registers P k steps ahead: no LDS and no barrier on the weight stream.  The
// 128 rows of A (393 KB for the head, more than LDS holds) go through LDS in
// phases of P k steps (64 KB, two buffers): the next phase is loaded into
// registers while the current one is read, and written to LDS at the phase's
// end, one barrier per phase.  Each k step a wavefront reads the 8 A
// fragments of its 4 row strips from LDS and runs 12 MFMAs, per element in
// the row panels' order (lo.hi, hi.lo, hi.hi, k ascending).  Wavefronts past
// the block's range only load A and meet the barriers.
// Measured on MI355X in the GPT-2 forward (alternating runs on one box):
// 0.5926 -> 0.5841 ms against 128 x 128 blocks sharing their weight
// fragments through LDS (393 blocks, so 137 CUs ran two and set the time;
// that kernel took 35 us at 256 blocks and 54 us at 393).  Pinning each
// step's weight loads in place with scheduling barriers made it slower
// (0.593 ms).
template <int P, bool TAIL>
__global__ void __launch_bounds__(512) gemm_x3_head(GArgs p, int64_t G) {
  constexpr int PHASE = 4 * P * 1024;        // bf16 elements of A per phase: 4 strips x P steps x hi, lo
  constexpr int PER = PHASE / (8 * 512);     // 16-byte pieces per thread per phase
  __shared__ __attribute__((aligned(16))) bf16_t sA[2 * PHASE];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t T = p.K >> 4;
  const int nph = (int)((T + P - 1) / P);
  const int64_t Sm = (p.M + 31) / 32, Sn = (p.N + 31) / 32;
  const int64_t tm = blockIdx.y;
  const int64_t s0 = (int64_t)blockIdx.x * Sn / G, s1 = ((int64_t)blockIdx.x + 1) * Sn / G;
  const bf16_t* A = (const bf16_t*)p.A;
  const bf16_t* B = (const bf16_t*)p.B;
  // piece q = tid + 512 r of a phase lands at q * 8 in the phase buffer, so
  // fragment (strip i, step t, part h) is the 1 KB at ((i P + t) 2 + h) 512:
  // piece r of this thread is strip r / 2, step tid / 128 + 4 (r % 2), part
  // (tid / 64) % 2, lane tid % 64
  static_assert(P == 8 && PER == 8, "piece mapping assumes 8 steps per phase");
  const int t0 = threadIdx.x >> 7;
  int64_t abase[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t sa = tm * 4 + i < Sm ? tm * 4 + i : Sm - 1;
    abase[i] = (sa * T * 2 + ((threadIdx.x >> 6) & 1)) * 512 + lane * 8;
  }
  bf16x8_t ast[PER];
#define AGPU_HEAD_ISSUE_A(ph)                                                              \
  _Pragma("unroll") for (int r = 0; r < PER; ++r) {                                        \
    const int64_t kk_ = (int64_t)(ph) * P + t0 + 4 * (r & 1);                              \
    ast[r] = *(const bf16x8_t*)(A + abase[r >> 1] + (kk_ < T ? kk_ : T - 1) * 1024);       \
  }
  // (with TAIL, steps past K are written as zeros)
#define AGPU_HEAD_WRITE_A(ph)                                                              \
  _Pragma("unroll") for (int r = 0; r < PER; ++r) {                                        \
    bf16x8_t v_ = ast[r];                                                                  \
    if (TAIL && (int64_t)(ph) * P + t0 + 4 * (r & 1) >= T) v_ = bf16x8_t{};                \
    ((bf16x8_t*)(sA + ((ph) & 1) * PHASE))[threadIdx.x + 512 * r] = v_;                    \
  }
  // (at most 8 strips per block: the launch sizes the grid for that)
  const int64_t want = s0 + w;
  const bool mine = want < s1;
  const int64_t s = mine ? want : s0;
  const bf16_t* Bs = B + s * T * 1024 + lane * 8;
  bf16x8_t bh[P], bl[P];
  if (mine) {
#pragma unroll
    for (int t = 0; t < P; ++t) {
      const int64_t kk = t < T ? t : T - 1;
      bh[t] = *(const bf16x8_t*)(Bs + kk * 1024);
      bl[t] = *(const bf16x8_t*)(Bs + kk * 1024 + 512);
    }
  }
  AGPU_HEAD_ISSUE_A(0)
  AGPU_HEAD_WRITE_A(0)
  __syncthreads();
  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  // Every phase loads the next one (the one past the end re-reads the last
  // step and lands in the buffer no phase reads): no branch in the loop, so
  // the LDS reads of a step issue together ahead of its MFMAs.  With TAIL
  // (K not a multiple of 16 P), steps past K multiply zeros: their A pieces
  // are written as zeros and their weight fragments replaced by zeros.
  for (int ph = 0; ph < nph; ++ph) {
    AGPU_HEAD_ISSUE_A(ph + 1)
    const bf16_t* a = sA + (ph & 1) * PHASE + lane * 8;
    if (mine) {
#pragma unroll
      for (int t = 0; t < P; ++t) {
        const int64_t kk = (int64_t)ph * P + t;
        bf16x8_t ah[4], al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ah[i] = *(const bf16x8_t*)(a + ((i * P + t) * 2) * 512);
          al[i] = *(const bf16x8_t*)(a + ((i * P + t) * 2 + 1) * 512);
        }
        bf16x8_t bhv = bh[t], blv = bl[t];
        if (TAIL && kk >= T) {
          bhv = bf16x8_t{};
          blv = bf16x8_t{};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bhv, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], blv, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bhv, acc[i], 0, 0, 0);
        }
        // step kk + P into the registers just used (past the end: the last
        // step again, never used)
        const int64_t nx = kk + P < T ? kk + P : T - 1;
        bh[t] = *(const bf16x8_t*)(Bs + nx * 1024);
        bl[t] = *(const bf16x8_t*)(Bs + nx * 1024 + 512);
      }
    }
    AGPU_HEAD_WRITE_A(ph + 1)
    __syncthreads();
  }
  if (!mine) return;
  // acc[i], lane l, register r -> row (4 tm + i) 32 + 8 (r / 4) + 4 (l / 32) + r % 4, column 32 s + l % 32
  const int64_t col = s * 32 + (lane & 31);
  const int64_t cc = col < p.N ? col : p.N - 1;
  const float bias = p.bias ? ((const float*)p.bias)[cc] : 0.f;
  const bool cok = col < p.N;
  float* C = (float*)p.C;
  if (p.act == kActNone && !p.res && !p.mask) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = (tm * 4 + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (cok && row < p.M) C[row * p.c_sm + col] = p.alpha * acc[i][r] + bias;
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = (tm * 4 + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (!cok || row >= p.M) continue;
      float v = p.alpha * acc[i][r] + bias;
      if (p.act == kActRelu) v = fmaxf(v, 0.f);
      else if (p.act == kActGelu) v = gelu_tanh(v);
      else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
      if (p.res) v += ((const float*)p.res)[row * p.r_sm + col];
      if (p.mask) v = ((const float*)p.mask)[row * p.k_sm + col] > 0.f ? v : 0.f;
      C[row * p.c_sm + col] = v;
    }
}

#undef AGPU_HEAD_ISSUE_A
#undef AGPU_HEAD_WRITE_A

template <int FR, int FC, int WR, int WC, bool APK>
void launch_x3p_kt(const GArgs& p, int kt, int64_t T, dim3 grid, hipStream_t s) {
  switch (kt) {
    case 1: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 1, APK>), grid, dim3(256), 0, s, p, T); break;
    case 2: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 2, APK>), grid, dim3(256), 0, s, p, T); break;
    case 3: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 3, APK>), grid, dim3(256), 0, s, p, T); break;
    case 4: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 4, APK>), grid, dim3(256), 0, s, p, T); break;
    case 6: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 6, APK>), grid, dim3(256), 0, s, p, T); break;
    case 8: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 8, APK>), grid, dim3(256), 0, s, p, T); break;
    case 12: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 12, APK>), grid, dim3(256), 0, s, p, T); break;
    default: fail("gemm_x3p: %d k steps per block not built", kt);
  }
}

}  // namespace

int64_t packed_x3_elems(int64_t K, int64_t N) { return ((N + 31) / 32) * ((K + 15) / 16) * 2 * 512; }

void pack_weights_x3(const void* b, int64_t b_sk, int64_t b_sn, int64_t K, int64_t N, void* out, hipStream_t s) {
  const int64_t T = (K + 15) / 16, S = (N + 31) / 32;
  const int64_t threads = S * T * 64;
  if (threads == 0) return;
  hipLaunchKernelGGL(pack_x3_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     PackSrc{(const float*)b, b_sk, b_sn, K, N, T, (bf16_t*)out});
  check_launch("pack_weights_x3");
}

namespace {

// Outer-shaped fp32 GEMMs: M and N large, K at most a few hundred (the MLP
// weight gradient g^T h, M = N = 4096, K = 256, with its SGD step W += alpha
// g^T h as the epilogue).  Both operands are split once into packed x3
// fragments in the workspace (pack_x3_kernel: any strides, so g^T is read in
// place).  A block of four wavefronts owns a 128 x 128 output tile over the
// whole K; per k step it needs 16 fragments (4 row strips and 4 column
// strips, hi and lo; 1 KB each, contiguous), which its wavefronts copy
// global -> LDS with global_load_lds_dwordx4 (no registers, no conversion),
// four each, two k steps per stage, two stages in flight; each wavefront then
// reads the 8 fragments of its 64 x 64 quarter from LDS and runs 12 MFMAs per
// k step.  Loading each strip once per block instead of once per wavefront
// halves the L2 -> CU traffic, which bounds this kernel (measured on MI355X,
// M = N = 4096, K = 256 with the SGD epilogue: 54 us per-wavefront, 41 us
// shared; 256 x 128 and 256 x 256 tiles were not faster).  The residual and
// bias are loaded after the products, one 32-row half at a time, and each
// output is written once by the lane whose accumulator holds it.  One k step
// per LDS stage (32 KB) and 120 VGPRs let four blocks share a CU, so the
// 1024-tile MLP update runs in one round: C3 step 0.2537 -> 0.2477 ms against
// two k steps per stage (64 KB) at two blocks per CU.
constexpr int kOuterStage = 16 * 512;  // bf16 elements per LDS stage (one k step)

template <int T>
__device__ __forceinline__ void outer_tile(const GArgs& p, const bf16_t* __restrict__ apk,
                                           const bf16_t* __restrict__ bpk, int64_t bid, bf16_t* lds) {
  constexpr int S = 1;                  // k steps per stage
  constexpr int STAGE = S * 16 * 512;   // bf16 elements per stage
  constexpr int NST = T / S;
  static_assert(T % S == 0 && STAGE == kOuterStage, "whole stages");
  typedef __attribute__((address_space(3))) void* lds_ptr;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t tiles_m = p.M >> 7, tiles_n = p.N >> 7;
  int64_t tm, tn;
  if (tiles_m % 2 == 0 && tiles_n % 4 == 0) {
    // Workgroups go to the 8 XCDs in turn (block b to XCD b % 8): XCD x
    // takes the tiles of row half x / 4 and column quarter x % 4, so that
    // its L2 holds the half of A and the quarter of B it reads.
    const int64_t x = bid & 7, local = bid >> 3;
    const int64_t qn = tiles_n / 4;
    tm = (x >> 2) * (tiles_m / 2) + local / qn;
    tn = (x & 3) * qn + local % qn;
  } else {
    tm = bid / tiles_n;
    tn = bid % tiles_n;
  }
  // Fragment f of a k step (0..15): f < 8 row strip f / 2 of the tile, else
  // column strip (f - 8) / 2; part f % 2 (hi, lo).  Packed strip s, step t,
  // part h: ((s T + t) 2 + h) 512 + 8 l.  Wavefront w copies 4w .. 4w + 3.
  const bf16_t* src[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = 4 * w + q, g = f & 7;
    const bf16_t* base = f < 8 ? apk + (4 * tm + (g >> 1)) * T * 1024 : bpk + (4 * tn + (g >> 1)) * T * 1024;
    src[q] = base + (g & 1) * 512 + lane * 8;
  }
  auto issue = [&](int st) __attribute__((always_inline)) {
    bf16_t* dst = lds + (st & 1) * STAGE;
#pragma unroll
    for (int d = 0; d < S; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_amdgcn_global_load_lds(src[q] + (int64_t)(st * S + d) * 1024,
                                         (lds_ptr)(dst + (d * 16 + 4 * w + q) * 512), 16, 0, 0);
  };
  const int wm = w >> 1, wn = w & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  issue(0);
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    // this wavefront's copies of stage st have landed; after the barrier
    // every wavefront's have, and every wavefront is done with stage st - 1,
    // whose buffer stage st + 1 then overwrites
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (st + 1 < NST) issue(st + 1);
    const bf16_t* b = lds + (st & 1) * STAGE;
#pragma unroll
    for (int d = 0; d < S; ++d) {
      bf16x8_t ah[2], al[2], bh[2], bl[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ah[i] = *(const bf16x8_t*)(b + (d * 16 + (2 * wm + i) * 2) * 512 + lane * 8);
        al[i] = *(const bf16x8_t*)(b + (d * 16 + (2 * wm + i) * 2 + 1) * 512 + lane * 8);
        bh[i] = *(const bf16x8_t*)(b + (d * 16 + 8 + (2 * wn + i) * 2) * 512 + lane * 8);
        bl[i] = *(const bf16x8_t*)(b + (d * 16 + 8 + (2 * wn + i) * 2 + 1) * 512 + lane * 8);
      }
      // small terms first, then hi * hi (the row panels' order)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
        }
    }
  }
  // register e of subtile (i, j): row 32 i + 8 (e / 4) + 4 (lane / 32) + e % 4,
  // column 32 j + lane % 32 of the wavefront's 64 x 64 quarter
  const int64_t rbase = tm * 128 + wm * 64 + 4 * (lane >> 5), cbase = tn * 128 + wn * 64 + (lane & 31);
  float bias[2] = {0.f, 0.f};
  if (p.bias) {
    bias[0] = ((const float*)p.bias)[cbase];
    bias[1] = ((const float*)p.bias)[cbase + 32];
  }
  // one 32-row half of the quarter at a time (half the residual registers)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float res[2][16];
    if (p.res) {
      const float* R = (const float*)p.res;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          res[j][e] = R[(rbase + 32 * i + 8 * (e >> 2) + (e & 3)) * p.r_sm + cbase + 32 * j];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        EpiIn<float> in;
        in.bias = bias[j];
        in.res = p.res ? res[j][e] : 0.f;
        epilogue_finish<float>(p, 0, rbase + 32 * i + 8 * (e >> 2) + (e & 3), cbase + 32 * j, acc[i][j][e], in);
      }
  }
}

template <int T>
__global__ void __launch_bounds__(256, 3) gemm_x3_outer_kernel(GArgs p, const bf16_t* __restrict__ apk,
                                                           const bf16_t* __restrict__ bpk) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2 * kOuterStage];
  outer_tile<T>(p, apk, bpk, blockIdx.x, lds);
}

// Two outer products with the same K in one launch (the two weight updates
// of an MLP's last backward pair): blocks [0, tiles0) are the first
// product's tiles, the rest the second's.  As one grid the 2048 tiles of two
// 4096 x 4096 updates run in two full rounds of four blocks per CU: 75-81 us
// against 92-98 us as two pack + outer launch pairs (measured on MI355X).
template <int T>
__global__ void __launch_bounds__(256, 3) gemm_x3_outer2_kernel(GArgs p0, const bf16_t* __restrict__ apk0,
                                                            const bf16_t* __restrict__ bpk0, int64_t tiles0,
                                                            GArgs p1, const bf16_t* __restrict__ apk1,
                                                            const bf16_t* __restrict__ bpk1) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2 * kOuterStage];
  if ((int64_t)blockIdx.x < tiles0) outer_tile<T>(p0, apk0, bpk0, blockIdx.x, lds);
  else outer_tile<T>(p1, apk1, bpk1, (int64_t)blockIdx.x - tiles0, lds);
}

}  // namespace

bool gemm_x3_outer_ok(const Gemm& g) {
  return g.dt == DType::F32 && g.b_dt == DType::F32 && g.batch == 1 && !g.b_scale && !g.b_x3 && !g.a_x3 &&
         !g.b_packed && !g.ln_gamma && !g.mask && !g.pln_y && !g.pln_ypk && !g.c_pk && !g.no_reduce &&
         g.c_sm == g.N && g.M % 128 == 0 && g.N % 128 == 0 && (g.K == 128 || g.K == 256 || g.K == 512) &&
         (g.M / 128) * (g.N / 128) >= 256;
}

size_t gemm_x3_outer_workspace(const Gemm& g) { return (size_t)(g.M + g.N) * g.K * 4; }

void gemm_x3_outer(const Gemm& g, const GArgs& p, void* ws, hipStream_t s) {
  if (!gemm_x3_outer_ok(g) || !ws) fail("gemm: the outer-product plan does not fit this product");
  bf16_t* apk = (bf16_t*)ws;
  bf16_t* bpk = apk + g.M * g.K * 2;
  // A(m, k) = B'(k, n = m): A's rows packed as the weights' columns; both
  // operands in one launch
  const int64_t T = g.K / 16;
  const PackSrc pa{(const float*)g.A, g.a_sk, g.a_sm, g.K, g.M, T, apk};
  const PackSrc pb{(const float*)g.B, g.b_sk, g.b_sn, g.K, g.N, T, bpk};
  const int64_t nbb = ((g.N / 32) * T * 64 + 255) / 256;
  if (g.a_rowsum_acc) {
    // one block per 32-row strip of A, which also sums the strip's rows
    const int64_t nba = g.M / 32;
    hipLaunchKernelGGL(pack_x3_pair_sum_kernel, dim3((unsigned)(nba + nbb)), dim3(256), 0, s, pa, pb, nba,
                       (float*)g.a_rowsum_acc, g.alpha);
  } else {
    const int64_t nba = ((g.M / 32) * T * 64 + 255) / 256;
    hipLaunchKernelGGL(pack_x3_pair_kernel, dim3((unsigned)(nba + nbb)), dim3(256), 0, s, pa, pb, nba);
  }
  check_launch("pack_x3_pair");
  const int64_t tiles = (g.M / 128) * (g.N / 128);
  const dim3 grid((unsigned)tiles);
  if (g.K == 128) hipLaunchKernelGGL(gemm_x3_outer_kernel<8>, grid, dim3(256), 0, s, p, apk, bpk);
  else if (g.K == 256) hipLaunchKernelGGL(gemm_x3_outer_kernel<16>, grid, dim3(256), 0, s, p, apk, bpk);
  else hipLaunchKernelGGL(gemm_x3_outer_kernel<32>, grid, dim3(256), 0, s, p, apk, bpk);
  check_launch("gemm_x3_outer");
}

bool gemm_x3_outer2_ok(const Gemm& g0, const Gemm& g1) {
  return gemm_x3_outer_ok(g0) && gemm_x3_outer_ok(g1) && g0.K == g1.K && g0.a_rowsum_acc && g1.a_rowsum_acc &&
         g0.alpha == g1.alpha;
}

void gemm_x3_outer2(const Gemm& g0, const GArgs& p0, void* ws0, const Gemm& g1, const GArgs& p1, void* ws1,
                    hipStream_t s) {
  if (!gemm_x3_outer2_ok(g0, g1) || !ws0 || !ws1) fail("gemm: the paired outer-product plan does not fit");
  const int64_t T = g0.K / 16;
  bf16_t* apk0 = (bf16_t*)ws0;
  bf16_t* bpk0 = apk0 + g0.M * g0.K * 2;
  bf16_t* apk1 = (bf16_t*)ws1;
  bf16_t* bpk1 = apk1 + g1.M * g1.K * 2;
  const PackSrc pa0{(const float*)g0.A, g0.a_sk, g0.a_sm, g0.K, g0.M, T, apk0};
  const PackSrc pb0{(const float*)g0.B, g0.b_sk, g0.b_sn, g0.K, g0.N, T, bpk0};
  const PackSrc pa1{(const float*)g1.A, g1.a_sk, g1.a_sm, g1.K, g1.M, T, apk1};
  const PackSrc pb1{(const float*)g1.B, g1.b_sk, g1.b_sn, g1.K, g1.N, T, bpk1};
  const int64_t nba0 = g0.M / 32, nbb0 = ((g0.N / 32) * T * 64 + 255) / 256;
  const int64_t nba1 = g1.M / 32, nbb1 = ((g1.N / 32) * T * 64 + 255) / 256;
  hipLaunchKernelGGL(pack_x3_2pair_sum_kernel, dim3((unsigned)(nba0 + nbb0 + nba1 + nbb1)), dim3(256), 0, s, pa0,
                     pb0, nba0, nba0 + nbb0, (float*)g0.a_rowsum_acc, pa1, pb1, nba1, (float*)g1.a_rowsum_acc,
                     g0.alpha);
  check_launch("pack_x3_2pair");
  const int64_t tiles0 = (g0.M / 128) * (g0.N / 128), tiles1 = (g1.M / 128) * (g1.N / 128);
  const dim3 grid((unsigned)(tiles0 + tiles1));
  if (T == 8) hipLaunchKernelGGL(gemm_x3_outer2_kernel<8>, grid, dim3(256), 0, s, p0, apk0, bpk0, tiles0, p1, apk1, bpk1);
  else if (T == 16) hipLaunchKernelGGL(gemm_x3_outer2_kernel<16>, grid, dim3(256), 0, s, p0, apk0, bpk0, tiles0, p1, apk1, bpk1);
  else hipLaunchKernelGGL(gemm_x3_outer2_kernel<32>, grid, dim3(256), 0, s, p0, apk0, bpk0, tiles0, p1, apk1, bpk1);
  check_launch("gemm_x3_outer2");
}

void row_tile_stats(const float* x, int64_t x_sm, int64_t M, int64_t N, float* out, hipStream_t s) {
  if (N % 32 != 0 || ((uintptr_t)x & 15) || x_sm % 4 != 0) fail("row_tile_stats: N %% 32 == 0 and 16-byte rows needed");
  const int64_t n = M * (N / 32);
  if (n == 0) return;
  hipLaunchKernelGGL(row_tile_stats_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, x_sm, M, N / 32,
                     out);
  check_launch("row_tile_stats");
}

// Arrival counters of the split row-panel tiles finished in the kernel
// (gemm_x3_rows_pk with tile_cnt): zero when the code object loads, and
// every launch leaves the counters it used at zero.  One array per device;
// the runtime drives device 0 only, whose address split_counters_setup
// looks up (the array's name is a host stand-in, never a kernel argument).
constexpr int64_t kTileCounters = 1 << 16;
static __device__ __align__(256) unsigned tile_counters[kTileCounters];
static unsigned* g_tile_counters = nullptr;

bool split_counters_setup(std::string* err) {
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(tile_counters));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    if (err)
      *err = std::string("split-tile counters: hipGetSymbolAddress failed: ") +
             (e != hipSuccess ? hipGetErrorString(e) : "null address");
    return false;
  }
  g_tile_counters = (unsigned*)ptr;
  return true;
}

// The counters for a split row-panel launch of `tiles` output tiles, or null
// when its tiles go to the reduction launch instead.
unsigned* split_tile_counters(int64_t tiles) {
  return gemm_tune().inkernel_splits && g_tile_counters && tiles <= kTileCounters ? g_tile_counters : nullptr;
}

void pack_rows_x3(const void* x, int64_t x_sm, int64_t x_sk, int64_t M, int64_t K, void* out, hipStream_t s) {
  // X(m, k) = B(k, n = m): the weights' kernel with rows as columns
  pack_weights_x3(x, x_sk, x_sm, K, M, out, s);
}

X3Plan x3_plan(int64_t M, int64_t N, int64_t K, int cus, bool apk, bool split) {
  X3Plan pl;
  pl.apk = apk;
  const int64_t T = (K + 15) / 16;
  const int forced = gemm_tune().splits;
  // A forced tile family (applegpu_ffi_gemm_tune's cfg for packed weights):
  // 0 wide split tiles, 1 narrow split tiles, 2 the packed-A row panel.
  const int fcfg = gemm_tune().cfg;
  // Packed A with many columns (each weight strip would be read by several
  // row panels): the vocabulary-head panel, one weight strip per wavefront,
  // whole K.
  if (apk && !split && forced == 0 && (fcfg == -1 || fcfg == 3) && K % 32 == 0 &&
      (fcfg == 3 || (N >= 8192 && ((M + 31) / 32) * ((N + 31) / 32) >= 2048))) {
    pl.stream = true;
    pl.tiles_m = (M + 127) / 128;
    pl.tiles_n = (N + 127) / 128;
    pl.splits = 1;
    return pl;
  }
  // Packed A: the 8-wave row-panel kernel over K ranges of 8 kpw k steps,
  // whole K per block when that fits (no split-K reduction launch), else the
  // deepest range whose grid still gives every CU a block.
  if (apk && T % 8 == 0 && (fcfg == -1 || fcfg == 2)) {
    static const int kKpw[] = {12, 10, 8, 6, 4, 3, 2, 1};
    const int64_t tiles = ((M + 31) / 32) * ((N + 31) / 32);
    int kpw = 0;
    for (int c : kKpw) {
      if (T % (8 * c)) continue;
      const int64_t sp = T / (8 * c);
      if (forced > 0) {
        if (sp == forced) kpw = c;
        continue;
      }
      if (sp > 64 || (split && sp < 2)) continue;
      kpw = c;
      if (sp == 1 || tiles * sp >= (int64_t)cus * 3 / 4) break;
    }
    if (kpw) {
      pl.rows = true;
      pl.kpw = kpw;
      pl.tiles_m = (M + 31) / 32;
      pl.tiles_n = (N + 31) / 32;
      pl.splits = (int)(T / (8 * kpw));
      return pl;
    }
  }
  // fp32 A: whole rows per block when K allows it: no split-K reduction launch.
  const bool rows_k = !apk && K % 64 == 0 && (K / 64 == 4 || K / 64 == 8 || K / 64 == 12 || K / 64 == 16);
  if (forced == 0 && !split && rows_k && (fcfg == -1 || fcfg == 2)) {
    pl.rows = true;
    pl.kpw = (int)(K / 64);
    pl.tiles_m = (M + 31) / 32;
    pl.tiles_n = (N + 31) / 32;
    pl.splits = 1;
    return pl;
  }
  // Wide tiles (128 x 64: each wave 64 rows x 32 columns) for wide outputs;
  // narrow ones (128 x 32: each wave 32 rows, the four waves share their B
  // fragments, and each weight column is read by one block per K range)
  // up to 1024 columns.
  pl.wide = fcfg == 0 || fcfg == 1 ? fcfg == 0 : N > 1024;
  const int64_t bn = pl.wide ? 64 : 32;
  pl.tiles_m = (M + 127) / 128;
  pl.tiles_n = (N + bn - 1) / bn;
  const int64_t tiles = pl.tiles_m * pl.tiles_n;
  // The deepest per-block K range (fewest splits) whose grid still gives
  // nearly every CU a block; failing that, the most splits on offer.
  static const int kKt[] = {12, 8, 6, 4, 3, 2, 1};
  pl.kt = 0;
  // A forced split count (applegpu_ffi_gemm_tune) applies when it leaves a
  // k-step count the kernel is built for.
  if (forced > 0 && T % forced == 0) {
    const int64_t kt = T / forced;
    for (int c : kKt)
      if (c == kt) {
        pl.kt = c;
        pl.splits = forced;
        return pl;
      }
  }
  for (int kt : kKt) {
    if (T % kt) continue;
    if (T / kt > 64) break;  // keep the reduction's split count modest
    pl.kt = kt;
    if (tiles * (T / kt) >= (int64_t)cus * 15 / 16) break;
  }
  if (pl.kt == 0) pl.kt = 1;
  pl.splits = (int)(T / pl.kt);
  return pl;
}

bool gemm_x3_ln_ok(int64_t M, int64_t N, int64_t K) { return x3_plan(M, N, K, 256).rows; }

static void launch_rows_pk(const X3Plan& pl, const GArgs& p0, hipStream_t s) {
  if (p0.K != 128LL * pl.kpw * pl.splits) fail("internal: gemm_x3_rows_pk plan does not cover K");
  GArgs p = p0;
  const int64_t main = pl.tiles_m * pl.tiles_n * pl.splits;
  if (main > 0x7fffff00) fail("gemm_x3_rows_pk: grid too large");
  // blocks beyond the tiles read ahead what the graph walk asked this launch
  // to (none when it asked nothing)
  p.pf = make_prefetch((int)main, 512);
  const dim3 grid((unsigned)(main + p.pf.blocks));
  switch (pl.kpw) {
    case 1: hipLaunchKernelGGL((gemm_x3_rows_pk<1>), grid, dim3(512), 0, s, p); break;
    case 2: hipLaunchKernelGGL((gemm_x3_rows_pk<2>), grid, dim3(512), 0, s, p); break;
    case 3: hipLaunchKernelGGL((gemm_x3_rows_pk<3>), grid, dim3(512), 0, s, p); break;
    case 4: hipLaunchKernelGGL((gemm_x3_rows_pk<4>), grid, dim3(512), 0, s, p); break;
    case 6: hipLaunchKernelGGL((gemm_x3_rows_pk<6>), grid, dim3(512), 0, s, p); break;
    case 8: hipLaunchKernelGGL((gemm_x3_rows_pk<8>), grid, dim3(512), 0, s, p); break;
    case 10: hipLaunchKernelGGL((gemm_x3_rows_pk<10>), grid, dim3(512), 0, s, p); break;
    case 12: hipLaunchKernelGGL((gemm_x3_rows_pk<12>), grid, dim3(512), 0, s, p); break;
    default: fail("gemm_x3_rows_pk: %d k steps per wave not built", pl.kpw);
  }
}

template <bool LN>
static void launch_rows(const X3Plan& pl, const GArgs& p, hipStream_t s) {
  const dim3 grid((unsigned)(pl.tiles_m * pl.tiles_n));
  switch (pl.kpw) {
    case 4: hipLaunchKernelGGL((gemm_x3_rows<4, LN>), grid, dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL((gemm_x3_rows<8, LN>), grid, dim3(256), 0, s, p); break;
    case 12: hipLaunchKernelGGL((gemm_x3_rows<12, LN>), grid, dim3(256), 0, s, p); break;
    case 16: hipLaunchKernelGGL((gemm_x3_rows<16, LN>), grid, dim3(256), 0, s, p); break;
    default: fail("gemm_x3_rows: K = %lld not built", (long long)p.K);
  }
}

void gemm_x3p_launch(const X3Plan& pl, const GArgs& p, hipStream_t s) {
  if (pl.apk != p.a_x3) fail("internal: gemm_x3p plan and A operand disagree");
  const bool panel = pl.rows && pl.splits == 1;
  // the epilogue runs in this launch: unsplit, or packed-A split tiles
  // finished in the kernel
  const bool epi_here = panel || (pl.rows && pl.apk && p.tile_cnt);
  if (p.tile_cnt && !(pl.rows && pl.apk && pl.splits > 1))
    fail("internal: in-kernel split completion needs a split packed-A row-panel plan");
  if (p.c_pk && !(epi_here && p.N % 16 == 0))
    fail("gemm_x3p: packed output needs a row-panel plan that runs its epilogue and N %% 16 == 0");
  if (p.rs_out && !(epi_here && p.N % 32 == 0))
    fail("gemm_x3p: row statistics need a row-panel plan that runs its epilogue and N %% 32 == 0");
  if (p.rs_in && !(panel && pl.apk)) fail("gemm_x3p: a folded layer_norm needs the unsplit packed-A row-panel plan");
  if (pl.stream) {
    if (p.ln_g || !pl.apk) fail("internal: the vocabulary-head panel takes packed A only");
    if (pl.tiles_m > 65535) fail("gemm_x3_head: grid too large");
    // one block per CU, or more blocks when a CU's share passes 8 strips
    const int64_t Sn = (p.N + 31) / 32;
    const int64_t G = std::max((Sn + 7) / 8, std::min<int64_t>(Sn, 256));
    if (G > 0x7fffffff) fail("gemm_x3_head: grid too large");
    const dim3 grid((unsigned)G, (unsigned)pl.tiles_m);
    if ((p.K >> 4) % 8 == 0) hipLaunchKernelGGL((gemm_x3_head<8, false>), grid, dim3(512), 0, s, p, G);
    else hipLaunchKernelGGL((gemm_x3_head<8, true>), grid, dim3(512), 0, s, p, G);
    check_launch("gemm_x3_head");
    return;
  }
  if (pl.rows && pl.apk) {
    if (p.ln_g) fail("gemm_x3p: a layer_norm prologue needs fp32 A");
    launch_rows_pk(pl, p, s);
    check_launch("gemm_x3_rows_pk");
    return;
  }
  if (pl.rows) {
    if (p.ln_g) launch_rows<true>(pl, p, s);
    else launch_rows<false>(pl, p, s);
    check_launch("gemm_x3_rows");
    return;
  }
  if (p.ln_g) fail("gemm_x3p: a layer_norm prologue needs the row-panel plan");
  const int64_t T = (p.K + 15) / 16;
  const dim3 grid((unsigned)(pl.tiles_m * pl.tiles_n), (unsigned)pl.splits);
  if (pl.apk) {
    if (pl.wide) launch_x3p_kt<2, 1, 2, 2, true>(p, pl.kt, T, grid, s);
    else launch_x3p_kt<1, 1, 4, 1, true>(p, pl.kt, T, grid, s);
  } else {
    if (pl.wide) launch_x3p_kt<2, 1, 2, 2, false>(p, pl.kt, T, grid, s);
    else launch_x3p_kt<1, 1, 4, 1, false>(p, pl.kt, T, grid, s);
  }
  check_launch("gemm_x3p");
}

}  // namespace k
}  // namespace agpu
