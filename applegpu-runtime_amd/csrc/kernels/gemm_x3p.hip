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

__global__ void __launch_bounds__(256) pack_x3_kernel(const float* __restrict__ B, int64_t b_sk, int64_t b_sn,
                                                      int64_t K, int64_t N, int64_t T, bf16_t* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t S = (N + 31) / 32;
  if (gid >= S * T * 64) return;
  const int l = (int)(gid & 63);
  const int64_t st = gid >> 6;
  const int64_t t = st % T, s = st / T;
  const int64_t n = 32 * s + (l & 31);
  const int64_t k0 = 16 * t + 8 * (l >> 5);
  bf16x8_t h, lo;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t k = k0 + j;
    const float x = (n < N && k < K) ? B[k * b_sk + n * b_sn] : 0.f;
    bf16_t hj, lj;
    split_bf16(x, hj, lj);
    h[j] = hj;
    lo[j] = lj;
  }
  bf16_t* dst = out + (st * 2) * 512 + l * 8;
  *(bf16x8_t*)dst = h;
  *(bf16x8_t*)(dst + 512) = lo;
}

template <int FR, int FC, int WR, int WC, int KT>
__global__ void __launch_bounds__(256) gemm_x3p(GArgs p, int64_t T) {
  static_assert(WR * WC == 4, "four wavefronts per block");
  constexpr int BM = 32 * FR * WR, BN = 32 * FC * WC, KB = 16 * KT;
  constexpr int LDA = KB + 8;             // bf16 row pitch: 16-byte operand reads without bank conflicts
  constexpr int F4R = KB / 4;             // float4 per A row
  constexpr int NQ = BM * F4R / 256;      // float4 per thread
  static_assert(BM * F4R % 256 == 0, "A tile split over 256 threads");
  __shared__ __attribute__((aligned(16))) bf16_t sA[2][BM * LDA];

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
  // 2. The block's A tile, BM rows x KB k (rows past M read row M - 1).
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
  // 3. hi/lo into LDS, [row][k] with k contiguous.
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
      const bf16x8_t ah = *(const bf16x8_t*)&sA[0][r * LDA + ko];
      const bf16x8_t al = *(const bf16x8_t*)&sA[1][r * LDA + ko];
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
  int tm, tn;
  {
    const int id = blockIdx.x;
    if ((p.tiles_n & 7) == 0) {
      const int g = id / (8 * p.tiles_m), r = id % (8 * p.tiles_m);
      tm = r / 8;
      tn = g * 8 + (r & 7);
    } else {
      tm = id / p.tiles_n;
      tn = id % p.tiles_n;
    }
  }
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

  // 5. The four partials meet in LDS (the A tiles are no longer read); wave
  //    w finishes registers 4w..4w+3 of every lane: rows 8w..8w+7.
  __syncthreads();
  float* red = (float*)&sA[0][0];
#pragma unroll
  for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[e];
  __syncthreads();
  const int64_t col = n0 + (lane & 31);
  const int64_t cc = col < p.N ? col : p.N - 1;
  const float bias = p.bias ? ((const float*)p.bias)[cc] : 0.f;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int e = 4 * wave + rr;
    const int64_t orow = m0 + 8 * wave + 4 * (lane >> 5) + rr;
    const int64_t rc = orow < p.M ? orow : p.M - 1;
    const float res = p.res ? ((const float*)p.res)[rc * p.r_sm + cc] : 0.f;
    const float msk = p.mask ? ((const float*)p.mask)[rc * p.k_sm + cc] : 1.f;
    float v = red[(0 * 16 + e) * 64 + lane];
#pragma unroll
    for (int x = 1; x < 4; ++x) v += red[(x * 16 + e) * 64 + lane];
    v = p.alpha * v + bias;
    if (p.act == kActRelu) v = fmaxf(v, 0.f);
    else if (p.act == kActGelu) v = gelu_tanh(v);
    else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    v += res;
    if (p.mask) v = msk > 0.f ? v : 0.f;
    if (orow < p.M && col < p.N) ((float*)p.C)[orow * p.c_sm + col] = v;
  }
}

template <int FR, int FC, int WR, int WC>
void launch_x3p_kt(const GArgs& p, int kt, int64_t T, dim3 grid, hipStream_t s) {
  switch (kt) {
    case 1: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 1>), grid, dim3(256), 0, s, p, T); break;
    case 2: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 2>), grid, dim3(256), 0, s, p, T); break;
    case 3: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 3>), grid, dim3(256), 0, s, p, T); break;
    case 4: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 4>), grid, dim3(256), 0, s, p, T); break;
    case 6: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 6>), grid, dim3(256), 0, s, p, T); break;
    case 8: hipLaunchKernelGGL((gemm_x3p<FR, FC, WR, WC, 8>), grid, dim3(256), 0, s, p, T); break;
    default: fail("gemm_x3p: %d k steps per block not built", kt);
  }
}

}  // namespace

int64_t packed_x3_elems(int64_t K, int64_t N) { return ((N + 31) / 32) * ((K + 15) / 16) * 2 * 512; }

void pack_weights_x3(const void* b, int64_t b_sk, int64_t b_sn, int64_t K, int64_t N, void* out, hipStream_t s) {
  const int64_t T = (K + 15) / 16, S = (N + 31) / 32;
  const int64_t threads = S * T * 64;
  if (threads == 0) return;
  hipLaunchKernelGGL(pack_x3_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, (const float*)b, b_sk,
                     b_sn, K, N, T, (bf16_t*)out);
  check_launch("pack_weights_x3");
}

X3Plan x3_plan(int64_t M, int64_t N, int64_t K, int cus) {
  X3Plan pl;
  const int64_t T = (K + 15) / 16;
  // Whole rows per block when K allows it: no split-K reduction launch.
  if (gemm_tune().splits == 0 && K % 64 == 0 && (K / 64 == 4 || K / 64 == 8 || K / 64 == 12 || K / 64 == 16)) {
    pl.rows = true;
    pl.kpw = (int)(K / 64);
    pl.tiles_m = (M + 31) / 32;
    pl.tiles_n = (N + 31) / 32;
    pl.splits = 1;
    return pl;
  }
  // Wide tiles (128 x 64: each wave 64 rows x 32 columns) when N gives a
  // dozen of them; narrow ones (128 x 32: each wave 32 rows, the four waves
  // share their B fragments) below that.
  pl.wide = N >= 768;
  const int64_t bn = pl.wide ? 64 : 32;
  pl.tiles_m = (M + 127) / 128;
  pl.tiles_n = (N + bn - 1) / bn;
  const int64_t tiles = pl.tiles_m * pl.tiles_n;
  // The deepest per-block K range (fewest splits) whose grid still gives
  // nearly every CU a block; failing that, the most splits on offer.
  static const int kKt[] = {8, 6, 4, 3, 2, 1};
  pl.kt = 0;
  // A forced split count (applegpu_ffi_gemm_tune) applies when it leaves a
  // k-step count the kernel is built for.
  const int forced = gemm_tune().splits;
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
  if (pl.rows) {
    if (p.ln_g) launch_rows<true>(pl, p, s);
    else launch_rows<false>(pl, p, s);
    check_launch("gemm_x3_rows");
    return;
  }
  if (p.ln_g) fail("gemm_x3p: a layer_norm prologue needs the row-panel plan");
  const int64_t T = (p.K + 15) / 16;
  const dim3 grid((unsigned)(pl.tiles_m * pl.tiles_n), (unsigned)pl.splits);
  if (pl.wide) launch_x3p_kt<2, 1, 2, 2>(p, pl.kt, T, grid, s);
  else launch_x3p_kt<1, 1, 4, 1>(p, pl.kt, T, grid, s);
  check_launch("gemm_x3p");
}

}  // namespace k
}  // namespace agpu
