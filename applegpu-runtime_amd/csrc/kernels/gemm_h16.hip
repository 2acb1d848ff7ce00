// Large fp16 / bf16 GEMMs, both operands contiguous along k: C[M, N] =
// epilogue(A[M, K] B[K, N]) with B given as W [N][K] (torch Linear weights,
// GPT-2's k-major projection weights, the tied LM head) — the C4 prefill
// (M = 8 x 512 tokens).  Same arithmetic as the tiled GEMMs (fp32
// accumulation over k; the reference's matmul/linear,
// crates/core/src/kernel_templates.rs:987-1072).
//
// One block owns a BM x BN tile over the whole K, in stages of 64 k:
//  - Global -> LDS with global_load_lds_dwordx4: each wave instruction
//    copies one 1 KB window of 8 rows x 64 k into LDS with no register
//    staging.  Lane p of the instruction reads row p / 8, 16-byte chunk
//    (p % 8) ^ (row % 8) of the window, so every row's 128 bytes are one
//    contiguous read and the chunks land XOR-swizzled: the MFMA operand
//    reads below (32 rows at one chunk) then hit distinct LDS banks.
//  - NB stages in flight; one barrier per stage.
//  - WM x WN wavefronts, each a (BM / WM) x (BN / WN) block of 32 x 32
//    v_mfma_f32_32x32x16 tiles, with the operands swapped (W as the MFMA's
//    A side) so that each lane's accumulators are 4 consecutive columns of
//    one output row: the epilogue reads bias and residual and writes C 8
//    bytes at a time.
// Measured on MI355X at the C4 prefill shapes (M = 4096): alone, 256 x 256
// tiles with 16 wavefronts run 4096 x 1280 x 3840 at 780-840 TFLOP/s; inside
// the prefill (36 layers back to back, clocks under sustained MFMA load)
// 65 us against 74 us for the register-staged 128 x 128 tiles (gemm_mf).
// Where 256 x 256 tiles leave CUs idle or need a second round (N = 1280 and
// 5120, the 50257-column head), the 256 x 128 and 128 x 128 variants of this
// kernel were slower in the prefill than gemm_mf (fc 131 vs 121 us, proj and
// fc2 82 vs 74 us, head 957 vs ~843 us), so the plan takes it only for grids
// of 256 x 256 tiles that fill one round of the CUs.
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr;

// The LDS copy as a device function: issued from inside a lambda the builtin
// left the kernel without a host-side launch stub.
__device__ __forceinline__ void lds_copy16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr)l, 16, 0, 0);
}

template <typename T> struct Mfma32h;
template <> struct Mfma32h<half_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma32h<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ float h16_act(int act, float v) {
  if (act == kActRelu) return fmaxf(v, 0.f);
  if (act == kActGelu) return gelu_tanh(v);
  if (act == kActGeluExact) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
  return v;
}

template <typename T, int BM, int BN, int NB, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) gemm_h16_kernel(GArgs p) {
  constexpr int NW = WM * WN, WT_M = BM / WM, WT_N = BN / WN, TM = WT_M / 32, TN = WT_N / 32;
  constexpr int AW = BM / 8, BW = BN / 8;  // 1 KB windows per stage
  constexpr int STAGE = (AW + BW) * 512;   // elements
  constexpr int LPW = (AW + BW) / NW;      // window copies per wavefront per stage
  static_assert((AW + BW) % NW == 0 && TM >= 1 && TN >= 1, "tile shape");
  typedef typename Mfma32h<T>::vec V8;
  __shared__ __attribute__((aligned(16))) T lds[NB * STAGE];
  const T* __restrict__ A = (const T*)p.A;
  const T* __restrict__ B = (const T*)p.B;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t tiles_n = (p.N + BN - 1) / BN;
  const int64_t tm = (int64_t)blockIdx.x / tiles_n, tn = (int64_t)blockIdx.x % tiles_n;
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int lr = lane >> 3, lc = (lane & 7) ^ lr;
  const int nk = (int)(p.K / 64);
  // window q of this wavefront: rows of A, then rows of W (rows past M or N
  // repeat the last row; their outputs are not stored)
  auto wsrc = [&](int q) __attribute__((always_inline)) {
    const int win = w * LPW + q;
    if (win < AW) {
      const int64_t r = m0 + win * 8 + lr;
      return A + (r < p.M ? r : p.M - 1) * p.a_sm + lc * 8;
    }
    const int64_t r = n0 + (win - AW) * 8 + lr;
    return B + (r < p.N ? r : p.N - 1) * p.b_sn + lc * 8;
  };
  auto issue = [&](int st) __attribute__((always_inline)) {
    T* dst = lds + (st % NB) * STAGE;
#pragma unroll
    for (int q = 0; q < LPW; ++q) lds_copy16(wsrc(q) + (int64_t)st * 64, dst + (w * LPW + q) * 512);
  };
  // element offset of row r (of the tile), 16-byte chunk c, in a stage
  auto foff = [](int r, int c) { const int rr = r & 7; return (r >> 3) * 512 + (rr * 8 + (c ^ rr)) * 8; };
  const int wm = w / WN, wn = w % WN;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
#pragma unroll
  for (int st = 0; st < NB - 1; ++st)
    if (st < nk) issue(st);
  for (int st = 0; st < nk; ++st) {
    // this wavefront's copies of stage st have landed (the NB - 2 stages
    // issued after it may still be in flight); after the barrier every
    // wavefront's have, and every wavefront is done with stage st - 1,
    // whose buffer the next issue overwrites
    if (NB > 2 && st + NB - 2 < nk) {
      constexpr int n = (NB > 2 ? NB - 2 : 0) * LPW;
      constexpr int imm = (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
      __builtin_amdgcn_s_waitcnt(imm);
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    if (st + NB - 1 < nk) issue(st + NB - 1);
    const T* a = lds + (st % NB) * STAGE;
    const T* b = a + AW * 512;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      V8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *(const V8*)(a + foff(wm * WT_M + 32 * i + (lane & 31), c));
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *(const V8*)(b + foff(wn * WT_N + 32 * j + (lane & 31), c));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32h<T>::run(bf[j], af[i], acc[i][j]);
    }
  }
  // C^T layout of each 32 x 32 tile: lane l, register e -> row l % 32,
  // column 8 (e / 4) + 4 (l / 32) + e % 4
  const T* bias = (const T*)p.bias;
  const T* R = (const T*)p.res;
  T* C = (T*)p.C;
  const bool vec = p.vec_a;  // host: N, ldc, ldr multiples of 4 and 8-byte aligned bases
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = m0 + wm * WT_M + 32 * i + (lane & 31);
    if (row >= p.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = n0 + wn * WT_N + 32 * j + 8 * g + 4 * (lane >> 5);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = p.alpha * acc[i][j][4 * g + e];
        if (vec && col + 3 < p.N) {
          if (bias) {
            T bb[4];
            *(uint2*)bb = *(const uint2*)&bias[col];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += to_f(bb[e]);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = h16_act(p.act, v[e]);
          if (R) {
            T rr[4];
            *(uint2*)rr = *(const uint2*)&R[row * p.r_sm + col];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += to_f(rr[e]);
          }
          T o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = from_f<T>(v[e]);
          *(uint2*)&C[row * p.c_sm + col] = *(const uint2*)o;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e >= p.N) continue;
            float x = v[e] + (bias ? to_f(bias[col + e]) : 0.f);
            x = h16_act(p.act, x);
            if (R) x += to_f(R[row * p.r_sm + col + e]);
            C[row * p.c_sm + col + e] = from_f<T>(x);
          }
        }
      }
  }
}

bool al16(const void* q) { return ((uintptr_t)q & 15) == 0; }
bool al8(const void* q) { return ((uintptr_t)q & 7) == 0; }

// 256 x 256 tiles with 16 wavefronts, for grids of 3/4 to 1 round of the
// CUs (see above).
bool h16_fits(const Gemm& g, int cus) {
  const int64_t t256 = ((g.M + 255) / 256) * ((g.N + 255) / 256);
  return t256 >= (int64_t)cus * 3 / 4 && t256 <= cus;
}

}  // namespace

bool gemm_h16_ok(const Gemm& g, int cus) {
  if (!h16_fits(g, cus)) return false;
  const bool is16 = g.dt == DType::F16 || g.dt == DType::BF16;
  return is16 && g.b_dt == g.dt && g.batch == 1 && !g.b_scale && !g.b_x3 && !g.a_x3 && !g.b_packed &&
         !g.ln_gamma && !g.mask && !g.pln_y && !g.pln_ypk && !g.c_pk && !g.no_reduce && g.M >= 256 && g.N >= 128 &&
         g.K >= 64 && g.K % 64 == 0 && g.a_sk == 1 && g.b_sk == 1 && g.a_sm % 8 == 0 && g.b_sn % 8 == 0 &&
         al16(g.A) && al16(g.B) && g.c_sm == g.N && g.M * g.N >= 1024LL * 1024;
}

void gemm_h16(const Gemm& g, const GArgs& p_in, int cus, hipStream_t s) {
  if (!gemm_h16_ok(g, cus)) fail("gemm: the 16-bit large-tile plan does not fit this product");
  GArgs p = p_in;
  p.vec_a = g.N % 4 == 0 && al8(g.C) && (!g.bias || al8(g.bias)) &&
            (!g.residual || (al8(g.residual) && g.r_sm % 4 == 0));
  const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 255) / 256);
  if (g.dt == DType::F16)
    hipLaunchKernelGGL((gemm_h16_kernel<half_t, 256, 256, 2, 4, 4>), dim3((unsigned)tiles), dim3(1024), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_h16_kernel<bf16_t, 256, 256, 2, 4, 4>), dim3((unsigned)tiles), dim3(1024), 0, s, p);
  check_launch("gemm_h16");
}

}  // namespace k
}  // namespace agpu
