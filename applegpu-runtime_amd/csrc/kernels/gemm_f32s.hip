// fp32 GEMMs with few rows and large fp32 weights (C5's X [64, 8192] times
// the dequantized W [8192, 8192]^T): each weight byte is read once, straight
// into registers, and split there into bf16 hi/lo MFMA fragments.
//
// The tiled kernel (gemm_mf) stages both operands through LDS and converts
// each weight element in the block that loads it; at 64 rows it streamed the
// weights at 3.2-3.7 TB/s in every tile shape and split count tried.  Here a
// block of 8 wavefronts owns 256 output columns over one of KS ranges of K,
// and wavefront w one 32-column strip of them: its lanes load the strip's
// fp32 weights for P k steps ahead (lane l: column l % 32, k 8 (l / 32) ..
// + 7 of each 16-k step, two 16-byte loads), split them and run the
// products against the A fragments of the step.  A (at most 64 rows) is
// split into packed hi/lo fragments by the whole block, P k steps at a time,
// into one of two LDS buffers while the other is read.  Each range's
// partial sums go to the split-K workspace, and the split-K reduction adds
// them in range order and applies the epilogue, so results repeat exactly.
// Products per k step and row strip: lo.hi, hi.lo, hi.hi (fp32 accumulate).
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {

namespace {

constexpr int kF32sP = 8;          // k steps per A phase and per weight read-ahead
constexpr int kF32sCols = 256;     // output columns per block (8 wavefronts x 32)

__device__ __forceinline__ void split8(const float4& a, const float4& b, bf16x8_t& hi, bf16x8_t& lo) {
  bf16x2_t h[4], l[4];
  split_bf16x2(a.x, a.y, h[0], l[0]);
  split_bf16x2(a.z, a.w, h[1], l[1]);
  split_bf16x2(b.x, b.y, h[2], l[2]);
  split_bf16x2(b.z, b.w, h[3], l[3]);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hi[2 * j] = h[j].x;
    hi[2 * j + 1] = h[j].y;
    lo[2 * j] = l[j].x;
    lo[2 * j + 1] = l[j].y;
  }
}

// RS row strips of 32 (M <= 32 RS); grid (N / 256) x KS blocks of 512
// threads; p.k_per_split = K / KS, a multiple of 16 P.
template <int RS>
__global__ void __launch_bounds__(512, 1) gemm_f32_stream_kernel(GArgs p, int KS) {
  constexpr int P = kF32sP;
  constexpr int PHASE = RS * P * 1024;  // bf16 elements of packed A per phase
  static_assert(RS * P * 64 % 512 == 0, "A pieces split over 512 threads");
  constexpr int PER = RS * P * 64 / 512;  // A pieces (8 k of one row) per thread per phase
  __shared__ __attribute__((aligned(16))) bf16_t sA[2 * PHASE];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t grp = blockIdx.x / KS, ks = blockIdx.x % KS;
  const int64_t kbase = ks * p.k_per_split;
  const int T = (int)(p.k_per_split >> 4);
  const int nph = T / P;
  const float* A = (const float*)p.A;
  const float* B = (const float*)p.B;
  // this lane's weights: column n, k offset 8 (lane / 32) within each step
  const int64_t n = grp * kF32sCols + w * 32 + (lane & 31);
  const float* Bn = B + n * p.b_sn + kbase + 8 * (lane >> 5);
  // A piece q = tid + 512 r: row strip i, step t, lane l (row 32 i + l % 32,
  // k 16 t + 8 (l / 32)); its hi and lo halves land at ((i P + t) 2 + h) 512
  // + 8 l of the phase buffer.  Rows past M load row 0 and are zeroed.
  const float* arow[PER];
  int aoff[PER], ast_[PER];
  bool aok[PER];
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int q = threadIdx.x + 512 * r;
    const int l = q & 63, t = (q >> 6) % P, i = q / (64 * P);
    const int64_t row = 32 * i + (l & 31);
    aok[r] = row < p.M;
    arow[r] = A + (aok[r] ? row : 0) * p.a_sm + kbase + 8 * (l >> 5);
    aoff[r] = 16 * t;
    ast_[r] = ((i * P + t) * 2) * 512 + 8 * l;
  }
  float4 araw[PER][2];
#define AGPU_F32S_LOAD_A(ph)                                                                  \
  _Pragma("unroll") for (int r = 0; r < PER; ++r) {                                           \
    const float* s_ = arow[r] + (int64_t)(ph) * (16 * P) + aoff[r];                           \
    araw[r][0] = *(const float4*)s_;                                                          \
    araw[r][1] = *(const float4*)(s_ + 4);                                                    \
  }
#define AGPU_F32S_WRITE_A(ph)                                                                 \
  _Pragma("unroll") for (int r = 0; r < PER; ++r) {                                           \
    bf16x8_t h_, l_;                                                                          \
    split8(araw[r][0], araw[r][1], h_, l_);                                                   \
    if (!aok[r]) { h_ = bf16x8_t{}; l_ = bf16x8_t{}; }                                        \
    bf16_t* d_ = sA + ((ph) & 1) * PHASE + ast_[r];                                           \
    *(bf16x8_t*)d_ = h_;                                                                      \
    *(bf16x8_t*)(d_ + 512) = l_;                                                              \
  }
  // Phases run from a start that depends on the block's column group and K
  // range, so that at any one time the grid's blocks read different k
  // offsets of the weight rows: rows 32 KB apart (C5's 8192-float rows)
  // read at one offset fall into few memory channels.  Measured on MI355X
  // (C5's GEMM, cold weights): 97-98 us with every block starting at its
  // range's first phase, 82-84 us starting at phase ks % nph, 70-78 us at
  // (group + ks) % nph; rotating the steps within a phase as well measured
  // 79-85 us.  (The tiled kernel took 85-89 us with its reduction.)
  const int rot = (int)((grp + ks) % nph);
  auto phys = [&](int ph) __attribute__((always_inline)) { return ph + rot < nph ? ph + rot : ph + rot - nph; };
  float4 braw[P][2];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    braw[t][0] = *(const float4*)(Bn + 16 * (phys(0) * P + t));
    braw[t][1] = *(const float4*)(Bn + 16 * (phys(0) * P + t) + 4);
  }
  AGPU_F32S_LOAD_A(phys(0))
  AGPU_F32S_WRITE_A(0)
  __syncthreads();
  f32x16 acc[RS];
#pragma unroll
  for (int i = 0; i < RS; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  for (int ph = 0; ph < nph; ++ph) {
    // the next phase's A (the one past the end re-reads this one; its
    // buffer is never read)
    const int nx_ph = phys(ph + 1 < nph ? ph + 1 : ph);
    AGPU_F32S_LOAD_A(nx_ph)
    const bf16_t* a = sA + (ph & 1) * PHASE + 8 * lane;
#pragma unroll
    for (int t = 0; t < P; ++t) {
      bf16x8_t bh, bl;
      split8(braw[t][0], braw[t][1], bh, bl);
      // this step's registers take the weights P steps on (past the range's
      // end: this step again, never used)
      const int nt = phys(ph + 1 < nph ? ph + 1 : ph) * P + t;
      braw[t][0] = *(const float4*)(Bn + 16 * nt);
      braw[t][1] = *(const float4*)(Bn + 16 * nt + 4);
#pragma unroll
      for (int i = 0; i < RS; ++i) {
        const bf16x8_t ah = *(const bf16x8_t*)(a + ((i * P + t) * 2) * 512);
        const bf16x8_t al = *(const bf16x8_t*)(a + ((i * P + t) * 2 + 1) * 512);
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc[i], 0, 0, 0);
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc[i], 0, 0, 0);
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc[i], 0, 0, 0);
      }
      // each step's loads stay in their step (without this the scheduler
      // sinks a phase's weight loads below its products)
      __builtin_amdgcn_sched_barrier(0);
    }
    AGPU_F32S_WRITE_A(ph + 1)
    __syncthreads();
  }
#undef AGPU_F32S_LOAD_A
#undef AGPU_F32S_WRITE_A
  // partial sums of this K range: acc[i], lane l, register r -> row
  // 32 i + 8 (r / 4) + 4 (l / 32) + r % 4, column n
  float* ws = p.ws + ks * (p.M * p.N);
#pragma unroll
  for (int i = 0; i < RS; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row < p.M) ws[row * p.N + n] = acc[i][r];
    }
}

// Ranges of K per column group: the most that keep the grid within one
// block per CU (a block's 8 wavefronts take two wavefront slots of every
// SIMD, so a second block per CU would wait), each range a whole number of
// A phases (16 P k); two ranges when the column groups alone fill the CUs.
int f32s_splits(const Gemm& g, int cus) {
  const int64_t groups = g.N / kF32sCols;
  for (int ks : {16, 8, 4, 2})
    if (g.K % (16LL * kF32sP * ks) == 0 && groups * ks <= cus) return ks;
  if (g.K % (32LL * kF32sP) == 0 && groups * 2 <= 2LL * cus) return 2;
  return 0;
}

}  // namespace

bool gemm_f32_stream_ok(const Gemm& g, int cus) {
  const uintptr_t al = 15;
  return g.dt == DType::F32 && g.b_dt == DType::F32 && g.batch == 1 && !g.b_scale && !g.b_x3 && !g.a_x3 &&
         !g.b_packed && !g.ln_gamma && !g.c_pk && !g.pln_y && !g.pln_ypk && !g.no_reduce && !g.a_rowsum_acc &&
         !g.rs_out && !g.rs_in && g.M >= 2 && g.M <= 64 && g.N % kF32sCols == 0 && g.N * g.K >= (8LL << 20) &&
         g.a_sk == 1 && g.a_sm % 4 == 0 && ((uintptr_t)g.A & al) == 0 && g.b_sk == 1 && g.b_sn % 4 == 0 &&
         ((uintptr_t)g.B & al) == 0 && f32s_splits(g, cus) > 0 && g.N * g.K < (1LL << 31) &&
         (size_t)f32s_splits(g, cus) * g.M * g.N * sizeof(float) <= g.max_ws;
}

int gemm_f32_stream_splits(const Gemm& g, int cus) { return gemm_f32_stream_ok(g, cus) ? f32s_splits(g, cus) : 0; }

void gemm_f32_stream(const Gemm& g, const GArgs& p, int cus, hipStream_t s) {
  const int ks = gemm_f32_stream_splits(g, cus);
  // every range must be a whole, nonzero number of phases: the kernel's
  // phase count and rotation assume it
  if (!ks || p.splits != ks || p.k_per_split * ks != g.K || p.k_per_split < 16 * kF32sP ||
      p.k_per_split % (16 * kF32sP) != 0 || !p.ws)
    fail("internal: gemm_f32_stream plan does not match its arguments");
  const dim3 grid((unsigned)(g.N / kF32sCols * ks));
  if (g.M <= 32) hipLaunchKernelGGL((gemm_f32_stream_kernel<1>), grid, dim3(512), 0, s, p, ks);
  else hipLaunchKernelGGL((gemm_f32_stream_kernel<2>), grid, dim3(512), 0, s, p, ks);
  check_launch("gemm_f32_stream");
}

}  // namespace k
}  // namespace agpu
