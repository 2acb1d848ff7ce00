// Skinny GEMM for decode steps: C[M, N] = epilogue(A[M, K] B[K, N]) with
// M <= 16 token rows, 16-bit operands and B contiguous along k (W^T: torch
// Linear weights [N][K], the tied LM head, or GPT-2 Conv1D weights stored
// k-major at load time).
//
// Same arithmetic as the reference's matmul/linear (fp32 accumulate,
// crates/core/src/kernel_templates.rs:987-1072; Linear = x W^T + b,
// backend_cpp/applegpu_backend.cpp:584-620).  At such M the weights are all
// of the traffic, so the kernel is built to have as much of B in flight as
// possible and nothing between the loads and the MFMAs:
//  - one v_mfma_f32_16x16x32 per 16 columns x 32 k: lane l's A operand is
//    row l%16 of A at k + 8*(l/16) .. +8 and its B operand column l%16 of
//    W^T at the same k, each a single 16-byte global load (no LDS staging;
//    rows >= M read row M-1 and columns >= N read column N-1, and those
//    outputs are dropped);
//  - a block of 16 waves owns 16 columns and splits K 16 ways, each wave
//    issuing its next kSkUnroll steps' loads before multiplying;
//  - the 16 partial 16x16 tiles meet in LDS, are summed in wave order
//    (deterministic) and pass through the fused epilogue (alpha, bias,
//    activation, residual) once.
// The k-reduction happens inside the MFMA accumulators, so there is no
// cross-lane reduction, no split-K workspace and no second launch.  (A
// scalar-FMA variant that streamed B and staged A in LDS was slower than the
// 32x32 MFMA tiles at every decode shape: each weight needs M activation
// values, so it was bound by LDS operand traffic.)
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kSkWaves = 16;   // waves per block, splitting K
constexpr int kSkUnroll = 4;   // 32-deep k steps each wave keeps in flight
constexpr int kSkMaxM = 16;

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename E> struct Mfma16;
template <> struct Mfma16<half_t> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma16<bf16_t> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__global__ void __launch_bounds__(64 * kSkWaves) gemm_skinny_mfma(GArgs p) {
  typedef typename Mfma16<T>::vec V8;
  __shared__ float red[kSkWaves][16 * 16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t row = (lane & 15) < p.M ? (lane & 15) : p.M - 1;
  const int64_t col = n0 + (lane & 15) < p.N ? n0 + (lane & 15) : p.N - 1;
  const int kq = 8 * (lane >> 4);  // this lane's k offset inside a step
  const int64_t steps = (p.K + 31) / 32;
  const T* A0 = (const T*)p.A + row * p.a_sm;   // first 8-run of the row: always legal (K >= 8)
  const T* B0 = (const T*)p.B + col * p.b_sn;

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // wave w takes steps w, w + 16, w + 32, ...
  for (int64_t s0 = w; s0 < steps; s0 += (int64_t)kSkWaves * kSkUnroll) {
    V8 a[kSkUnroll], b[kSkUnroll];
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      const int64_t st = s0 + (int64_t)u * kSkWaves;
      // a step past the last, or this lane's 8-run past K (K % 8 == 0, so
      // runs are whole), reads the row's first run and multiplies zeros
      const bool ok = st < steps && st * 32 + kq < p.K;
      const int64_t kc = ok ? st * 32 + kq : 0;
      a[u] = *(const V8*)(A0 + kc);
      b[u] = *(const V8*)(B0 + kc);
      if (!ok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          a[u][e] = T(0);
          b[u][e] = T(0);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) acc = Mfma16<T>::run(a[u], b[u], acc);
  }

  // C layout of a 16x16 MFMA tile: lane l, register r -> row 4*(l/16) + r,
  // column l%16.
#pragma unroll
  for (int r = 0; r < 4; ++r) red[w][(4 * (lane >> 4) + r) * 16 + (lane & 15)] = acc[r];
  __syncthreads();
  if (tid >= 256) return;
  const int m = tid >> 4, c = tid & 15;
  const int64_t n = n0 + c;
  if (m >= p.M || n >= p.N) return;
  float v = 0.f;
#pragma unroll
  for (int ww = 0; ww < kSkWaves; ++ww) v += red[ww][tid];
  epilogue_store<T>(p, 0, m, n, v);
}

bool al16(const void* q) { return ((uintptr_t)q & 15) == 0; }

}  // namespace

SkinnyPlan skinny_plan(const Gemm& g, int cus) {
  (void)cus;
  SkinnyPlan pl{};
  const bool is16 = g.dt == DType::F16 || g.dt == DType::BF16;
  // 16-byte operand runs along k for both A rows and W^T columns
  const bool aligned = al16(g.A) && al16(g.B) && g.a_sk == 1 && g.b_sk == 1 && g.a_sm % 8 == 0 &&
                       g.b_sn % 8 == 0 && g.K % 8 == 0 && g.K >= 8;
  if (!(is16 && g.b_dt == g.dt && !g.b_scale && g.batch == 1 && g.M >= 1 && g.M <= kSkMaxM && aligned &&
        !gemm_tune().no_skinny && gemm_tune().cfg < 0 && gemm_tune().splits == 0))
    return pl;
  const int64_t blocks = (g.N + 15) / 16;
  if (blocks > 0x7fffffffLL) return pl;
  pl.use = true;
  pl.blocks = blocks;
  return pl;
}

void gemm_skinny(const Gemm& g, const SkinnyPlan& pl, const GArgs& p, hipStream_t s) {
  const dim3 grid((unsigned)pl.blocks);
  if (g.dt == DType::F16)
    hipLaunchKernelGGL((gemm_skinny_mfma<half_t>), grid, dim3(64 * kSkWaves), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_skinny_mfma<bf16_t>), grid, dim3(64 * kSkWaves), 0, s, p);
  check_launch("gemm_skinny");
}

}  // namespace k
}  // namespace agpu
