// Skinny GEMM for decode steps: C[M, N] = epilogue(A[M, K] B[K, N]) with
// M <= 16 token rows and 16-bit operands, B contiguous along k (W^T: torch
// Linear weights [N][K], the tied LM head, GPT-2 Conv1D weights stored
// k-major) or pre-packed for this kernel (pack_weights below).
//
// Same arithmetic as the reference's matmul/linear (fp32 accumulate,
// crates/core/src/kernel_templates.rs:987-1072; Linear = x W^T + b,
// backend_cpp/applegpu_backend.cpp:584-620).  At such M the weights are all
// of the traffic, so the kernel keeps as much of B in flight as it can and
// puts nothing between the loads and the MFMAs:
//  - one v_mfma_f32_16x16x32 per 16 columns x 32 k: lane l's B operand is
//    column l%16 at k + 8*(l/16) .. +8 and its A operand row l%16 at the same
//    k (rows >= M use row M-1 and columns >= N column N-1; those outputs are
//    dropped);
//  - a block of 16 waves owns 16 columns and splits the 32-deep k steps 16
//    ways (wave w takes steps w, w+16, ...), each wave issuing its next 4
//    (12 for long K) steps' loads before multiplying;
//  - the 16 partial 16x16 tiles meet in LDS, are summed in wave order
//    (deterministic) and pass through the fused epilogue (alpha, bias,
//    activation, residual) once.
// Memory layout matters more than anything else here (measured on MI355X,
// 80 blocks streaming 13 MB: 9.6 us when each wave instruction reads 16
// columns x 64 bytes of W^T, 5.2 us for contiguous 1 KB runs).  So:
//  - PACKED: B comes in the layout [N/16][K/32][64 lanes][8]: the operands of
//    one wave instruction are 1 KB contiguous; padding is zero;
//  - XLDS: the M rows of A (M*K <= 16384 elements, K <= 2048) are staged in
//    LDS once per block, so A operands come from LDS instead of global
//    memory (an 80 KB variant for the long-K projection measured slower: one
//    block per CU).  With
//    a layer-norm prologue (A = layer_norm(x) over K: the GPT-2 ln_1/ln_2 ->
//    projection pairs) wave w computes mean and 1/std of row w by two passes
//    over the row in registers (the reference's formula,
//    crates/core/src/kernel_templates.rs:1075-1116) and stages the row
//    normalised, g * (x - mean) * rstd + b rounded to the operand type, as
//    the layer_norm kernel would have stored it.
// The staged rows are loaded first and the first steps' B loads right after,
// so the weights are in flight while the staging (and its layer-norm
// statistics) runs.  The k-reduction happens inside the MFMA
// accumulators: no cross-lane reduction, no split-K workspace and no second
// launch.  (A scalar-FMA variant that staged A in LDS and a split-K variant
// that finished in the last block were both slower than the MFMA tiles: the
// first is bound by LDS operand traffic, the second by the device-scope
// fences, which write back and invalidate the XCD's L2.)
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kSkWaves = 16;        // waves per block, splitting K
constexpr int kSkMaxM = 16;
constexpr int kSkXlds = 16384;      // A elements staged in LDS (32 KB)
constexpr int kSkRowMaxK = 2048;    // row a wave holds in registers for the LN statistics

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

// UN: steps in flight per wave; LN: layer-norm the A rows (needs XLDS);
// PACKED: B in the packed layout; XS > 0: A rows staged in LDS (XS elements).
template <typename T, int UN, bool LN, bool PACKED, int XS>
__global__ void __launch_bounds__(64 * kSkWaves) gemm_skinny_mfma(GArgs p) {
  constexpr bool XLDS = XS > 0;
  static_assert(!LN || XLDS, "the layer-norm prologue stages A in LDS");
  typedef typename Mfma16<T>::vec V8;
  __shared__ float red[kSkWaves][16 * 16];
  __shared__ __attribute__((aligned(16))) T xs[XLDS ? XS : 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t row = (lane & 15) < p.M ? (lane & 15) : p.M - 1;
  const int64_t col = n0 + (lane & 15) < p.N ? n0 + (lane & 15) : p.N - 1;
  const int kq = 8 * (lane >> 4);  // this lane's k offset inside a step
  const int64_t steps = (p.K + 31) / 32;
  const T* A0 = (const T*)p.A + row * p.a_sm;   // global A row (!XLDS)
  // B: packed -> this block's run of steps, else column `col` of W^T
  const T* B0 = PACKED ? (const T*)p.B + ((int64_t)blockIdx.x * steps * 64 + lane) * 8 : (const T*)p.B + col * p.b_sn;

  auto load_b = [&](V8 (&b)[UN], int64_t s0) {
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t st = s0 + (int64_t)u * kSkWaves;
      if constexpr (PACKED) {
        b[u] = *(const V8*)(B0 + (st < steps ? st : 0) * 512);
        if (st >= steps) {
#pragma unroll
          for (int e = 0; e < 8; ++e) b[u][e] = T(0);
        }
      } else {
        // a step past the last, or this lane's 8-run past K (K % 8 == 0, so
        // runs are whole), reads the column's first run and multiplies zeros
        const bool ok = st < steps && st * 32 + kq < p.K;
        b[u] = *(const V8*)(B0 + (ok ? st * 32 + kq : 0));
        if (!ok) {
#pragma unroll
          for (int e = 0; e < 8; ++e) b[u][e] = T(0);
        }
      }
    }
  };

  // The staged A row (and gamma, beta) is loaded first, then this wave's
  // first B steps, then the epilogue operands: a wave's loads complete in
  // issue order, so the staging below waits for its row only, while the
  // weight stream is still in flight.
  constexpr int R = kSkRowMaxK / 512;  // 8-runs per lane of a staged row
  V8 run[XLDS ? R : 1], lg[LN ? R : 1], lb[LN ? R : 1];
  if constexpr (XLDS) {
    if (w < p.M) {
      const T* xr = (const T*)p.A + w * p.a_sm;
#pragma unroll
      for (int c = 0; c < R; ++c) {
        const int64_t kk = (int64_t)(lane + 64 * c) * 8;
        if (kk < p.K) {
          run[c] = *(const V8*)(xr + kk);
          if constexpr (LN) {
            lg[c] = *(const V8*)((const T*)p.ln_g + kk);
            lb[c] = *(const V8*)((const T*)p.ln_b + kk);
          }
        }
      }
    }
  }
  V8 b[UN];
  load_b(b, w);  // in flight during the staging below
  // threads 0..255 each finish one output (m, n0 + c): its bias/residual now
  // (every thread loads, from a clamped legal element: no divergent branch
  // around the loads)
  const int om = (tid >> 4) & 15, oc = tid & 15;
  const bool owns = tid < 256 && om < p.M && n0 + oc < p.N;
  const EpiIn<T> ein = epilogue_load<T>(p, 0, om < p.M ? om : p.M - 1, n0 + oc < p.N ? n0 + oc : p.N - 1);

  if constexpr (XLDS) {
    if (w < p.M) {
      if constexpr (LN) {
        float sum = 0.f;
#pragma unroll
        for (int c = 0; c < R; ++c)
          if ((int64_t)(lane + 64 * c) * 8 < p.K) {
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += (float)run[c][e];
          }
        const float mean = wave_sum(sum) / (float)p.K;
        float sq = 0.f;
#pragma unroll
        for (int c = 0; c < R; ++c)
          if ((int64_t)(lane + 64 * c) * 8 < p.K) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float d = (float)run[c][e] - mean;
              sq += d * d;
            }
          }
        const float rs = 1.f / sqrtf(wave_sum(sq) / (float)p.K + p.ln_eps);
#pragma unroll
        for (int c = 0; c < R; ++c) {
          if ((int64_t)(lane + 64 * c) * 8 < p.K) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              run[c][e] = T((float)lg[c][e] * ((float)run[c][e] - mean) * rs + (float)lb[c][e]);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < R; ++c) {
        const int64_t kk = (int64_t)(lane + 64 * c) * 8;
        if (kk < p.K) *(V8*)&xs[w * p.K + kk] = run[c];
      }
    }
    __syncthreads();
  }

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t s0 = w; s0 < steps; s0 += (int64_t)kSkWaves * UN) {
    V8 a[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t st = s0 + (int64_t)u * kSkWaves;
      const bool ok = st < steps && st * 32 + kq < p.K;
      const int64_t kc = ok ? st * 32 + kq : 0;
      if constexpr (XLDS) a[u] = *(const V8*)&xs[row * p.K + kc];
      else a[u] = *(const V8*)(A0 + kc);
      if (!ok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[u][e] = T(0);
      }
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) acc = Mfma16<T>::run(a[u], b[u], acc);
    if (s0 + (int64_t)kSkWaves * UN < steps) load_b(b, s0 + (int64_t)kSkWaves * UN);
  }

  // C layout of a 16x16 MFMA tile: lane l, register r -> row 4*(l/16) + r,
  // column l%16.
#pragma unroll
  for (int r = 0; r < 4; ++r) red[w][(4 * (lane >> 4) + r) * 16 + (lane & 15)] = acc[r];
  __syncthreads();
  if (!owns) return;
  float v = 0.f;
#pragma unroll
  for (int ww = 0; ww < kSkWaves; ++ww) v += red[ww][tid];
  epilogue_finish<T>(p, 0, om, n0 + oc, v, ein);
}

// out[t][s][l][e] = W^T[16t + l%16][32s + 8(l/16) + e], zero outside [N, K).
template <typename T>
__global__ void __launch_bounds__(256) pack_weights_kernel(const T* __restrict__ w, int64_t s_n, int64_t s_k,
                                                           int64_t N, int64_t K, T* __restrict__ out,
                                                           int64_t total) {
  const int64_t steps = (K + 31) / 32;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t e = i & 7, l = (i >> 3) & 63, ts = i >> 9;
    const int64_t s = ts % steps, t = ts / steps;
    const int64_t n = 16 * t + (l & 15), k = 32 * s + 8 * (l >> 4) + e;
    out[i] = (n < N && k < K) ? w[n * s_n + k * s_k] : T(0);
  }
}

bool al16(const void* q) { return ((uintptr_t)q & 15) == 0; }

}  // namespace

int64_t packed_weight_elems(int64_t N, int64_t K) { return ((N + 15) / 16) * ((K + 31) / 32) * 512; }

void pack_weights(DType dt, const void* w, int64_t s_n, int64_t s_k, int64_t N, int64_t K, void* out,
                  hipStream_t s) {
  const int64_t total = packed_weight_elems(N, K);
  if (total == 0) return;
  int64_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  if (dt == DType::F16)
    hipLaunchKernelGGL((pack_weights_kernel<half_t>), dim3((unsigned)g), dim3(256), 0, s, (const half_t*)w, s_n, s_k,
                       N, K, (half_t*)out, total);
  else if (dt == DType::BF16)
    hipLaunchKernelGGL((pack_weights_kernel<bf16_t>), dim3((unsigned)g), dim3(256), 0, s, (const bf16_t*)w, s_n, s_k,
                       N, K, (bf16_t*)out, total);
  else
    fail("pack_weights: fp16 or bf16 weights only");
  check_launch("pack_weights");
}

// A operand requirements shared by the layouts: 16-byte runs along k.
static bool skinny_a_ok(const Gemm& g) {
  const bool is16 = g.dt == DType::F16 || g.dt == DType::BF16;
  return is16 && g.b_dt == g.dt && !g.b_scale && g.batch == 1 && g.M >= 1 && g.M <= kSkMaxM && al16(g.A) &&
         g.a_sk == 1 && (g.M == 1 || g.a_sm % 8 == 0) && g.K % 8 == 0 && g.K >= 8 && !gemm_tune().no_skinny &&
         gemm_tune().cfg < 0 && gemm_tune().splits == 0;
}

// LDS staging of A: 0 = none, else the array size the launch uses.
static int skinny_xlds(const Gemm& g) {
  if (g.M * g.K <= kSkXlds && g.K <= kSkRowMaxK) return kSkXlds;
  return 0;
}

bool gemm_skinny_ln_ok(const Gemm& g) {
  Gemm probe = g;
  probe.ln_gamma = probe.ln_beta = nullptr;
  return skinny_plan(probe, 0).use && skinny_xlds(g) == kSkXlds && g.ln_gamma && g.ln_beta && al16(g.ln_gamma) &&
         al16(g.ln_beta);
}

SkinnyPlan skinny_plan(const Gemm& g, int cus) {
  (void)cus;
  SkinnyPlan pl{};
  if (!skinny_a_ok(g)) return pl;
  if (!g.b_packed && !(al16(g.B) && g.b_sk == 1 && g.b_sn % 8 == 0)) return pl;
  const int64_t blocks = (g.N + 15) / 16;
  if (blocks > 0x7fffffffLL) return pl;
  pl.use = true;
  pl.blocks = blocks;
  return pl;
}

template <typename T, bool PK>
static void launch_skinny(const GArgs& p, dim3 grid, bool deep, bool ln, int xs, hipStream_t s) {
  const dim3 blk(64 * kSkWaves);
  if (ln) hipLaunchKernelGGL((gemm_skinny_mfma<T, 4, true, PK, kSkXlds>), grid, blk, 0, s, p);
  else if (xs) {
    if (deep) hipLaunchKernelGGL((gemm_skinny_mfma<T, 12, false, PK, kSkXlds>), grid, blk, 0, s, p);
    else hipLaunchKernelGGL((gemm_skinny_mfma<T, 4, false, PK, kSkXlds>), grid, blk, 0, s, p);
  } else {
    if (deep) hipLaunchKernelGGL((gemm_skinny_mfma<T, 12, false, PK, 0>), grid, blk, 0, s, p);
    else hipLaunchKernelGGL((gemm_skinny_mfma<T, 4, false, PK, 0>), grid, blk, 0, s, p);
  }
}

void gemm_skinny(const Gemm& g, const SkinnyPlan& pl, const GArgs& p, hipStream_t s) {
  const dim3 grid((unsigned)pl.blocks);
  const bool ln = g.ln_gamma != nullptr;
  if (ln && !gemm_skinny_ln_ok(g)) fail("gemm: layer-norm prologue not supported for this operand");
  if (g.b_packed && !al16(g.B)) fail("gemm: packed weights must be 16-byte aligned");
  // 4 steps in flight when each wave has at most 4 (K <= 2048), else 12
  const bool deep = (g.K + 32 * kSkWaves - 1) / (32 * kSkWaves) > 4;
  const int xlds = skinny_xlds(g);
  if (g.dt == DType::F16) {
    if (g.b_packed) launch_skinny<half_t, true>(p, grid, deep, ln, xlds, s);
    else launch_skinny<half_t, false>(p, grid, deep, ln, xlds, s);
  } else {
    if (g.b_packed) launch_skinny<bf16_t, true>(p, grid, deep, ln, xlds, s);
    else launch_skinny<bf16_t, false>(p, grid, deep, ln, xlds, s);
  }
  check_launch("gemm_skinny");
}

}  // namespace k
}  // namespace agpu
