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

constexpr int kSkMaxM = 16;
constexpr int kSkXlds = 16384;      // A elements staged in LDS (32 KB): M K <= 16384, K <= 2048
constexpr int kSkXldsWide = 49152;  // the wide staging (96 KB, one block per CU): M <= 8, K <= 6144
constexpr int kSkRowMaxK = 2048;    // row a wave normalises in registers (the layer-norm prologue)
constexpr int kSkMaxUn = 12;        // steps in flight per wave

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

// W: waves per block (8 when M <= 8, else 16; wave w stages row w); UN:
// steps in flight per wave (the launch picks ceil(steps / W), so no wave
// loads a step it does not own); LN: layer-norm the A rows (needs XLDS);
// PACKED: B in the packed layout; XS > 0: A rows staged in LDS (XS
// elements), R = ceil(W UN / 16) 8-runs per lane covering a row of K.
template <typename T, int W, int UN, bool LN, bool PACKED, int XS>
__global__ void __launch_bounds__(64 * W) gemm_skinny_mfma(GArgs p) {
  constexpr bool XLDS = XS > 0;
  constexpr int R = XLDS ? (W * UN + 15) / 16 : 1;
  static_assert(!LN || XLDS, "the layer-norm prologue stages A in LDS");
  static_assert(!LN || R <= kSkRowMaxK / 512, "the layer-norm row is held in registers");
  typedef typename Mfma16<T>::vec V8;
  __shared__ float red[W][16 * 16];
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
      const int64_t st = s0 + (int64_t)u * W;
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

  // Wave w < M stages row w: it loads the row (and gamma, beta) first, then
  // every wave issues its first B steps, so the staging waits for its own
  // loads only (a wave's loads complete in issue order) while the weights
  // stream in.  The lanes' runs past K load from clamped in-range addresses
  // rather than under a per-lane branch, which would make the wave wait for
  // each load as it issues.  Waves past M load nothing here: every load
  // instruction of the block takes the CU's one vector-memory path, and the
  // weights should not queue behind copies of rows that are not needed.
  // The epilogue operands are loaded after the staging.
  const bool stager = XLDS && w < p.M;
  V8 run[XLDS ? R : 1], lg[LN ? R : 1], lb[LN ? R : 1];
  if (stager) {
    const T* xr = (const T*)p.A + w * p.a_sm;
#pragma unroll
    for (int c = 0; c < R; ++c) {
      const int64_t kk = (int64_t)(lane + 64 * c) * 8;
      const int64_t kc = kk < p.K ? kk : 0;
      run[c] = *(const V8*)(xr + kc);
      if constexpr (LN) {
        lg[c] = *(const V8*)((const T*)p.ln_g + kc);
        lb[c] = *(const V8*)((const T*)p.ln_b + kc);
      }
    }
  }
  // Compiler and scheduling barriers keep the issue order: staging loads,
  // then the weights, then the staging arithmetic.  Without them the
  // compiler sinks gamma/beta into the store below and schedules the weight
  // loads behind the statistics, and the staging then waits for the weights.
  if constexpr (XLDS) __builtin_amdgcn_sched_barrier(0);
  V8 b[UN];
  load_b(b, w);
  if constexpr (XLDS) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (XLDS) {
    if (stager) {
      if constexpr (LN) {
        float sum = 0.f;
#pragma unroll
        for (int c = 0; c < R; ++c) {
          const bool in = (int64_t)(lane + 64 * c) * 8 < p.K;
#pragma unroll
          for (int e = 0; e < 8; ++e) sum += in ? (float)run[c][e] : 0.f;
        }
        const float mean = wave_sum(sum) / (float)p.K;
        float sq = 0.f;
#pragma unroll
        for (int c = 0; c < R; ++c) {
          const bool in = (int64_t)(lane + 64 * c) * 8 < p.K;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = (float)run[c][e] - mean;
            sq += in ? d * d : 0.f;
          }
        }
        const float rs = 1.f / sqrtf(wave_sum(sq) / (float)p.K + p.ln_eps);
#pragma unroll
        for (int c = 0; c < R; ++c) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            run[c][e] = T((float)lg[c][e] * ((float)run[c][e] - mean) * rs + (float)lb[c][e]);
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
  // threads 0..255 each finish one output (m, n0 + c): its bias/residual now
  // (every thread loads, from a clamped legal element: no divergent branch
  // around the loads), behind the weights still in flight
  const int om = (tid >> 4) & 15, oc = tid & 15;
  const bool owns = tid < 256 && om < p.M && n0 + oc < p.N;
  const EpiIn<T> ein = epilogue_load<T>(p, 0, om < p.M ? om : p.M - 1, n0 + oc < p.N ? n0 + oc : p.N - 1);

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t s0 = w; s0 < steps; s0 += (int64_t)W * UN) {
    V8 a[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t st = s0 + (int64_t)u * W;
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
    if (s0 + (int64_t)W * UN < steps) load_b(b, s0 + (int64_t)W * UN);
  }

  // C layout of a 16x16 MFMA tile: lane l, register r -> row 4*(l/16) + r,
  // column l%16.
#pragma unroll
  for (int r = 0; r < 4; ++r) red[w][(4 * (lane >> 4) + r) * 16 + (lane & 15)] = acc[r];
  __syncthreads();
  if (!owns) return;
  float v = 0.f;
#pragma unroll
  for (int ww = 0; ww < W; ++ww) v += red[ww][tid];
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

// LDS staging of A: 0 = none (A operands from global memory), else the
// staging array the launch uses.
static int skinny_xlds(const Gemm& g) {
  if (g.M * g.K <= kSkXlds && g.K <= kSkRowMaxK) return kSkXlds;
  if (g.M <= 8 && g.M * g.K <= kSkXldsWide && (g.K + 511) / 512 <= kSkMaxUn) return kSkXldsWide;
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

// Launch shapes: 8 waves when M <= 8 (one staged row each; several blocks
// share a CU), 16 otherwise, and for the wide staging (one block per CU
// streaming a long K); UN = ceil(steps / W), so that each wave's first
// loads are exactly its steps (capped at kSkMaxUn for unstaged long K,
// which loops).
template <int U, int LO, int HI>
constexpr int clamp_un() { return U < LO ? LO : (U > HI ? HI : U); }

// UN in [LO, HI]: only those variants are instantiated.
template <typename T, bool PK, int W, bool LN, int XS, int LO, int HI>
static void launch_un(const GArgs& p, dim3 grid, int un, hipStream_t s) {
  const dim3 blk(64 * W);
#define AGPU_SK(U) \
  hipLaunchKernelGGL((gemm_skinny_mfma<T, W, clamp_un<U, LO, HI>(), LN, PK, XS>), grid, blk, 0, s, p)
  switch (un < LO ? LO : (un > HI ? HI : un)) {
    case 1: AGPU_SK(1); break;
    case 2: AGPU_SK(2); break;
    case 3: AGPU_SK(3); break;
    case 4: AGPU_SK(4); break;
    case 5: AGPU_SK(5); break;
    case 6: AGPU_SK(6); break;
    case 7: AGPU_SK(7); break;
    case 8: AGPU_SK(8); break;
    case 9: AGPU_SK(9); break;
    case 10: AGPU_SK(10); break;
    case 11: AGPU_SK(11); break;
    default: AGPU_SK(12); break;
  }
#undef AGPU_SK
}

template <typename T, bool PK>
static void launch_skinny(const GArgs& p, dim3 grid, bool ln, int xs, hipStream_t s) {
  const int64_t steps = (p.K + 31) / 32;
  auto un_for = [&](int w) { return (int)std::min<int64_t>((steps + w - 1) / w, kSkMaxUn); };
  if (xs == kSkXlds) {
    if (p.M <= 8) {
      // K <= 2048: at most 8 steps per wave
      if (ln) launch_un<T, PK, 8, true, kSkXlds, 1, 8>(p, grid, un_for(8), s);
      else launch_un<T, PK, 8, false, kSkXlds, 1, 8>(p, grid, un_for(8), s);
    } else {
      // M K <= 16384 with M > 8: K < 2048, at most 4 steps per wave
      if (ln) launch_un<T, PK, 16, true, kSkXlds, 1, 4>(p, grid, un_for(16), s);
      else launch_un<T, PK, 16, false, kSkXlds, 1, 4>(p, grid, un_for(16), s);
    }
  } else if (xs == kSkXldsWide) {
    // 2048 < K <= 6144 (M <= 8): 5 to 12 steps per wave
    launch_un<T, PK, 16, false, kSkXldsWide, 5, kSkMaxUn>(p, grid, un_for(16), s);
  } else {
    launch_un<T, PK, 16, false, 0, 1, kSkMaxUn>(p, grid, un_for(16), s);
  }
}

void gemm_skinny(const Gemm& g, const SkinnyPlan& pl, const GArgs& p, hipStream_t s) {
  const dim3 grid((unsigned)pl.blocks);
  const bool ln = g.ln_gamma != nullptr;
  if (ln && !gemm_skinny_ln_ok(g)) fail("gemm: layer-norm prologue not supported for this operand");
  if (g.b_packed && !al16(g.B)) fail("gemm: packed weights must be 16-byte aligned");
  const int xlds = skinny_xlds(g);
  if (g.dt == DType::F16) {
    if (g.b_packed) launch_skinny<half_t, true>(p, grid, ln, xlds, s);
    else launch_skinny<half_t, false>(p, grid, ln, xlds, s);
  } else {
    if (g.b_packed) launch_skinny<bf16_t, true>(p, grid, ln, xlds, s);
    else launch_skinny<bf16_t, false>(p, grid, ln, xlds, s);
  }
  check_launch("gemm_skinny");
}

}  // namespace k
}  // namespace agpu
