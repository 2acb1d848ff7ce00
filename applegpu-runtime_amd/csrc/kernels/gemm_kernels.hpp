// Shared pieces of the gfx950 GEMM kernels: launch arguments, the fused
// epilogue, XCD-aware tile scheduling and the bf16-MFMA kernel family
// (gemm_mf).  Included by gemm.hip and by the per-dtype launch units
// gemm_mf_{f32,f16,bf16}.hip, which instantiate the kernels in parallel.
#pragma once

#include <type_traits>

#include "device.hpp"


namespace agpu {
namespace k {
using namespace dev;


typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct GArgs {
  const void* A; const void* B; void* C;
  int64_t M, N, K;
  int64_t a_sm, a_sk, a_sb, b_sk, b_sn, b_sb, c_sm, c_sb;
  int64_t batch;
  int splits;
  int64_t k_per_split;
  float alpha;
  const void* bias;
  int act;
  const void* res; int64_t r_sm, r_sb;
  const void* mask; int64_t k_sm, k_sb;
  float* ws;
  int tiles_m, tiles_n;
  bool vec_a, vec_b;
  const float* b_scale;
  const void* ln_g; const void* ln_b; float ln_eps;
  const void* pln_g; const void* pln_b; void* pln_y; float pln_eps;
  // packed-x3 row operands (bf16 hi/lo MFMA fragments, see x3_row_offset):
  // A read packed, C and the layer_norm output also (or only) written packed
  bool a_x3;
  bf16_t* c_pk;
  bf16_t* pln_ypk;
  PfArgs pf;  // read-ahead blocks (split-K layer_norm reductions)
  // row statistics for a layer_norm folded into the next GEMM (row-panel
  // plans): rs_out receives, per output row and 32-column tile, the tile's
  // sum and sum of squared deviations from the tile mean ([M, N / 32, 2]);
  // with rs_in (the A rows' statistics, [M, rs_tiles, 2] over rs_n columns)
  // the epilogue forms inv * (acc - mean * rs_cs[n]) before the bias
  float* rs_out;
  const float* rs_in;
  const float* rs_cs;
  int rs_tiles;
  int64_t rs_n;
  float rs_eps;
  // rowsum_acc[m] += alpha * sum_k A(m, k) (gemm_a_rowsum_fused plans)
  float* rowsum_acc;
  // split row-panel launches that finish each output tile in the kernel:
  // one arrival counter per tile (zero before the launch, zero after it);
  // null = the splits' sums go to the workspace for a reduction launch
  unsigned* tile_cnt;
};

// Epilogue operands of one output, loadable ahead of the product (they do
// not depend on it), so that their latency hides under the main loop; kept
// raw until the epilogue (converting at the load would make the compiler
// wait for them right there).
template <typename T>
struct EpiIn {
  T bias = T(0), res = T(0), mask = T(1);
};
// Branch-free: an absent operand reads the output element itself (a legal
// address; the value is not used), so no load sits behind a branch that the
// compiler would close with a wait.
template <typename T>
__device__ __forceinline__ EpiIn<T> epilogue_load(const GArgs& p, int64_t b, int64_t row, int64_t col) {
  const T* out = (const T*)p.C + b * p.c_sb + row * p.c_sm + col;
  const T* bp = p.bias ? (const T*)p.bias + col : out;
  const T* rp = p.res ? (const T*)p.res + b * p.r_sb + row * p.r_sm + col : out;
  const T* mp = p.mask ? (const T*)p.mask + b * p.k_sb + row * p.k_sm + col : out;
  EpiIn<T> e;
  e.bias = *bp;
  e.res = *rp;
  e.mask = *mp;
  return e;
}
template <typename T>
__device__ __forceinline__ void epilogue_finish(const GArgs& p, int64_t b, int64_t row, int64_t col, float acc,
                                                const EpiIn<T>& e) {
  float v = p.alpha * acc + (p.bias ? to_f(e.bias) : 0.f);
  if (p.act == kActRelu) v = fmaxf(v, 0.f);
  else if (p.act == kActGelu) v = gelu_tanh(v);
  else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
  v += p.res ? to_f(e.res) : 0.f;
  if (p.mask) v = to_f(e.mask) > 0.f ? v : 0.f;
  ((T*)p.C)[b * p.c_sb + row * p.c_sm + col] = from_f<T>(v);
}

template <typename T>
__device__ __forceinline__ void epilogue_store(const GArgs& p, int64_t b, int64_t row, int64_t col, float acc) {
  float v = p.alpha * acc;
  if (p.bias) v += to_f(((const T*)p.bias)[col]);
  if (p.act == kActRelu) v = fmaxf(v, 0.f);
  else if (p.act == kActGelu) v = gelu_tanh(v);
  else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
  if (p.res) v += to_f(((const T*)p.res)[b * p.r_sb + row * p.r_sm + col]);
  if (p.mask) v = to_f(((const T*)p.mask)[b * p.k_sb + row * p.k_sm + col]) > 0.f ? v : 0.f;
  ((T*)p.C)[b * p.c_sb + row * p.c_sm + col] = from_f<T>(v);
}

// epilogue_store's arithmetic, returning the value as stored (rounded to T).
template <typename T>
__device__ __forceinline__ float epilogue_apply(const GArgs& p, int64_t b, int64_t row, int64_t col, float acc) {
  float v = p.alpha * acc;
  if (p.bias) v += to_f(((const T*)p.bias)[col]);
  if (p.act == kActRelu) v = fmaxf(v, 0.f);
  else if (p.act == kActGelu) v = gelu_tanh(v);
  else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
  if (p.res) v += to_f(((const T*)p.res)[b * p.r_sb + row * p.r_sm + col]);
  if (p.mask) v = to_f(((const T*)p.mask)[b * p.k_sb + row * p.k_sm + col]) > 0.f ? v : 0.f;
  const T o = from_f<T>(v);
  ((T*)p.C)[b * p.c_sb + row * p.c_sm + col] = o;
  return to_f(o);
}

// Tile scheduling: XCD-aware remap, then 8-row tile groups.
__device__ __forceinline__ void tile_coords(const GArgs& p, int& tm, int& tn) {
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int GM = 8;
  const int per_group = GM * p.tiles_n;
  const int group = bid / per_group;
  const int first_m = group * GM;
  const int gsz = min(p.tiles_m - first_m, GM);
  const int in_group = bid % per_group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

// ── bf16 MFMA kernel family: fp32 via bf16x3, or fp16/bf16 operands ───────
// One 256-thread block (4 wavefronts) computes a BM x BN tile of C.  The
// waves form a WM x WN x WK grid: WM x WN split the tile, WK split every
// K slice of the block (in-block split-K, reduced through LDS at the end, so
// skinny problems fill the GPU without a second launch).  Each wave owns
// (BM/WM) x (BN/WN) outputs as 32x32 MFMA blocks and KW k values of each
// BK = KW*WK slice.
//
// Global -> registers (16-byte loads along whichever axis is contiguous,
// next slice prefetched while the current one is multiplied) -> LDS, laid
// out [row][k] with k contiguous and rows padded by 8 elements, so that one
// lane's MFMA operand (8 consecutive k of one row) is a single 16-byte read.
// fp32 operands are split on the way into LDS: hi = bf16(x) (round to
// nearest even), lo = bf16(x - hi); C += Ahi*Bhi + Ahi*Blo + Alo*Bhi with
// fp32 accumulation (Henry, Tang, Heinecke, "Leveraging the bfloat16
// artificial intelligence datatype for higher-precision computations", 2019).
// The dropped lo*lo term and the two roundings leave a relative error near
// 2^-16 per product, far inside the 1e-3 fp32 GEMM tolerance.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename E> struct Mfma32;
template <> struct Mfma32<bf16_t> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma32<half_t> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// hi = bf16(x) (RNE), lo = bf16(x - hi); non-finite x keeps lo = 0 so that
// an infinite operand gives an infinite (not NaN) product.
__device__ __forceinline__ void split_bf16(float x, bf16_t& hi, bf16_t& lo) {
  hi = (bf16_t)x;
  const float r = x - (float)hi;
  lo = (bf16_t)(__builtin_isfinite(x) ? r : 0.f);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// split_bf16 of two values at once: each rounding is one v_cvt_pk_bf16_f32
// for the pair (the scalar form converts one value per instruction).
__device__ __forceinline__ void split_bf16x2(float x0, float x1, bf16x2_t& hi, bf16x2_t& lo) {
  const f32x2_t x = {x0, x1};
  hi = __builtin_convertvector(x, bf16x2_t);
  f32x2_t r = x - __builtin_convertvector(hi, f32x2_t);
  r.x = __builtin_isfinite(x0) ? r.x : 0.f;
  r.y = __builtin_isfinite(x1) ? r.y : 0.f;
  lo = __builtin_convertvector(r, bf16x2_t);
}

// Packed x3 rows: a matrix X [M, K] (K % 16 == 0) stored as the A operand
// of v_mfma_f32_32x32x16_bf16, hi = bf16(x), lo = bf16(x - hi).  Element
// (r, k) of part h sits at ((s T + t) 2 + h) 512 + 8 l + j with s = r / 32,
// t = k / 16, l = r % 32 + 32 ((k / 8) % 2), j = k % 8 and T = K / 16: one
// lane's operand (8 consecutive k of one row) is 16 contiguous bytes and one
// wavefront's fragment 1 KB.  Rows past M (up to the next multiple of 32) are
// never written; the products they feed are never stored.  It is the layout
// of the packed weights with rows in place of columns.
__device__ __forceinline__ int64_t x3_row_offset(int64_t r, int64_t k, int64_t T) {
  const int64_t l = (r & 31) + 32 * ((k >> 3) & 1);
  return (((r >> 5) * T + (k >> 4)) * 2) * 512 + l * 8 + (k & 7);
}
// Stores x[0..3] = X(r, k..k+3), k % 4 == 0, as hi and lo (8 bytes each).
__device__ __forceinline__ void x3_store4(bf16_t* pk, int64_t T, int64_t r, int64_t k, const float (&x)[4]) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x2_t h0, l0, h1, l1;
  split_bf16x2(x[0], x[1], h0, l0);
  split_bf16x2(x[2], x[3], h1, l1);
  bf16_t* d = pk + x3_row_offset(r, k, T);
  *(bf16x4_t*)d = bf16x4_t{h0.x, h0.y, h1.x, h1.y};
  *(bf16x4_t*)(d + 512) = bf16x4_t{l0.x, l0.y, l1.x, l1.y};
}

// Per-thread share of a ROWS x BK operand slice.  KCONT: the operand is
// contiguous along k (A row-major, or B = W^T with W [n][k]); the thread owns
// one row and EPT consecutive k.  !KCONT: contiguous along rows (A column-
// major, B row-major [k][n]); the thread owns VW consecutive rows for each of
// KP consecutive k and transposes them in registers, so its LDS writes are
// runs of KP contiguous k.  Lanes walk k fastest there: a wave's writes then
// cover consecutive LDS words (no bank conflicts) while each of its 16-byte
// global loads still reads whole rows segments of the operand.
//
// load_fast: interior slices, unconditional 16-byte loads.  Rows past the
// operand are clamped onto its last row (KCONT) or last VW-row group (!KCONT,
// which needs rows % VW == 0): they only feed output rows or columns that are
// never stored, so they need no masking.  load_edge: any slice, element
// loads from clamped (always legal) addresses plus a validity mask applied
// when the slice is written to LDS; used outside the main loop (the K
// remainder) or by the slow variant for shapes load_fast cannot take.
template <typename TI, int ROWS, int BK, bool KCONT>
struct GLoad {
  static constexpr int VW = 16 / (int)sizeof(TI);
  static constexpr int EPT = ROWS * BK / 256;
  static_assert(EPT % VW == 0 && EPT <= 64, "operand slice size");
  static constexpr int KP = KCONT ? EPT : EPT / VW;
  static constexpr int KQ = BK / KP;  // !KCONT: lanes along k
  TI v[EPT];  // KCONT: v[k]; !KCONT: v[j * VW + c] = X(k0 + j, r0 + c)
  uint64_t valid;

  __device__ __forceinline__ static void coords(int& r, int& kk) {
    const int t = threadIdx.x;
    if constexpr (KCONT) {
      constexpr int TPR = BK / EPT;
      r = t / TPR;
      kk = (t % TPR) * EPT;
      if constexpr (TPR == 2 && ROWS % 16 == 0 && BK % 16 == 0 && EPT <= 32) {
        // Rows are permuted within groups of 16 so that a store phase of 16
        // lanes (8 rows, two lanes each) hits every LDS bank once.  The LDS
        // tiles hold 2-byte elements with a pitch of BK + 8, i.e. u = BK/8 + 1
        // (odd) 16-byte chunks, and the two lanes of a row start c = EPT/8
        // chunks apart.  With g = u*r mod 16, the 8 rows of a phase take the
        // g whose bit log2(c) equals the phase, so their chunks g and g + c
        // are 16 distinct ones.  Each lane pair still reads one whole row
        // segment from global memory.
        constexpr int u = BK / 8 + 1, c = EPT / 8;
        constexpr int lc = c == 1 ? 0 : c == 2 ? 1 : 2;
        constexpr int uinv = (u * u * u) & 15;  // u^4 = 1 mod 16 for odd u
        const int q = r & 15;
        const int g = (q & (c - 1)) | (((q >> 3) & 1) << lc) | ((q & 7 & ~(c - 1)) << 1);
        r = (r & ~15) | ((uinv * g) & 15);
      }
    } else {
      r = (t / KQ) * VW;
      kk = (t % KQ) * KP;
    }
  }

  __device__ __forceinline__ void load_fast(const TI* __restrict__ base, int64_t s_row, int64_t s_k, int64_t r0,
                                            int64_t rmax, int64_t k0) {
    int r, kk;
    coords(r, kk);
    if constexpr (KCONT) {
      const int64_t gr = r0 + r < rmax ? r0 + r : rmax - 1;
      const TI* src = base + gr * s_row + k0 + kk;
#pragma unroll
      for (int i = 0; i < EPT; i += VW) *(uint4*)&v[i] = *(const uint4*)(src + i);
    } else {
      const int64_t gr = r0 + r < rmax ? r0 + r : rmax - VW;
      const TI* src = base + (k0 + kk) * s_k + gr;
#pragma unroll
      for (int j = 0; j < KP; ++j) *(uint4*)&v[j * VW] = *(const uint4*)(src + j * s_k);
    }
  }

  __device__ __forceinline__ void load_edge(const TI* __restrict__ base, int64_t s_row, int64_t s_k, int64_t r0,
                                            int64_t rmax, int64_t k0, int64_t kmax) {
    int r, kk;
    coords(r, kk);
    const int64_t gr = r0 + r, gk = k0 + kk;
    uint64_t ok = 0;
    if constexpr (KCONT) {
      const bool rok = gr < rmax;
      const int64_t rr = rok ? gr : rmax - 1;
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        const bool e = rok && gk + i < kmax;
        const int64_t kc = gk + i < kmax ? gk + i : kmax - 1;
        v[i] = base[rr * s_row + kc];
        ok |= (uint64_t)e << i;
      }
    } else {
#pragma unroll
      for (int j = 0; j < KP; ++j) {
        const bool kok = gk + j < kmax;
        const int64_t kc = kok ? gk + j : kmax - 1;
#pragma unroll
        for (int c = 0; c < VW; ++c) {
          const bool e = kok && gr + c < rmax;
          const int64_t rc = gr + c < rmax ? gr + c : rmax - 1;
          v[j * VW + c] = base[kc * s_k + rc];
          ok |= (uint64_t)e << (j * VW + c);
        }
      }
    }
    valid = ok;
  }

  template <bool MASKED>
  __device__ __forceinline__ TI at(int e) const {
    if constexpr (MASKED) return ((valid >> e) & 1) ? v[e] : TI(0);
    else return v[e];
  }

  // fp32 (or int8 codes times a per-row scale `rs`, KCONT only) operand ->
  // hi/lo bf16 LDS tiles (row pitch LD elements).
  template <bool MASKED>
  __device__ __forceinline__ void store_split(bf16_t* __restrict__ hi, bf16_t* __restrict__ lo, int LD,
                                              float rs = 1.f) const {
    int r, kk;
    coords(r, kk);
    if constexpr (KCONT) {
#pragma unroll
      for (int i = 0; i < EPT; i += 8) {
        bf16x8_t h, l;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float x0 = std::is_same<TI, int8_t>::value ? (float)at<MASKED>(i + e) * rs : (float)at<MASKED>(i + e);
          const float x1 =
              std::is_same<TI, int8_t>::value ? (float)at<MASKED>(i + e + 1) * rs : (float)at<MASKED>(i + e + 1);
          bf16x2_t a, b;
          split_bf16x2(x0, x1, a, b);
          h[e] = a.x;
          h[e + 1] = a.y;
          l[e] = b.x;
          l[e + 1] = b.y;
        }
        *(bf16x8_t*)&hi[r * LD + kk + i] = h;
        *(bf16x8_t*)&lo[r * LD + kk + i] = l;
      }
    } else if constexpr (KP % 2 == 0) {
#pragma unroll
      for (int c = 0; c < VW; ++c) {
        bf16_t h[KP], l[KP];
#pragma unroll
        for (int j = 0; j < KP; j += 2) {
          bf16x2_t a, b;
          split_bf16x2((float)at<MASKED>(j * VW + c), (float)at<MASKED>((j + 1) * VW + c), a, b);
          h[j] = a.x;
          h[j + 1] = a.y;
          l[j] = b.x;
          l[j + 1] = b.y;
        }
        store_run(&hi[(r + c) * LD + kk], h);
        store_run(&lo[(r + c) * LD + kk], l);
      }
    } else {
#pragma unroll
      for (int c = 0; c < VW; ++c) {
        bf16_t h[KP], l[KP];
#pragma unroll
        for (int j = 0; j < KP; ++j) split_bf16((float)at<MASKED>(j * VW + c), h[j], l[j]);
        store_run(&hi[(r + c) * LD + kk], h);
        store_run(&lo[(r + c) * LD + kk], l);
      }
    }
  }

  // 16-bit operand -> one LDS tile.
  template <bool MASKED>
  __device__ __forceinline__ void store_plain(TI* __restrict__ t, int LD) const {
    int r, kk;
    coords(r, kk);
    if constexpr (KCONT) {
#pragma unroll
      for (int i = 0; i < EPT; i += 8) {
        TI run[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) run[e] = at<MASKED>(i + e);
        *(uint4*)&t[r * LD + kk + i] = *(const uint4*)run;
      }
    } else {
#pragma unroll
      for (int c = 0; c < VW; ++c) {
        TI run[KP];
#pragma unroll
        for (int j = 0; j < KP; ++j) run[j] = at<MASKED>(j * VW + c);
        store_run(&t[(r + c) * LD + kk], run);
      }
    }
  }

  // KP contiguous 2-byte values, written with the widest aligned LDS store.
  template <typename E>
  __device__ __forceinline__ static void store_run(E* dst, const E* src) {
    if constexpr (KP * sizeof(E) == 16) *(uint4*)dst = *(const uint4*)src;
    else if constexpr (KP * sizeof(E) == 8) *(uint2*)dst = *(const uint2*)src;
    else if constexpr (KP * sizeof(E) == 4) *(uint32_t*)dst = *(const uint32_t*)src;
    else {
#pragma unroll
      for (int j = 0; j < KP; ++j) dst[j] = src[j];
    }
  }
};

template <int A, int B> struct CMax { static constexpr int v = A > B ? A : B; };

// TI: global operand type (float, or the 16-bit type E itself); E: LDS/MFMA
// element type; X3: fp32 operands split into hi/lo (TI = float, E = bf16).
// ST: LDS stages (2: double-buffered, one barrier per slice; 1: a single
// buffer and two barriers per slice, for tiles too large to double).
// FAST: the operands qualify for GLoad::load_fast (16-byte aligned rows,
// K % VW == 0, and rows % VW == 0 for an operand contiguous along rows): the
// K remainder (K mod BK of this block's range) is multiplied first, from a
// masked load, and every later slice is full.  !FAST: every slice is loaded
// with GLoad::load_edge.
template <typename TI, typename TB, typename E, int BM, int BN, int WM, int WN, int WK, int KW, int ST, bool AK,
          bool BKC, bool FAST>
__global__ void __launch_bounds__(256) gemm_mf(GArgs p) {
  constexpr bool X3 = sizeof(TI) == 4;
  // TB = int8: B holds int8 codes, B(k, n) = code * b_scale[n] (KCONT only).
  constexpr bool QB = std::is_same<TB, int8_t>::value;
  static_assert(!QB || (X3 && BKC), "int8 B operand: fp32 A, k-contiguous B");
  static_assert(WM * WN * WK == 4, "four wavefronts per block");
  constexpr int BK = KW * WK;
  constexpr int LD = BK + 8;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1 && KW % 16 == 0, "tile shape");
  static_assert(ST == 1 || ST == 2, "one or two LDS stages");
  constexpr int NA = X3 ? 2 : 1;
  constexpr int AE = BM * LD, BE = BN * LD;
  constexpr int STAGE = NA * (AE + BE);
  constexpr int TILE_BYTES = ST * STAGE * (int)sizeof(E);
  constexpr int RED_BYTES = (WK - 1) * WM * WN * TM * TN * 16 * 64 * 4;
  __shared__ __attribute__((aligned(16))) char smem[CMax<TILE_BYTES, RED_BYTES>::v];
  E* const lds = (E*)smem;

  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t z = blockIdx.y;
  const int64_t b = z / p.splits;
  const int split = (int)(z % p.splits);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  int64_t kend = kbeg + p.k_per_split;
  if (kend > p.K) kend = p.K;
  const TI* A = (const TI*)p.A + b * p.a_sb;
  const TB* B = (const TB*)p.B + b * p.b_sb;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wk = wave / (WM * WN), wmn = wave % (WM * WN);
  const int wm = (wmn / WN) * (BM / WM), wn = (wmn % WN) * (BN / WN);
  float bscale = 1.f;  // QB: the scale of this thread's B row
  if constexpr (QB) {
    int r, kk;
    GLoad<TB, BN, KW * WK, BKC>::coords(r, kk);
    bscale = p.b_scale[n0 + r < p.N ? n0 + r : p.N - 1];
  }

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // PD = 2 for fp32 operands on the fast path (below); 16-bit operands and
  // the masked-load variant keep the one-set loop in the else branch (with
  // two sets the compiler put their loaders' arrays in scratch memory).
  constexpr int PD = X3 && FAST ? 2 : 1;
  if constexpr (PD == 2) {
    // Two register sets of operand slices: slice s is fetched into set s % 2
    // two slices before it is multiplied, so while slice kt is multiplied the
    // loads of slices kt+1 and kt+2 are both in flight (at the fp32 shapes of
    // the workloads the loop is bound by load latency, not by the MFMAs).
    GLoad<TI, BM, BK, AK> ga0, ga1;
    GLoad<TB, BN, BK, BKC> gb0, gb1;
    auto put = [&](auto masked, int stage, const auto& la, const auto& lb) __attribute__((always_inline)) {
      constexpr bool MK = decltype(masked)::value;
      E* s = lds + stage * STAGE;
      if constexpr (X3) {
        la.template store_split<MK>(s, s + AE, LD);
        lb.template store_split<MK>(s + 2 * AE, s + 2 * AE + BE, LD, bscale);
      } else {
        la.template store_plain<MK>(s, LD);
        lb.template store_plain<MK>(s + AE, LD);
      }
    };
    auto fetch_edge = [&](auto& la, auto& lb, int64_t k, int64_t kmax) __attribute__((always_inline)) {
      la.load_edge(A, p.a_sm, p.a_sk, m0, p.M, k, kmax);
      lb.load_edge(B, p.b_sn, p.b_sk, n0, p.N, k, kmax);
    };
    auto fetch_fast = [&](auto& la, auto& lb, int64_t k) __attribute__((always_inline)) {
      la.load_fast(A, p.a_sm, p.a_sk, m0, p.M, k);
      lb.load_fast(B, p.b_sn, p.b_sk, n0, p.N, k);
    };

    typedef typename Mfma32<E>::vec V8;
    auto compute = [&](int buf) __attribute__((always_inline)) {
      const E* s = lds + buf * STAGE;
      const E* a_hi = s;
      const E* b_hi = s + NA * AE;
  #pragma unroll
      for (int ks = 0; ks < KW; ks += 16) {
        const int ko = wk * KW + ks + 8 * (lane >> 5);
        V8 ah[TM], bh[TN];
  #pragma unroll
        for (int i = 0; i < TM; ++i) ah[i] = *(const V8*)&a_hi[(wm + i * 32 + (lane & 31)) * LD + ko];
  #pragma unroll
        for (int j = 0; j < TN; ++j) bh[j] = *(const V8*)&b_hi[(wn + j * 32 + (lane & 31)) * LD + ko];
        if constexpr (X3) {
          const E* a_lo = s + AE;
          const E* b_lo = s + 2 * AE + BE;
          V8 al[TM], bl[TN];
  #pragma unroll
          for (int i = 0; i < TM; ++i) al[i] = *(const V8*)&a_lo[(wm + i * 32 + (lane & 31)) * LD + ko];
  #pragma unroll
          for (int j = 0; j < TN; ++j) bl[j] = *(const V8*)&b_lo[(wn + j * 32 + (lane & 31)) * LD + ko];
          // small terms first, then hi*hi
  #pragma unroll
          for (int i = 0; i < TM; ++i)
  #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<E>::run(al[i], bh[j], acc[i][j]);
  #pragma unroll
          for (int i = 0; i < TM; ++i)
  #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<E>::run(ah[i], bl[j], acc[i][j]);
        }
  #pragma unroll
        for (int i = 0; i < TM; ++i)
  #pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<E>::run(ah[i], bh[j], acc[i][j]);
      }
    };

    // Slice schedule.  FAST: an optional masked remainder slice 0, then full
    // slices from k_full.  !FAST: every slice masked.
    const int64_t span = kend > kbeg ? kend - kbeg : 0;
    const int64_t tail = FAST ? span % BK : 0;
    const int64_t k_full = kbeg + tail;
    const int64_t nk = FAST ? span / BK + (tail ? 1 : 0) : (span + BK - 1) / BK;
    std::integral_constant<bool, true> masked;
    std::integral_constant<bool, false> plain;
    // k of full slice s >= 1 (FAST).  Fetches past the last slice re-read the
    // last one (legal addresses, no branch around the loads); what they bring
    // is never multiplied.
    auto slice_k = [&](int64_t s) __attribute__((always_inline)) {
      const int64_t c = s < nk ? s : nk - 1;
      return FAST ? k_full + (c - (tail ? 1 : 0)) * BK : kbeg + c * BK;
    };
    auto fetch_main = [&](auto& la, auto& lb, int64_t s) __attribute__((always_inline)) {
      if constexpr (FAST) fetch_fast(la, lb, slice_k(s));
      else fetch_edge(la, lb, slice_k(s), kend);
    };
    auto put_main = [&](int stage, const auto& la, const auto& lb) __attribute__((always_inline)) {
      if constexpr (FAST) put(plain, stage, la, lb);
      else put(masked, stage, la, lb);
    };
    if (nk > 0) {
      if constexpr (FAST) {
        if (tail) {
          fetch_edge(ga0, gb0, kbeg, k_full);
          put(masked, 0, ga0, gb0);
        } else {
          fetch_fast(ga0, gb0, k_full);
          put(plain, 0, ga0, gb0);
        }
        if (PD == 2 && nk > 1) fetch_fast(ga1, gb1, slice_k(1));
      } else {
        fetch_edge(ga0, gb0, kbeg, kend);
        put(masked, 0, ga0, gb0);
        if (PD == 2 && nk > 1) fetch_edge(ga1, gb1, slice_k(1), kend);
      }
    }
    __syncthreads();

    // One slice: fetch slice kt+PD into set F, multiply slice kt, then store
    // slice kt+1 (set P) into the other LDS stage.  The loop is unrolled by two
    // so that stages and register sets are compile-time choices.
    auto iter = [&](int64_t kt, int stage, auto& fa, auto& fb, const auto& pa, const auto& pb) __attribute__((always_inline)) {
      fetch_main(fa, fb, kt + PD);
      compute(stage);
      if constexpr (ST == 2) {
        put_main(stage ^ 1, pa, pb);
        __syncthreads();
      } else {
        __syncthreads();
        put_main(0, pa, pb);
        __syncthreads();
      }
    };
    {
      int64_t kt = 0;
      for (; kt + 1 < nk; kt += 2) {
        iter(kt, 0, ga0, gb0, ga1, gb1);
        iter(kt + 1, ST == 2 ? 1 : 0, ga1, gb1, ga0, gb0);
      }
      if (kt < nk) {  // odd slice count: the last slice sits in stage 0
        compute(0);
        __syncthreads();  // the in-block split-K reduction reuses the stages
      }
    }
  } else {
    GLoad<TI, BM, BK, AK> ga;
    GLoad<TB, BN, BK, BKC> gb;
    auto put = [&](auto masked, int stage) {
      constexpr bool MK = decltype(masked)::value;
      E* s = lds + stage * STAGE;
      if constexpr (X3) {
        ga.template store_split<MK>(s, s + AE, LD);
        gb.template store_split<MK>(s + 2 * AE, s + 2 * AE + BE, LD, bscale);
      } else {
        ga.template store_plain<MK>(s, LD);
        gb.template store_plain<MK>(s + AE, LD);
      }
    };
    auto fetch_edge = [&](int64_t k, int64_t kmax) {
      ga.load_edge(A, p.a_sm, p.a_sk, m0, p.M, k, kmax);
      gb.load_edge(B, p.b_sn, p.b_sk, n0, p.N, k, kmax);
    };
    auto fetch_fast = [&](int64_t k) {
      ga.load_fast(A, p.a_sm, p.a_sk, m0, p.M, k);
      gb.load_fast(B, p.b_sn, p.b_sk, n0, p.N, k);
    };

    typedef typename Mfma32<E>::vec V8;
    auto compute = [&](int buf) {
      const E* s = lds + buf * STAGE;
      const E* a_hi = s;
      const E* b_hi = s + NA * AE;
  #pragma unroll
      for (int ks = 0; ks < KW; ks += 16) {
        const int ko = wk * KW + ks + 8 * (lane >> 5);
        V8 ah[TM], bh[TN];
  #pragma unroll
        for (int i = 0; i < TM; ++i) ah[i] = *(const V8*)&a_hi[(wm + i * 32 + (lane & 31)) * LD + ko];
  #pragma unroll
        for (int j = 0; j < TN; ++j) bh[j] = *(const V8*)&b_hi[(wn + j * 32 + (lane & 31)) * LD + ko];
        if constexpr (X3) {
          const E* a_lo = s + AE;
          const E* b_lo = s + 2 * AE + BE;
          V8 al[TM], bl[TN];
  #pragma unroll
          for (int i = 0; i < TM; ++i) al[i] = *(const V8*)&a_lo[(wm + i * 32 + (lane & 31)) * LD + ko];
  #pragma unroll
          for (int j = 0; j < TN; ++j) bl[j] = *(const V8*)&b_lo[(wn + j * 32 + (lane & 31)) * LD + ko];
          // small terms first, then hi*hi
  #pragma unroll
          for (int i = 0; i < TM; ++i)
  #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<E>::run(al[i], bh[j], acc[i][j]);
  #pragma unroll
          for (int i = 0; i < TM; ++i)
  #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<E>::run(ah[i], bl[j], acc[i][j]);
        }
  #pragma unroll
        for (int i = 0; i < TM; ++i)
  #pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<E>::run(ah[i], bh[j], acc[i][j]);
      }
    };

    // Slice schedule.  FAST: an optional masked remainder slice first, then
    // full slices from k_full.  !FAST: every slice masked.
    const int64_t span = kend > kbeg ? kend - kbeg : 0;
    const int64_t tail = FAST ? span % BK : 0;
    const int64_t k_full = kbeg + tail;
    const int64_t nk = FAST ? span / BK + (tail ? 1 : 0) : (span + BK - 1) / BK;
    std::integral_constant<bool, true> masked;
    std::integral_constant<bool, false> plain;
    if (nk > 0) {
      if constexpr (FAST) {
        if (tail) {
          fetch_edge(kbeg, k_full);
          put(masked, 0);
        } else {
          fetch_fast(k_full);
          put(plain, 0);
        }
      } else {
        fetch_edge(kbeg, kend);
        put(masked, 0);
      }
    }
    __syncthreads();

    for (int64_t kt = 0; kt < nk; ++kt) {
      const int buf = ST == 2 ? (int)(kt & 1) : 0;
      const bool more = kt + 1 < nk;
      if (more) {
        if constexpr (FAST) fetch_fast(k_full + (kt + 1 - (tail ? 1 : 0)) * BK);
        else fetch_edge(kbeg + (kt + 1) * BK, kend);
      }
      compute(buf);
      if constexpr (ST == 2) {
        if (more) {
          if constexpr (FAST) put(plain, buf ^ 1);
          else put(masked, buf ^ 1);
        }
        __syncthreads();
      } else {
        __syncthreads();
        if (more) {
          if constexpr (FAST) put(plain, 0);
          else put(masked, 0);
          __syncthreads();
        }
      }
    }

  }

  // In-block split-K: waves wk > 0 hand their partial sums to wave wk = 0
  // through LDS (the tile buffers are free after the loop's last barrier).
  // No wave leaves before the block's last barrier.
  const bool owner = WK == 1 || wk == 0;
  if constexpr (WK > 1) {
    float* red = (float*)smem;
    constexpr int PER = TM * TN * 16 * 64;
    if (wk > 0) {
      float* dst = red + ((wk - 1) * (WM * WN) + wmn) * PER;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[((i * TN + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (owner) {
#pragma unroll
      for (int w = 1; w < WK; ++w) {
        const float* src = red + ((w - 1) * (WM * WN) + wmn) * PER;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] += src[((i * TN + j) * 16 + r) * 64 + lane];
      }
    }
  }

  // Output layout of a 32x32 block: lane l, register r ->
  //   row = 8*(r/4) + 4*(l/32) + r%4, col = l%32.
  typedef typename std::conditional<X3, float, E>::type TC;
  auto for_each_out = [&](auto&& fn) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col = n0 + wn + j * 32 + (lane & 31);
        if (col >= p.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row >= p.M) continue;
          fn(row, col, acc[i][j][r]);
        }
      }
  };
  if (p.splits == 1) {
    if (!owner) return;
    // epilogue_store's arithmetic, with each 32x32 block's operands loaded
    // together first (uniform branches, clamped rows and columns) instead of
    // one dependent load per output: the residual of an in-place update
    // (w += alpha * A B) is a full tile read.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col = n0 + wn + j * 32 + (lane & 31);
        const int64_t cc = col < p.N ? col : p.N - 1;
        const int64_t r0 = m0 + wm + i * 32 + 4 * (lane >> 5);
        float bias = 0.f, res[16], msk[16];
        if (p.bias) bias = to_f(((const TC*)p.bias)[cc]);
        if (p.res) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t row = r0 + 8 * (r >> 2) + (r & 3);
            res[r] = to_f(((const TC*)p.res)[b * p.r_sb + (row < p.M ? row : p.M - 1) * p.r_sm + cc]);
          }
        }
        if (p.mask) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t row = r0 + 8 * (r >> 2) + (r & 3);
            msk[r] = to_f(((const TC*)p.mask)[b * p.k_sb + (row < p.M ? row : p.M - 1) * p.k_sm + cc]);
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = r0 + 8 * (r >> 2) + (r & 3);
          float v = p.alpha * acc[i][j][r] + bias;
          if (p.act == kActRelu) v = fmaxf(v, 0.f);
          else if (p.act == kActGelu) v = gelu_tanh(v);
          else if (p.act == kActGeluExact) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
          if (p.res) v += res[r];
          if (p.mask) v = msk[r] > 0.f ? v : 0.f;
          if (row < p.M && col < p.N) ((TC*)p.C)[b * p.c_sb + row * p.c_sm + col] = from_f<TC>(v);
        }
      }
    return;
  }
  // Split K across blocks: every split stores its partial tile and
  // splitk_reduce sums them in split order.  (Summing them in the block that
  // finishes a tile last would need a device-scope release per block, which
  // on MI355X writes back the XCD's whole L2: slower than the second launch.)
  const int64_t plane = p.M * p.N;
  if (owner)
    for_each_out([&](int64_t row, int64_t col, float v) {
      p.ws[((int64_t)split * p.batch + b) * plane + row * p.N + col] = v;
    });
}

// Tile configurations of gemm_mf: id, BM, BN, WM, WN, WK, KW, ST.
#define AGPU_MF_CONFIGS(X)             \
  X(0, 128, 128, 2, 2, 1, 32, 2)       \
  X(1, 64, 128, 1, 2, 2, 16, 2)        \
  X(2, 64, 64, 1, 1, 4, 16, 2)         \
  X(3, 32, 64, 1, 1, 4, 16, 2)         \
  X(4, 32, 32, 1, 1, 4, 16, 2)         \
  X(5, 128, 128, 2, 2, 1, 64, 1)       \
  X(6, 64, 64, 2, 2, 1, 64, 2)         \
  X(7, 64, 128, 2, 2, 1, 64, 1)       \
  X(8, 32, 32, 1, 1, 4, 64, 2)         \
  X(9, 32, 64, 1, 1, 4, 64, 1)         \
  X(10, 64, 64, 1, 1, 4, 32, 1)
struct MfShape { int bm, bn, bk; };
constexpr MfShape kMfShape[kMfConfigs] = {{128, 128, 32}, {64, 128, 32}, {64, 64, 64},   {32, 64, 64},
                                          {32, 32, 64},   {128, 128, 64}, {64, 64, 64},   {64, 128, 64},
                                          {32, 32, 256},  {32, 64, 256},  {64, 64, 128}};

template <typename TI, typename E, bool FAST>
void launch_mf(const GArgs& p, int cfg, bool ak, bool bk, dim3 grid, hipStream_t s) {
#define AGPU_MF_CASE(ID, BM, BN, WM, WN, WK, KW, ST)                                                       \
  case ID:                                                                                                \
    if (ak && bk)                                                                                         \
      hipLaunchKernelGGL((gemm_mf<TI, TI, E, BM, BN, WM, WN, WK, KW, ST, true, true, FAST>), grid, dim3(256), 0, s, p);   \
    else if (ak)                                                                                          \
      hipLaunchKernelGGL((gemm_mf<TI, TI, E, BM, BN, WM, WN, WK, KW, ST, true, false, FAST>), grid, dim3(256), 0, s, p);  \
    else if (bk)                                                                                          \
      hipLaunchKernelGGL((gemm_mf<TI, TI, E, BM, BN, WM, WN, WK, KW, ST, false, true, FAST>), grid, dim3(256), 0, s, p);  \
    else                                                                                                  \
      hipLaunchKernelGGL((gemm_mf<TI, TI, E, BM, BN, WM, WN, WK, KW, ST, false, false, FAST>), grid, dim3(256), 0, s, p); \
    break;
  switch (cfg) {
    AGPU_MF_CONFIGS(AGPU_MF_CASE)
    default: fail("gemm: unknown tile configuration %d", cfg);
  }
#undef AGPU_MF_CASE
}

// Skinny GEMM (M <= 16, one batch, 16-bit, B k-contiguous; gemm_skinny.hip):
// use = false when the problem does not qualify.
struct SkinnyPlan {
  bool use = false;
  int64_t blocks = 0;  // one block per 16 columns
};
SkinnyPlan skinny_plan(const Gemm& g, int cus);
void gemm_skinny(const Gemm& g, const SkinnyPlan& pl, const GArgs& p, hipStream_t s);

// GEMMs with a unit extent (gemm_thin.hip): N == 1, M == 1 (fp32, B rows
// contiguous along n) or K == 1; kThinNone when the problem is not one.
enum { kThinNone = 0, kThinN1, kThinM1, kThinK1 };
int thin_kind(const Gemm& g);
void gemm_thin(int kind, DType dt, const GArgs& p, hipStream_t s);

// The packed-weight bf16x3 GEMM (gemm_x3p.hip): partial sums into p.ws when
// the plan splits K, else the epilogue into C.
void gemm_x3p_launch(const X3Plan& pl, const GArgs& p, hipStream_t s);
// Arrival counters for a split packed-A row-panel launch of `tiles` tiles
// that finishes its tiles in the kernel, or null (reduction launch instead).
unsigned* split_tile_counters(int64_t tiles);

// Outer-shaped fp32 products (M, N multiples of 128 with at least 256 tiles
// of 128 x 128, K = 128, 256 or 512; one batch, no mask): both operands
// packed into the workspace (gemm_x3_outer_workspace bytes), then one
// four-wavefront block per 128 x 128 tile over the whole K (gemm_x3p.hip).
bool gemm_x3_outer_ok(const Gemm& g);
// Large fp16 / bf16 products with both operands contiguous along k (A rows,
// W [N][K]), M >= 256, K % 64 == 0, one batch, no mask: swizzled direct
// global -> LDS tiles of 256 x 256 for grids that fill one round of the
// CUs (gemm_h16.hip).
bool gemm_h16_ok(const Gemm& g, int cus);
void gemm_h16(const Gemm& g, const GArgs& p, int cus, hipStream_t s);
size_t gemm_x3_outer_workspace(const Gemm& g);
void gemm_x3_outer(const Gemm& g, const GArgs& p, void* ws, hipStream_t s);
// Two such products with the same K and a row-sum accumulator each (two SGD
// weight updates with their bias steps) as one pack launch and one GEMM
// launch; each product's workspace is its own gemm_x3_outer_workspace.
// fp32 products with at most 64 rows and large fp32 weights contiguous along
// k (gemm_f32s.hip): each weight byte read once into registers and split
// there, K split into ranges reduced by the split-K reduction.
bool gemm_f32_stream_ok(const Gemm& g, int cus);
int gemm_f32_stream_splits(const Gemm& g, int cus);
void gemm_f32_stream(const Gemm& g, const GArgs& p, int cus, hipStream_t s);
bool gemm_x3_outer2_ok(const Gemm& g0, const Gemm& g1);
void gemm_x3_outer2(const Gemm& g0, const GArgs& p0, void* ws0, const Gemm& g1, const GArgs& p1, void* ws1,
                    hipStream_t s);

// Defined in gemm_mf_{f32,f16,bf16}_{fast,edge}.hip.
void launch_mf_f32(const GArgs& p, int cfg, bool ak, bool bk, bool fast, dim3 grid, hipStream_t s);
void launch_mf_f16(const GArgs& p, int cfg, bool ak, bool bk, bool fast, dim3 grid, hipStream_t s);
void launch_mf_bf16(const GArgs& p, int cfg, bool ak, bool bk, bool fast, dim3 grid, hipStream_t s);
void launch_mf_f32_fast(const GArgs& p, int cfg, bool ak, bool bk, dim3 grid, hipStream_t s);
void launch_mf_f16_fast(const GArgs& p, int cfg, bool ak, bool bk, dim3 grid, hipStream_t s);
void launch_mf_bf16_fast(const GArgs& p, int cfg, bool ak, bool bk, dim3 grid, hipStream_t s);
// fp32 A times int8 B codes with per-n scales (k-contiguous B), configs 0
// and 6 only; defined in gemm_mf_i8.hip.
void launch_mf_f32_i8(const GArgs& p, int cfg, bool ak, bool fast, dim3 grid, hipStream_t s);

}  // namespace k
}  // namespace agpu
