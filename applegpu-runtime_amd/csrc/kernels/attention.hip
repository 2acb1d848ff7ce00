// Fused scaled-dot-product attention: O = softmax(scale * Q K^T [causal]) V.
//
// Reference semantics (crates/core/src/ops.rs:1531-1620): scores = Q @ K^T,
// then * (1/sqrt(d_k)), then softmax (or softmax_causal: key j is visible to
// query i iff j <= i, diagonal at (0,0), kernel_templates.rs:468-497), then
// @ V.  The reference materialises the transpose, the [.., Tq, Tk] score
// tensor and runs five kernels; here one kernel streams K/V tiles through LDS
// with an online softmax (running max and sum per query row), so scores never
// reach HBM.
//
// Layout: one 256-thread block owns 16 query rows of one (batch, head); 16
// threads share a row (lanes of a row are one 16-lane group of a wavefront,
// so row max/sum are 4 xor-shuffles).  Thread (r, sub) keeps its query row in
// registers, scores keys sub, sub+16, ... of each 64-key tile (K tile rows
// padded to D+4 floats: the 16 lanes' float4 reads hit distinct banks), and
// accumulates output dims [sub*D/16, (sub+1)*D/16) from a P tile in LDS.
// Q, K, V and O are read/written through their own (batch, head, token)
// strides with unit stride along d, so head splits of a fused QKV projection
// and the head-merge transpose cost nothing.
//
// Inputs with d = 64 or 128 and 16-byte aligned rows take the MFMA kernels
// (flash_attn_mfma for 16-bit, flash_attn_f32 below); other cases take the
// scalar kernel.
#include "device.hpp"
#include "gemm_kernels.hpp"  // x3_store4: packed x3 rows of the output

#include <type_traits>

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kQT = 16;  // query rows per block
constexpr int kKT = 64;  // keys per LDS tile
constexpr int kTPR = 16; // threads per query row

struct AArgs {
  const void* q; const void* k; const void* v; void* o;
  int64_t B, H, Tq, Tk;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale;
  int causal;
  int q_tiles;
  // Q/K/V given as split-K partial sums of their projection (fp32 kernel,
  // NSP > 0 partials `plane` elements apart) plus a bias, b_sh per head
  const float* qb; const float* kb; const float* vb;
  int64_t b_sh, plane;
  PfArgs pf;  // read-ahead blocks (fp32 kernel)
  bf16_t* o_pk;  // fp32 kernel: packed x3 rows of [B*Tq, H*D] instead of o
};

// Four consecutive fp32 values: a plain load, or (NSP > 0) the sum of NSP
// split-K partials in split order plus the bias: the split-K reduction's
// arithmetic, so the values equal the materialised projection's.
template <int NSP>
__device__ __forceinline__ float4 ld_part4(const float* ptr, int64_t plane, const float* bias) {
  float4 a = *(const float4*)ptr;
  if constexpr (NSP > 0) {
#pragma unroll
    for (int sp = 1; sp < NSP; ++sp) {
      const float4 b = *(const float4*)(ptr + sp * plane);
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    const float4 c = *(const float4*)bias;
    a.x += c.x; a.y += c.y; a.z += c.z; a.w += c.w;
  }
  return a;
}

template <typename T, int D>
__global__ void __launch_bounds__(256) flash_attn(AArgs p) {
  constexpr int KP = D + 4;     // K row pitch (floats)
  constexpr int PP = kKT + 4;   // P row pitch
  constexpr int DPT = D / kTPR; // output dims per thread
  constexpr int KPT = kKT / kTPR;  // keys per thread per tile
  __shared__ __attribute__((aligned(16))) float Ks[kKT * KP];
  __shared__ __attribute__((aligned(16))) float Vs[kKT * D];
  __shared__ __attribute__((aligned(16))) float Ps[kQT * PP];

  const int tid = threadIdx.x;
  const int r = tid / kTPR, sub = tid % kTPR;
  const int64_t bh = blockIdx.x / p.q_tiles;
  const int qt = (int)(blockIdx.x % p.q_tiles);
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q0 = (int64_t)qt * kQT;
  const int64_t qi = q0 + r;
  const bool row_ok = qi < p.Tq;

  const T* Q = (const T*)p.q + b * p.q_sb + h * p.q_sh;
  const T* K = (const T*)p.k + b * p.k_sb + h * p.k_sh;
  const T* V = (const T*)p.v + b * p.v_sb + h * p.v_sh;

  // Loads use clamped, always-legal rows and are masked afterwards: no
  // per-thread branches around global loads, so they all stay in flight.
  const int64_t qrow = row_ok ? qi : p.Tq - 1;
  float q[D];
#pragma unroll
  for (int d = 0; d < D; ++d) q[d] = to_f(Q[qrow * p.q_st + d]);
#pragma unroll
  for (int d = 0; d < D; ++d) q[d] = row_ok ? q[d] * p.scale : 0.f;

  float o[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) o[i] = 0.f;
  float m = -INFINITY, l = 0.f;

  int64_t kv_end = p.Tk;
  if (p.causal) {
    const int64_t last_q = q0 + kQT - 1 < p.Tq - 1 ? q0 + kQT - 1 : p.Tq - 1;
    kv_end = last_q + 1 < p.Tk ? last_q + 1 : p.Tk;
  }

  for (int64_t j0 = 0; j0 < kv_end; j0 += kKT) {
    // stage K and V tiles as fp32: all loads first, then the LDS stores
    constexpr int EPT = kKT * D / 256;
    float kr[EPT], vr[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = tid + 256 * i;
      const int c = e / D, d = e % D;
      const int64_t j = j0 + c < p.Tk ? j0 + c : p.Tk - 1;
      kr[i] = to_f(K[j * p.k_st + d]);
      vr[i] = to_f(V[j * p.v_st + d]);
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = tid + 256 * i;
      const int c = e / D, d = e % D;
      const bool ok = j0 + c < p.Tk;
      Ks[c * KP + d] = ok ? kr[i] : 0.f;
      Vs[c * D + d] = ok ? vr[i] : 0.f;
    }
    __syncthreads();

    float s[KPT];
    float tmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < KPT; ++jj) {
      const int c = sub + kTPR * jj;
      const float* kr = &Ks[c * KP];
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 kv = *(const float4*)&kr[d];
        acc += q[d] * kv.x;
        acc += q[d + 1] * kv.y;
        acc += q[d + 2] * kv.z;
        acc += q[d + 3] * kv.w;
      }
      const int64_t j = j0 + c;
      const bool vis = j < p.Tk && (!p.causal || j <= qi);
      s[jj] = vis ? acc : -INFINITY;
      tmax = fmaxf(tmax, s[jj]);
    }
#pragma unroll
    for (int x = 1; x < kTPR; x <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, x, 64));
    const float m_new = fmaxf(m, tmax);
    // m_new is finite for every row that has a visible key in this tile or an
    // earlier one; rows with none keep zero weight.
    const float alpha = (m == -INFINITY) ? 0.f : expf(m - m_new);
    float psum = 0.f;
#pragma unroll
    for (int jj = 0; jj < KPT; ++jj) {
      const float pv = (s[jj] == -INFINITY) ? 0.f : expf(s[jj] - m_new);
      psum += pv;
      Ps[r * PP + sub + kTPR * jj] = pv;
    }
#pragma unroll
    for (int x = 1; x < kTPR; x <<= 1) psum += __shfl_xor(psum, x, 64);
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int i = 0; i < DPT; ++i) o[i] *= alpha;
    __syncthreads();

    const int c_end = (int)(kv_end - j0 < kKT ? kv_end - j0 : kKT);
    for (int c = 0; c < c_end; ++c) {
      const float pv = Ps[r * PP + c];
      const float* vr = &Vs[c * D + sub * DPT];
#pragma unroll
      for (int i = 0; i < DPT; ++i) o[i] += pv * vr[i];
    }
    __syncthreads();
  }

  if (!row_ok) return;
  T* O = (T*)p.o + b * p.o_sb + h * p.o_sh + qi * p.o_st;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int i = 0; i < DPT; ++i) O[sub * DPT + i] = from_f<T>(o[i] * inv);
}


// ── MFMA flash attention (16-bit Q/K/V) ─────────────────────────────────────
// One block of 4 wavefronts owns QB = 64*QG query rows of one (batch, head);
// each wavefront owns QG groups of 16 rows.  K/V tiles of 64 keys are staged
// in LDS (double-buffered: the next tile's global loads are in flight while
// the current one is multiplied) and shared by the 4 wavefronts.
//
// Both products use v_mfma_f32_16x16x32 (lane l: A row l%16 and B column
// l%16, each at k = 8*(l/16)..+8; C register r of lane l is row 4*(l/16)+r,
// column l%16), oriented so that softmax needs no data movement:
//  - S^T = K Q^T: A = 16 keys x 32 dims of K (a 16-byte LDS read), B = this
//    lane's query row, held in registers for the whole kernel.  C then gives
//    every lane 16 scores of ONE query (l%16) for keys 16t + 4*(l/16) + r;
//  - the online softmax of a query is lane-local plus two xor shuffles (the
//    four lanes sharing l%16) for the tile max; the running sum stays
//    lane-partial until the end;
//  - O^T += V^T P^T: B = the lane's own probabilities (converted to the input
//    type), A = V^T.  The k index of an MFMA may be any permutation of the
//    keys as long as A and B agree, so V is stored in LDS transposed, [d][key],
//    with each 32-key group permuted so that the 8 keys lane group g holds
//    (4g..4g+3 and 16+4g..16+4g+3) are 8 consecutive elements: A is one
//    16-byte LDS read too;
//  - O^T's C layout gives lane l query l%16 and dims 16u + 4*(l/16) + r, so
//    the per-query rescale is one multiply per register.
// Scores are scaled by scale*log2(e) and exponentiated with exp2, which is
// exp of the scaled score.  Causal (key j visible to query i iff j <= i):
// a block stops at its last query's key; a wavefront skips tiles entirely
// after its queries, masks only the tiles that cross them, and blocks run
// heaviest query tiles first.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <typename E> struct FaMfma;
template <> struct FaMfma<half_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct FaMfma<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr int kFaWaves = 4;
constexpr int kFaKeys = 64;  // keys per LDS tile

// Position of key k (0..63) of a tile inside its V^T row: within each group
// of 32, key 16h + 4g + r goes to 8g + 4h + r.
__device__ __forceinline__ int fa_vpos(int k) {
  return (k & 32) | ((k & 12) << 1) | ((k & 16) >> 2) | (k & 3);
}

// One K/V tile in registers: K as KU 16-byte chunks, V as VU pairs of chunks
// of two consecutive keys (they become 32-bit pairs in the transposed tile).
// Named registers rather than arrays: with arrays the compiler kept the tile
// in scratch memory across the products.
template <typename T, int D>
struct FaTile {
  static constexpr int CH = D / 8;
  static constexpr int KU = kFaKeys * CH / (64 * kFaWaves);
  static constexpr int VU = (kFaKeys / 2) * CH / (64 * kFaWaves);
  static_assert(KU <= 4 && VU <= 2, "tile registers");
  uint4 k0, k1, k2, k3, va0, vb0, va1, vb1;

  __device__ __forceinline__ static uint4 ld(const T* base, int64_t row, int64_t stride, int64_t Tk, int col) {
    const int64_t j = row < Tk ? row : Tk - 1;  // rows past Tk repeat row Tk-1
    return *(const uint4*)(base + j * stride + col);
  }
  __device__ __forceinline__ void load(const T* K, const T* V, const AArgs& p, int64_t j0, int tid) {
    constexpr int NT = 64 * kFaWaves;
    k0 = ld(K, j0 + tid / CH, p.k_st, p.Tk, 8 * (tid % CH));
    if constexpr (KU > 1) k1 = ld(K, j0 + (tid + NT) / CH, p.k_st, p.Tk, 8 * (tid % CH));
    if constexpr (KU > 2) k2 = ld(K, j0 + (tid + 2 * NT) / CH, p.k_st, p.Tk, 8 * (tid % CH));
    if constexpr (KU > 3) k3 = ld(K, j0 + (tid + 3 * NT) / CH, p.k_st, p.Tk, 8 * (tid % CH));
    va0 = ld(V, j0 + 2 * (tid / CH), p.v_st, p.Tk, 8 * (tid % CH));
    vb0 = ld(V, j0 + 2 * (tid / CH) + 1, p.v_st, p.Tk, 8 * (tid % CH));
    if constexpr (VU > 1) {
      va1 = ld(V, j0 + 2 * ((tid + NT) / CH), p.v_st, p.Tk, 8 * (tid % CH));
      vb1 = ld(V, j0 + 2 * ((tid + NT) / CH) + 1, p.v_st, p.Tk, 8 * (tid % CH));
    }
  }
  template <int VP>
  __device__ __forceinline__ static void put_v(T* Vt, int e, uint4 a4, uint4 c4) {
    const int d0 = 8 * (e % CH);
    const int pos = fa_vpos(2 * (e / CH));  // even: keys 2m and 2m+1 land side by side
    const uint32_t a[4] = {a4.x, a4.y, a4.z, a4.w};
    const uint32_t c[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      *(uint32_t*)&Vt[(d0 + 2 * x) * VP + pos] = (a[x] & 0xffffu) | (c[x] << 16);
      *(uint32_t*)&Vt[(d0 + 2 * x + 1) * VP + pos] = (a[x] >> 16) | (c[x] & 0xffff0000u);
    }
  }
  template <int KP, int VP>
  __device__ __forceinline__ void store(T* Ks, T* Vt, int tid) const {
    constexpr int NT = 64 * kFaWaves;
    const int col = 8 * (tid % CH);
    *(uint4*)&Ks[(tid / CH) * KP + col] = k0;
    if constexpr (KU > 1) *(uint4*)&Ks[((tid + NT) / CH) * KP + col] = k1;
    if constexpr (KU > 2) *(uint4*)&Ks[((tid + 2 * NT) / CH) * KP + col] = k2;
    if constexpr (KU > 3) *(uint4*)&Ks[((tid + 3 * NT) / CH) * KP + col] = k3;
    put_v<VP>(Vt, tid, va0, vb0);
    if constexpr (VU > 1) put_v<VP>(Vt, tid + NT, va1, vb1);
  }
};

template <typename T, int D, int QG>
__global__ void __launch_bounds__(64 * kFaWaves) flash_attn_mfma(AArgs p) {
  static_assert(D % 64 == 0, "d must be a multiple of 64");
  typedef typename FaMfma<T>::vec V8;
  constexpr int QB = kFaWaves * QG * 16;  // query rows per block
  constexpr int KP = D + 8;               // K tile row pitch (elements)
  constexpr int VP = kFaKeys + 8;         // V^T row pitch (elements)
  constexpr int DS = D / 32;              // 32-deep steps of Q K^T
  constexpr int DT = D / 16;              // 16-dim tiles of O^T
  __shared__ __attribute__((aligned(16))) T Ks[2][kFaKeys * KP];
  __shared__ __attribute__((aligned(16))) T Vt[2][D * VP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t BH = p.B * p.H;
  const int64_t bh = blockIdx.x % BH;
  const int64_t tq = blockIdx.x / BH;
  const int64_t qt = p.causal ? p.q_tiles - 1 - tq : tq;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q0 = qt * QB;
  const int64_t qw = q0 + (int64_t)w * QG * 16;  // this wavefront's first query

  const T* Q = (const T*)p.q + b * p.q_sb + h * p.q_sh;
  const T* K = (const T*)p.k + b * p.k_sb + h * p.k_sh;
  const T* V = (const T*)p.v + b * p.v_sb + h * p.v_sh;

  int64_t kv_end = p.Tk;
  if (p.causal) {
    const int64_t qe = q0 + QB < p.Tq ? q0 + QB : p.Tq;
    kv_end = qe < p.Tk ? qe : p.Tk;
  }
  const int ntiles = (int)((kv_end + kFaKeys - 1) / kFaKeys);


  // Q operands: column l%16 of each group, dims 32s + 8g .. +8
  V8 qf[QG][DS];
  int lim[QG];  // keys < lim are visible to this lane's query
#pragma unroll
  for (int gi = 0; gi < QG; ++gi) {
    const int64_t qi = qw + 16 * gi + l16;
    const int64_t qr = qi < p.Tq ? qi : p.Tq - 1;
#pragma unroll
    for (int s = 0; s < DS; ++s) qf[gi][s] = *(const V8*)(Q + qr * p.q_st + 32 * s + 8 * g);
    lim[gi] = (int)(p.causal ? (qi + 1 < p.Tk ? qi + 1 : p.Tk) : p.Tk);
  }

  f32x4 acc[QG][DT];
  float m[QG], ls[QG];
#pragma unroll
  for (int gi = 0; gi < QG; ++gi) {
    m[gi] = -INFINITY;
    ls[gi] = 0.f;
#pragma unroll
    for (int u = 0; u < DT; ++u) acc[gi][u] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float c2 = p.scale * 1.4426950408889634f;

  if (ntiles > 0) {
    FaTile<T, D> t0;
    t0.load(K, V, p, 0, tid);
    t0.template store<KP, VP>(Ks[0], Vt[0], tid);
  }
  __syncthreads();

  // One tile: S^T, online softmax, O^T update, then the next tile's LDS
  // stores.  MASK applies the visibility test to every score; tiles wholly
  // visible to all of the block's queries skip it.  Both loop bodies are
  // branch-free, so the next tile's global loads stay at the top and are
  // in flight during the products.
  auto tile = [&](int it, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int buf = it & 1;
    const int j0 = it * kFaKeys;
    // the next tile's loads (unconditional: past the end they reread row Tk-1)
    FaTile<T, D> nx;
    nx.load(K, V, p, (int64_t)j0 + kFaKeys, tid);

    const T* Kb = Ks[buf];
    const T* Vb = Vt[buf];
    f32x4 st[QG][4];
#pragma unroll
    for (int gi = 0; gi < QG; ++gi)
#pragma unroll
      for (int t = 0; t < 4; ++t) st[gi][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const V8 a = *(const V8*)&Kb[(16 * t + l16) * KP + 32 * s + 8 * g];
#pragma unroll
        for (int gi = 0; gi < QG; ++gi) st[gi][t] = FaMfma<T>::run(a, qf[gi][s], st[gi][t]);
      }
    V8 pf[QG][2];
#pragma unroll
    for (int gi = 0; gi < QG; ++gi) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = st[gi][t][r] * c2;
          if constexpr (MASK) v = j0 + 16 * t + 4 * g + r < lim[gi] ? v : -INFINITY;
          st[gi][t][r] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m[gi], mx);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float alpha = __builtin_amdgcn_exp2f(m[gi] - mu);
      m[gi] = mn;
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = __builtin_amdgcn_exp2f(st[gi][t][r] - mu);
          ps += pv;
          pf[gi][t >> 1][4 * (t & 1) + r] = (T)pv;
        }
      ls[gi] = ls[gi] * alpha + ps;
#pragma unroll
      for (int u = 0; u < DT; ++u) acc[gi][u] *= alpha;
    }
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const V8 a = *(const V8*)&Vb[(16 * u + l16) * VP + 32 * s + 8 * g];
#pragma unroll
        for (int gi = 0; gi < QG; ++gi) acc[gi][u] = FaMfma<T>::run(a, pf[gi][s], acc[gi][u]);
      }
    // the LDS stores into the other buffer stay after this tile's LDS reads
    asm volatile("" ::: "memory");
    nx.template store<KP, VP>(Ks[buf ^ 1], Vt[buf ^ 1], tid);
    __syncthreads();
  };

  // leading tiles visible in full to every query of the block
  int nfull = (int)(p.Tk / kFaKeys);
  if (p.causal && (q0 + 1) / kFaKeys < nfull) nfull = (int)((q0 + 1) / kFaKeys);
  if (nfull > ntiles) nfull = ntiles;
  int it = 0;
  for (; it < nfull; ++it) tile(it, std::integral_constant<bool, false>());
  for (; it < ntiles; ++it) tile(it, std::integral_constant<bool, true>());

  T* O = (T*)p.o + b * p.o_sb + h * p.o_sh;
#pragma unroll
  for (int gi = 0; gi < QG; ++gi) {
    float l = ls[gi] + __shfl_xor(ls[gi], 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t qi = qw + 16 * gi + l16;
    if (qi >= p.Tq) continue;
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      T o4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o4[r] = from_f<T>(acc[gi][u][r] * inv);
      uint2 pk;
      __builtin_memcpy(&pk, o4, 8);
      *(uint2*)(O + qi * p.o_st + 16 * u + 4 * g) = pk;
    }
  }
}


// ── MFMA flash attention, fp32 ─────────────────────────────────────────────
// The 16-bit kernel's structure with v_mfma_f32_16x16x4_f32 (exact fp32
// products, fp32 accumulation): lane l's A operand is row l%16 and B operand
// column l%16 at k = l/16; C register r of lane l is row 4*(l/16)+r,
// column l%16.  The k index of each product is permuted (A and B agree), so
// that every operand a lane needs is a run of consecutive floats:
//  - S^T = K Q^T: step s gives lane group g = l/16 the dimension
//    d = g*D/4 + s, so a lane's K operands are D/4 consecutive floats of
//    one key row (16-byte LDS reads) and its query row is held the same way;
//  - O^T += V^T P^T: one product per key (t, r) of the lane's scores, B =
//    the lane's own probability; O^T row rho of 16-row tile u is dimension
//    d = (D/16)*rho + u, so a lane's V operands are D/16 consecutive floats
//    of one key row and its outputs are runs of D/16 consecutive floats.
// Both K and V tiles sit in LDS untransposed, rows padded by 4 floats.
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int D, int NSP>
struct FaTile32 {
  static constexpr int C4 = D / 4;                           // float4 chunks per row
  static constexpr int NU = kFaKeys * C4 / (64 * kFaWaves);  // chunks per thread per operand
  static_assert(NU <= 8, "tile registers");
  // named registers (with arrays the compiler kept the tile in scratch memory)
  float4 k0, k1, k2, k3, k4, k5, k6, k7, v0, v1, v2, v3, v4, v5, v6, v7;

  template <int I>
  __device__ __forceinline__ void ld1(const float* K, const float* V, const float* KB, const float* VB,
                                      const AArgs& p, int64_t j0, int tid, float4& k, float4& v) {
    if constexpr (I < NU) {
      const int e = tid + 64 * kFaWaves * I;
      const int64_t j = j0 + e / C4 < p.Tk ? j0 + e / C4 : p.Tk - 1;  // rows past Tk repeat row Tk-1
      k = ld_part4<NSP>(K + j * p.k_st + 4 * (e % C4), p.plane, KB + 4 * (e % C4));
      v = ld_part4<NSP>(V + j * p.v_st + 4 * (e % C4), p.plane, VB + 4 * (e % C4));
    }
  }
  template <int KP, int I>
  __device__ __forceinline__ void st1(float* Ks, float* Vs, int tid, const float4& k, const float4& v) const {
    if constexpr (I < NU) {
      const int e = tid + 64 * kFaWaves * I;
      *(float4*)&Ks[(e / C4) * KP + 4 * (e % C4)] = k;
      *(float4*)&Vs[(e / C4) * KP + 4 * (e % C4)] = v;
    }
  }
  __device__ __forceinline__ void load(const float* K, const float* V, const float* KB, const float* VB,
                                       const AArgs& p, int64_t j0, int tid) {
    ld1<0>(K, V, KB, VB, p, j0, tid, k0, v0); ld1<1>(K, V, KB, VB, p, j0, tid, k1, v1);
    ld1<2>(K, V, KB, VB, p, j0, tid, k2, v2); ld1<3>(K, V, KB, VB, p, j0, tid, k3, v3);
    ld1<4>(K, V, KB, VB, p, j0, tid, k4, v4); ld1<5>(K, V, KB, VB, p, j0, tid, k5, v5);
    ld1<6>(K, V, KB, VB, p, j0, tid, k6, v6); ld1<7>(K, V, KB, VB, p, j0, tid, k7, v7);
  }
  template <int KP>
  __device__ __forceinline__ void store(float* Ks, float* Vs, int tid) const {
    st1<KP, 0>(Ks, Vs, tid, k0, v0); st1<KP, 1>(Ks, Vs, tid, k1, v1);
    st1<KP, 2>(Ks, Vs, tid, k2, v2); st1<KP, 3>(Ks, Vs, tid, k3, v3);
    st1<KP, 4>(Ks, Vs, tid, k4, v4); st1<KP, 5>(Ks, Vs, tid, k5, v5);
    st1<KP, 6>(Ks, Vs, tid, k6, v6); st1<KP, 7>(Ks, Vs, tid, k7, v7);
  }
};

// The end of the key-split kernels: wavefronts 1..3 hand their running
// maximum, sum and output to wavefront 0 through LDS (`red`: 3 * 64 *
// (D/4 + 2) floats), which rescales and adds them in wavefront order.
// Returns false on the wavefronts that handed theirs over.
template <int D>
__device__ __forceinline__ bool fa32_merge(float* red, int w, int lane, float m, float& l, f32x4v (&acc)[D / 16]) {
  constexpr int DT = D / 16;
  constexpr int PER = DT * 4 + 2;
  if (w > 0) {
    float* dst = red + ((w - 1) * 64 + lane) * PER;
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[u * 4 + r] = acc[u][r];
    dst[DT * 4] = m;
    dst[DT * 4 + 1] = l;
  }
  __syncthreads();
  if (w > 0) return false;
  float mw[kFaWaves], lw[kFaWaves];
  mw[0] = m;
  lw[0] = l;
#pragma unroll
  for (int v = 1; v < kFaWaves; ++v) {
    const float* src = red + ((v - 1) * 64 + lane) * PER;
    mw[v] = src[DT * 4];
    lw[v] = src[DT * 4 + 1];
  }
  float M = mw[0];
#pragma unroll
  for (int v = 1; v < kFaWaves; ++v) M = fmaxf(M, mw[v]);
  const float Mu = M == -INFINITY ? 0.f : M;
  float sc[kFaWaves];
  l = 0.f;
#pragma unroll
  for (int v = 0; v < kFaWaves; ++v) {
    sc[v] = __builtin_amdgcn_exp2f(mw[v] - Mu);
    l += lw[v] * sc[v];
  }
#pragma unroll
  for (int u = 0; u < DT; ++u) acc[u] *= sc[0];
#pragma unroll
  for (int v = 1; v < kFaWaves; ++v) {
    const float* src = red + ((v - 1) * 64 + lane) * PER;
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[u][r] += src[u * 4 + r] * sc[v];
  }
  return true;
}

// Query row qi's output from the lane's O^T registers (register r of tile u:
// dimension (D/16)*(4g + r) + u), divided by the softmax sum l: fp32, or
// packed x3 rows when p.o_pk is set.
template <int D>
__device__ __forceinline__ void fa32_store(const AArgs& p, int64_t b, int64_t h, int64_t qi, int g, float l,
                                           const f32x4v (&acc)[D / 16]) {
  constexpr int DT = D / 16;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (qi >= p.Tq) return;
  float* O = (float*)p.o + b * p.o_sb + h * p.o_sh + qi * p.o_st;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float o[DT];
#pragma unroll
    for (int u = 0; u < DT; ++u) o[u] = acc[u][r] * inv;
#pragma unroll
    for (int u = 0; u < DT; u += 4) {
      if (p.o_pk) {
        const float o4[4] = {o[u], o[u + 1], o[u + 2], o[u + 3]};
        x3_store4(p.o_pk, p.H * D / 16, b * p.Tq + qi, h * D + DT * (4 * g + r) + u, o4);
      } else {
        *(float4*)(O + DT * (4 * g + r) + u) = make_float4(o[u], o[u + 1], o[u + 2], o[u + 3]);
      }
    }
  }
}

// KSPLIT: the block's 4 wavefronts share one group of 16 queries and split
// every key tile four ways (wavefront w takes its keys 16w..16w+15), then
// merge their running maxima, sums and outputs through LDS.  Used when there
// are too few 64-query blocks to fill the GPU (GPT-2 at 128 tokens: 24):
// each wavefront then does a quarter of the serial work.  At D = 64 that
// case runs flash_attn_f32_kr below instead, with its operands in registers.
// NSP > 0: Q, K and V are read as split-K partials plus bias (ld_part4).
template <int D, bool KSPLIT, int NSP>
__global__ void __launch_bounds__(64 * kFaWaves) flash_attn_f32(AArgs p) {
  static_assert(D % 64 == 0, "d must be a multiple of 64");
  if (prefetch_block(p.pf)) return;
  constexpr int QB_ROWS = KSPLIT ? 16 : kFaWaves * 16;  // query rows per block
  constexpr int NT = KSPLIT ? 1 : 4;  // 16-key sub-tiles per wavefront and tile (KSPLIT: sub-tile w)
  constexpr int KP = D + 4;          // K and V tile row pitch (floats)
  constexpr int DS = D / 4;          // 4-deep steps of Q K^T
  constexpr int DT = D / 16;         // 16-row tiles of O^T
  __shared__ __attribute__((aligned(16))) float Ks[2][kFaKeys * KP];
  __shared__ __attribute__((aligned(16))) float Vs[2][kFaKeys * KP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t BH = p.B * p.H;
  const int64_t bh = blockIdx.x % BH;
  const int64_t tq = blockIdx.x / BH;
  const int64_t qt = p.causal ? p.q_tiles - 1 - tq : tq;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q0 = qt * QB_ROWS;
  const int64_t qw = KSPLIT ? q0 : q0 + (int64_t)w * 16;
  const int tw = KSPLIT ? w : 0;  // first key sub-tile of this wavefront

  const float* Q = (const float*)p.q + b * p.q_sb + h * p.q_sh;
  const float* K = (const float*)p.k + b * p.k_sb + h * p.k_sh;
  const float* V = (const float*)p.v + b * p.v_sb + h * p.v_sh;
  // per-head bias (NSP > 0 only; otherwise unused, any legal address)
  const float* QB = NSP > 0 ? p.qb + h * p.b_sh : Q;
  const float* KB = NSP > 0 ? p.kb + h * p.b_sh : K;
  const float* VB = NSP > 0 ? p.vb + h * p.b_sh : V;

  int64_t kv_end = p.Tk;
  if (p.causal) {
    const int64_t qe = q0 + QB_ROWS < p.Tq ? q0 + QB_ROWS : p.Tq;
    kv_end = qe < p.Tk ? qe : p.Tk;
  }
  const int ntiles = (int)((kv_end + kFaKeys - 1) / kFaKeys);

  // query row l16 of this wavefront, dims g*DS .. g*DS + DS-1
  const int64_t qi = qw + l16;
  const int64_t qr = qi < p.Tq ? qi : p.Tq - 1;
  float qf[DS];
#pragma unroll
  for (int s = 0; s < DS; s += 4) {
    const float4 x = ld_part4<NSP>(Q + qr * p.q_st + g * DS + s, p.plane, QB + g * DS + s);
    qf[s] = x.x; qf[s + 1] = x.y; qf[s + 2] = x.z; qf[s + 3] = x.w;
  }
  const int lim = (int)(p.causal ? (qi + 1 < p.Tk ? qi + 1 : p.Tk) : p.Tk);

  f32x4v acc[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) acc[u] = f32x4v{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, ls = 0.f;
  const float c2 = p.scale * 1.4426950408889634f;

  if (ntiles > 0) {
    FaTile32<D, NSP> t0;
    t0.load(K, V, KB, VB, p, 0, tid);
    t0.template store<KP>(Ks[0], Vs[0], tid);
  }
  __syncthreads();

  auto tile = [&](int it, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int buf = it & 1;
    const int j0 = it * kFaKeys;
    // the next tile, in plain local registers (held in a struct, the tile
    // went to scratch memory once a scheduling barrier followed its loads)
    constexpr int NU = FaTile32<D, NSP>::NU;
    float4 k0, k1, k2, k3, k4, k5, k6, k7, v0, v1, v2, v3, v4, v5, v6, v7;
#define AGPU_FA32_LD(I)                                                                    \
    if constexpr (I < NU) {                                                                \
      const int e = tid + 64 * kFaWaves * I;                                               \
      const int64_t jn = (int64_t)j0 + kFaKeys + e / (D / 4);                              \
      const int64_t jc = jn < p.Tk ? jn : p.Tk - 1;                                        \
      k##I = ld_part4<NSP>(K + jc * p.k_st + 4 * (e % (D / 4)), p.plane, KB + 4 * (e % (D / 4))); \
      v##I = ld_part4<NSP>(V + jc * p.v_st + 4 * (e % (D / 4)), p.plane, VB + 4 * (e % (D / 4))); \
    }
    AGPU_FA32_LD(0) AGPU_FA32_LD(1) AGPU_FA32_LD(2) AGPU_FA32_LD(3)
    AGPU_FA32_LD(4) AGPU_FA32_LD(5) AGPU_FA32_LD(6) AGPU_FA32_LD(7)
#undef AGPU_FA32_LD
    // keep the loads here, ahead of the products (the scheduler otherwise
    // sinks them next to the LDS stores, where they are waited for at once)
    __builtin_amdgcn_sched_barrier(0);

    const float* Kb = Ks[buf];
    const float* Vb = Vs[buf];
    f32x4v st[NT];
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) {
      const int t = tw + ti;
      st[ti] = f32x4v{0.f, 0.f, 0.f, 0.f};
      const float* kr = Kb + (16 * t + l16) * KP + g * DS;
#pragma unroll
      for (int s = 0; s < DS; s += 4) {
        const float4 a = *(const float4*)(kr + s);
        st[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, qf[s], st[ti], 0, 0, 0);
        st[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, qf[s + 1], st[ti], 0, 0, 0);
        st[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, qf[s + 2], st[ti], 0, 0, 0);
        st[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, qf[s + 3], st[ti], 0, 0, 0);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int ti = 0; ti < NT; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = st[ti][r] * c2;
        if constexpr (MASK) v = j0 + 16 * (tw + ti) + 4 * g + r < lim ? v : -INFINITY;
        st[ti][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - mu);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int ti = 0; ti < NT; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(st[ti][r] - mu);
        ps += pv;
        st[ti][r] = pv;
      }
    ls = ls * alpha + ps;
#pragma unroll
    for (int u = 0; u < DT; ++u) acc[u] *= alpha;
#pragma unroll
    for (int ti = 0; ti < NT; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vr = Vb + (16 * (tw + ti) + 4 * g + r) * KP + DT * l16;
        float a[DT];
#pragma unroll
        for (int u = 0; u < DT; u += 4) {
          const float4 x = *(const float4*)(vr + u);
          a[u] = x.x; a[u + 1] = x.y; a[u + 2] = x.z; a[u + 3] = x.w;
        }
#pragma unroll
        for (int u = 0; u < DT; ++u) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], st[ti][r], acc[u], 0, 0, 0);
      }
#define AGPU_FA32_ST(I)                                                                    \
    if constexpr (I < NU) {                                                                \
      const int e = tid + 64 * kFaWaves * I;                                               \
      *(float4*)&Ks[buf ^ 1][(e / (D / 4)) * KP + 4 * (e % (D / 4))] = k##I;               \
      *(float4*)&Vs[buf ^ 1][(e / (D / 4)) * KP + 4 * (e % (D / 4))] = v##I;               \
    }
    AGPU_FA32_ST(0) AGPU_FA32_ST(1) AGPU_FA32_ST(2) AGPU_FA32_ST(3)
    AGPU_FA32_ST(4) AGPU_FA32_ST(5) AGPU_FA32_ST(6) AGPU_FA32_ST(7)
#undef AGPU_FA32_ST
    __syncthreads();
  };

  int nfull = (int)(p.Tk / kFaKeys);
  if (p.causal && (q0 + 1) / kFaKeys < nfull) nfull = (int)((q0 + 1) / kFaKeys);
  if (nfull > ntiles) nfull = ntiles;
  int it = 0;
  for (; it < nfull; ++it) tile(it, std::integral_constant<bool, false>());
  for (; it < ntiles; ++it) tile(it, std::integral_constant<bool, true>());

  float l = ls + __shfl_xor(ls, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if constexpr (KSPLIT) {
    // the tile buffers are free after the loop's last barrier
    if (!fa32_merge<D>(&Ks[0][0], w, lane, m, l, acc)) return;
  }
  fa32_store<D>(p, b, h, qi, g, l, acc);
}

// Key-split fp32 attention with register operands (D = 64): the case of
// flash_attn_f32<64, true, NSP> without its LDS tiles.  Wavefront w of the
// block takes the 16-key sub-tiles w, w+4, w+8, ... of the block's 16
// queries, which is the share of every 64-key tile it takes there, so no
// sub-tile is read by two wavefronts: each loads its K and V operands from
// global memory straight into registers, the next sub-tile's loads in
// flight while the current one's products run, and the block meets only
// for the merge.  The products, masks and online-softmax updates are the
// LDS kernel's, in the same order.
template <int NSP>
__global__ void __launch_bounds__(64 * kFaWaves) flash_attn_f32_kr(AArgs p) {
  if (prefetch_block(p.pf)) return;
  constexpr int D = 64, DS = D / 4, DT = D / 16;
  __shared__ __attribute__((aligned(16))) float red[(kFaWaves - 1) * 64 * (DT * 4 + 2)];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t BH = p.B * p.H;
  const int64_t bh = blockIdx.x % BH;
  const int64_t tq = blockIdx.x / BH;
  const int64_t qt = p.causal ? p.q_tiles - 1 - tq : tq;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q0 = qt * 16;

  const float* Q = (const float*)p.q + b * p.q_sb + h * p.q_sh;
  const float* K = (const float*)p.k + b * p.k_sb + h * p.k_sh;
  const float* V = (const float*)p.v + b * p.v_sb + h * p.v_sh;
  const float* QB = NSP > 0 ? p.qb + h * p.b_sh : Q;
  const float* KB = NSP > 0 ? p.kb + h * p.b_sh : K;
  const float* VB = NSP > 0 ? p.vb + h * p.b_sh : V;

  int64_t kv_end = p.Tk;
  if (p.causal) {
    const int64_t qe = q0 + 16 < p.Tq ? q0 + 16 : p.Tq;
    kv_end = qe < p.Tk ? qe : p.Tk;
  }
  const int nsub = (int)((kv_end + 15) / 16);

  // sub-tile t's operands of this lane: K row 16t + l16, dims 16g .. 16g+15;
  // V rows 16t + 4g + r (r = 0..3), dims 4*l16 .. 4*l16+3 (rows past Tk
  // repeat row Tk-1 and are masked)
  float4 ka0, ka1, ka2, ka3, va0, va1, va2, va3;
  float4 kb0, kb1, kb2, kb3, vb0, vb1, vb2, vb3;
#define AGPU_FA32R_LD(S, t)                                                                 \
  {                                                                                         \
    const int64_t jk = 16 * (int64_t)(t) + l16 < p.Tk ? 16 * (int64_t)(t) + l16 : p.Tk - 1; \
    const float* kr = K + jk * p.k_st + DS * g;                                             \
    k##S##0 = ld_part4<NSP>(kr, p.plane, KB + DS * g);                                      \
    k##S##1 = ld_part4<NSP>(kr + 4, p.plane, KB + DS * g + 4);                              \
    k##S##2 = ld_part4<NSP>(kr + 8, p.plane, KB + DS * g + 8);                              \
    k##S##3 = ld_part4<NSP>(kr + 12, p.plane, KB + DS * g + 12);                            \
    const int64_t jv = 16 * (int64_t)(t) + 4 * g;                                           \
    const float* vr = V + DT * l16;                                                         \
    v##S##0 = ld_part4<NSP>(vr + (jv < p.Tk ? jv : p.Tk - 1) * p.v_st, p.plane, VB + DT * l16);         \
    v##S##1 = ld_part4<NSP>(vr + (jv + 1 < p.Tk ? jv + 1 : p.Tk - 1) * p.v_st, p.plane, VB + DT * l16); \
    v##S##2 = ld_part4<NSP>(vr + (jv + 2 < p.Tk ? jv + 2 : p.Tk - 1) * p.v_st, p.plane, VB + DT * l16); \
    v##S##3 = ld_part4<NSP>(vr + (jv + 3 < p.Tk ? jv + 3 : p.Tk - 1) * p.v_st, p.plane, VB + DT * l16); \
  }
  if (w < nsub) AGPU_FA32R_LD(a, w)

  // query row l16, dims 16g .. 16g+15
  const int64_t qi = q0 + l16;
  const int64_t qr = qi < p.Tq ? qi : p.Tq - 1;
  float qf[DS];
#pragma unroll
  for (int s = 0; s < DS; s += 4) {
    const float4 x = ld_part4<NSP>(Q + qr * p.q_st + g * DS + s, p.plane, QB + g * DS + s);
    qf[s] = x.x; qf[s + 1] = x.y; qf[s + 2] = x.z; qf[s + 3] = x.w;
  }
  const int lim = (int)(p.causal ? (qi + 1 < p.Tk ? qi + 1 : p.Tk) : p.Tk);

  f32x4v acc[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) acc[u] = f32x4v{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, ls = 0.f;
  const float c2 = p.scale * 1.4426950408889634f;

  auto sub = [&](int t, const float4& k0, const float4& k1, const float4& k2, const float4& k3, const float4& v0,
                 const float4& v1, const float4& v2, const float4& v3) {
    f32x4v st = f32x4v{0.f, 0.f, 0.f, 0.f};
    const float4 kk[4] = {k0, k1, k2, k3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[i].x, qf[4 * i], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[i].y, qf[4 * i + 1], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[i].z, qf[4 * i + 2], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[i].w, qf[4 * i + 3], st, 0, 0, 0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = st[r] * c2;
      v = 16 * t + 4 * g + r < lim ? v : -INFINITY;
      st[r] = v;
      mx = fmaxf(mx, v);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - mu);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pv = __builtin_amdgcn_exp2f(st[r] - mu);
      ps += pv;
      st[r] = pv;
    }
    ls = ls * alpha + ps;
#pragma unroll
    for (int u = 0; u < DT; ++u) acc[u] *= alpha;
    const float4 vv[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r].x, st[r], acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r].y, st[r], acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r].z, st[r], acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r].w, st[r], acc[3], 0, 0, 0);
    }
  };

  for (int t = w; t < nsub; t += 2 * kFaWaves) {
    if (t + kFaWaves < nsub) AGPU_FA32R_LD(b, t + kFaWaves)
    __builtin_amdgcn_sched_barrier(0);
    sub(t, ka0, ka1, ka2, ka3, va0, va1, va2, va3);
    if (t + kFaWaves >= nsub) break;
    if (t + 2 * kFaWaves < nsub) AGPU_FA32R_LD(a, t + 2 * kFaWaves)
    __builtin_amdgcn_sched_barrier(0);
    sub(t + kFaWaves, kb0, kb1, kb2, kb3, vb0, vb1, vb2, vb3);
  }
#undef AGPU_FA32R_LD

  float l = ls + __shfl_xor(ls, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (!fa32_merge<D>(red, w, lane, m, l, acc)) return;
  fa32_store<D>(p, b, h, qi, g, l, acc);
}
}  // namespace

// 16-byte loads of every Q/K/V row and 8-byte stores of O need aligned bases
// and row/head/batch strides that are multiples of 8 elements.
static bool attention_mfma_ok(const Attn& a) {
  if (!(a.dt == DType::F16 || a.dt == DType::BF16 || a.dt == DType::F32) || !(a.D == 64 || a.D == 128)) return false;
  if (a.Tk >= (int64_t(1) << 30)) return false;  // key indices are 32-bit in the kernel
  if (((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v) % 16 != 0 || (uintptr_t)a.o % 8 != 0) return false;
  const int64_t st[12] = {a.q_sb, a.q_sh, a.q_st, a.k_sb, a.k_sh, a.k_st,
                          a.v_sb, a.v_sh, a.v_st, a.o_sb, a.o_sh, a.o_st};
  for (int64_t x : st)
    if (x % 8 != 0) return false;  // fp32: 4 would do; 8 keeps one rule
  return true;
}

template <typename T>
static void launch_fa_mfma(const AArgs& p, int64_t D, bool wide, unsigned blocks, hipStream_t s) {
  const dim3 grid(blocks), block(64 * kFaWaves);
  if (D == 64) {
    if (wide) hipLaunchKernelGGL((flash_attn_mfma<T, 64, 2>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((flash_attn_mfma<T, 64, 1>), grid, block, 0, s, p);
  } else {
    if (wide) hipLaunchKernelGGL((flash_attn_mfma<T, 128, 2>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((flash_attn_mfma<T, 128, 1>), grid, block, 0, s, p);
  }
}

template <bool KS, int D>
static void launch_fa32_d(const AArgs& p, int nsp, unsigned blocks, hipStream_t s) {
  const dim3 grid(blocks), block(64 * kFaWaves);
  switch (nsp) {
    case 0: hipLaunchKernelGGL((flash_attn_f32<D, KS, 0>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((flash_attn_f32<D, KS, 2>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((flash_attn_f32<D, KS, 4>), grid, block, 0, s, p); break;
    case 8: hipLaunchKernelGGL((flash_attn_f32<D, KS, 8>), grid, block, 0, s, p); break;
    default: fail("fused attention: %d projection partials (2, 4 or 8 supported)", nsp);
  }
}

static void launch_fa32_kr(const AArgs& p, int nsp, unsigned blocks, hipStream_t s) {
  const dim3 grid(blocks), block(64 * kFaWaves);
  switch (nsp) {
    case 0: hipLaunchKernelGGL((flash_attn_f32_kr<0>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((flash_attn_f32_kr<2>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((flash_attn_f32_kr<4>), grid, block, 0, s, p); break;
    case 8: hipLaunchKernelGGL((flash_attn_f32_kr<8>), grid, block, 0, s, p); break;
    default: fail("fused attention: %d projection partials (2, 4 or 8 supported)", nsp);
  }
}

template <bool KS>
static void launch_fa32(const AArgs& p0, const Attn& a, unsigned blocks, hipStream_t s) {
  AArgs p = p0;
  p.pf = make_prefetch((int)blocks, 64 * kFaWaves);
  blocks += (unsigned)p.pf.blocks;
  // key split at D = 64: operands in registers (GPT-2 small forward
  // 0.6129 -> 0.6039 ms against the LDS-tiled kernel, A/B on one box)
  if (a.D != 64) launch_fa32_d<KS, 128>(p, a.nsplit, blocks, s);
  else if constexpr (KS) launch_fa32_kr(p, a.nsplit, blocks, s);
  else launch_fa32_d<false, 64>(p, a.nsplit, blocks, s);
}

bool attention_partials_ok(const Attn& a) { return a.dt == DType::F32 && attention_mfma_ok(a); }

bool attention_supported(const Attn& a) {
  return (a.D == 64 || a.D == 128 || a.D == 32) && (a.dt == DType::F32 || a.dt == DType::F16 || a.dt == DType::BF16);
}

void attention(const Attn& a, hipStream_t s) {
  if (!attention_supported(a)) fail("fused attention: head dim %lld not supported", (long long)a.D);
  if (a.B * a.H * a.Tq == 0) return;
  AArgs p{};
  p.q = a.q; p.k = a.k; p.v = a.v; p.o = a.o;
  p.B = a.B; p.H = a.H; p.Tq = a.Tq; p.Tk = a.Tk;
  p.q_sb = a.q_sb; p.q_sh = a.q_sh; p.q_st = a.q_st;
  p.k_sb = a.k_sb; p.k_sh = a.k_sh; p.k_st = a.k_st;
  p.v_sb = a.v_sb; p.v_sh = a.v_sh; p.v_st = a.v_st;
  p.o_sb = a.o_sb; p.o_sh = a.o_sh; p.o_st = a.o_st;
  p.scale = a.scale;
  p.causal = a.causal ? 1 : 0;
  p.qb = (const float*)a.qb; p.kb = (const float*)a.kb; p.vb = (const float*)a.vb;
  p.b_sh = a.b_sh; p.plane = a.plane;
  p.o_pk = (bf16_t*)a.o_pk;
  if (a.nsplit > 0 && !attention_partials_ok(a)) fail("fused attention: projection partials need the fp32 MFMA kernel");
  if (a.o_pk && !(attention_mfma_ok(a) && a.dt == DType::F32 && (a.H * a.D) % 16 == 0 && ((uintptr_t)a.o_pk & 15) == 0))
    fail("fused attention: packed-row output needs the fp32 MFMA kernel and H*D %% 16 == 0");
  if (attention_mfma_ok(a) && a.dt == DType::F32) {
    // 64 queries per block when that gives every CU a block; else 16 per
    // block with the key tiles split across the block's wavefronts
    const bool ksplit = a.B * a.H * ((a.Tq + 63) / 64) < 256;
    p.q_tiles = (int)((a.Tq + (ksplit ? 15 : 63)) / (ksplit ? 16 : 64));
    const int64_t blocks = a.B * a.H * p.q_tiles;
    if (blocks > 0x7fffffff) fail("fused attention: grid too large");
    if (ksplit) {
      launch_fa32<true>(p, a, (unsigned)blocks, s);
      check_launch("attention");
      return;
    }
    launch_fa32<false>(p, a, (unsigned)blocks, s);
    check_launch("attention");
    return;
  }
  if (attention_mfma_ok(a)) {
    // 128 query rows per block when that still gives every CU a block
    const int64_t bh = a.B * a.H;
    const bool wide = bh * ((a.Tq + 127) / 128) >= 256;
    const int qb = wide ? 128 : 64;
    p.q_tiles = (int)((a.Tq + qb - 1) / qb);
    const int64_t blocks = bh * p.q_tiles;
    if (blocks > 0x7fffffff) fail("fused attention: grid too large");
    if (a.dt == DType::F16) launch_fa_mfma<half_t>(p, a.D, wide, (unsigned)blocks, s);
    else launch_fa_mfma<bf16_t>(p, a.D, wide, (unsigned)blocks, s);
    check_launch("attention");
    return;
  }
  p.q_tiles = (int)((a.Tq + kQT - 1) / kQT);
  int64_t blocks = a.B * a.H * p.q_tiles;
  if (blocks > 0x7fffffff) fail("fused attention: grid too large");
  AGPU_FLOAT_SWITCH(a.dt, {
    if (a.D == 64) hipLaunchKernelGGL((flash_attn<T, 64>), dim3((unsigned)blocks), dim3(256), 0, s, p);
    else if (a.D == 128) hipLaunchKernelGGL((flash_attn<T, 128>), dim3((unsigned)blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((flash_attn<T, 32>), dim3((unsigned)blocks), dim3(256), 0, s, p);
  });
  check_launch("attention");
}

}  // namespace k
}  // namespace agpu
