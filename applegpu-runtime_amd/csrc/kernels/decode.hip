// Decode-time attention over a preallocated KV cache, and the in-place append
// that fills it.
//
// The reference decodes by concatenating each step's K/V rows onto the
// previous cache (python/applegpu_runtime/models/gpt2.py:122-126: a fresh copy
// of the whole cache, per layer, per step) and then running non-causal
// attention of the one new query over it (gpt2.py:132-135 through
// crates/core/src/ops.rs:1531-1620).  Here each layer's cache is one
// [B, H, Tmax, D] allocation: kv_write stores the new rows at each sequence's
// position, read from device memory, and decode_attention reads each
// sequence's length from device memory.  Nothing a decode step launches then
// depends on a host-side length, so the step can be recorded once as a HIP
// graph and replayed for every token.
//
// decode_attention: within a block, D/8 lanes own one key, 8 elements each
// (one 16-byte load for 16-bit types), so a wave covers 64/(D/8) keys per
// step and the dot product is log2(D/8) xor shuffles; each key group keeps an
// online softmax (running max, sum and output), and the groups and waves of
// the block merge their states at the end.  With enough (batch, head, query
// row) rows for the CUs a 16-wave block owns a whole row; otherwise the key
// axis is split over blocks (split-KV), each leaving an unnormalised partial
// (max, sum, acc[D]) that a second kernel merges.  A row with no visible key
// gets zeros (the fused attention kernel uses the same convention).
#include "device.hpp"

#include <cstdlib>
#include <type_traits>
#include <cstring>

namespace agpu {
namespace k {
using namespace dev;

namespace {

// Two shapes of decode block: with enough (batch, head, query) rows to fill
// the CUs, one 16-wave block per row covers the whole context (no partials,
// no merge launch); with few rows, 4-wave blocks split the context and
// decode_merge combines their partials.
constexpr int kDRowsWhole = 128;          // rows at which a block takes a whole row
constexpr int kDWavesWhole = 16, kDUnrollWhole = 4, kDUnrollWhole6 = 6;
constexpr int kDWavesSplit = 4, kDUnrollSplit = 2;

struct DArgs {
  const void* q; const void* k; const void* v; void* o;
  const int32_t* lens;
  float* part;  // [rows][splits][D + 2]: acc[D], max, sum (unused when splits == 1)
  int64_t H, Tq, Tmax;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale;
  int splits, chunk;
  // append (Tq == 1): the new K and V rows [B, H, 1, D] (strides per batch
  // and head); they become cache row lens[b] - 1
  const void* kn; const void* vn;
  int64_t kn_sb, kn_sh, vn_sb, vn_sh;
  // read-ahead blocks (whole-row launches): rows pf.first .. of the grid's y
  PfArgs pf;
};

// 8 consecutive elements, raw: one 16-byte load (two for fp32) when VEC.
// Loads are issued into raw registers and converted where they are used, so
// a wave's loads of one iteration are all in flight together (converting at
// the load makes the compiler wait for each load before the next).
template <typename T, bool VEC>
struct Raw8 {
  static constexpr int NV = VEC ? (int)sizeof(T) / 2 : 1;  // uint4s per 8 elements
  uint4 v[NV];
  T s[VEC ? 1 : 8];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NV; ++i) v[i] = ((const uint4*)p)[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] = p[i];
    }
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NV; ++i) ((uint4*)p)[i] = v[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = s[i];
    }
  }
  __device__ __forceinline__ void to_float(float (&x)[8]) const {
    if constexpr (VEC) {
      T e[8];
      __builtin_memcpy(e, v, 16 * NV);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = to_f(e[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = to_f(s[i]);
    }
  }
};

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));

// q . k over 8 elements with fp32 accumulation: four v_dot2_f32_{f16,bf16}
// on raw 16-bit pairs (products exact in fp32, no conversions), else FMAs.
template <typename T, bool VEC>
__device__ __forceinline__ float dot8(const Raw8<T, VEC>& q, const Raw8<T, VEC>& k) {
  if constexpr (VEC && std::is_same<T, half_t>::value) {
    h2_t a[4], b[4];
    __builtin_memcpy(a, q.v, 16);
    __builtin_memcpy(b, k.v, 16);
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) d = __builtin_amdgcn_fdot2(a[i], b[i], d, false);
    return d;
  } else if constexpr (VEC && std::is_same<T, bf16_t>::value) {
    b2_t a[4], b[4];
    __builtin_memcpy(a, q.v, 16);
    __builtin_memcpy(b, k.v, 16);
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) d = __builtin_amdgcn_fdot2_f32_bf16(a[i], b[i], d, false);
    return d;
  } else {
    float x[8], y[8];
    q.to_float(x);
    k.to_float(y);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d += x[e] * y[e];
    return d;
  }
}

// Sum over aligned groups of G lanes (G = 2, 4, 8, 16) with DPP lane moves
// (VALU operand modifiers, no LDS round trip): quad_perm swaps for lane
// distance 1 and 2, row_half_mirror (lane i <-> 7-i in each 8) and
// row_mirror (i <-> 15-i in each 16) for the halves of 8- and 16-lane
// groups, each applied once the smaller groups already hold their sums.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (G >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror
  if constexpr (G >= 16) v += dpp_mov<0x140>(v); // row_mirror
  return v;
}

template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T* p, float (&x)[8]) {
  Raw8<T, VEC> r;
  r.load(p);
  r.to_float(x);
}

// Number of keys visible to query row i of a sequence holding `len` keys
// whose last Tq entries are the queries themselves: keys j <= len - Tq + i.
__device__ __forceinline__ int64_t visible_keys(const DArgs& p, int64_t b, int64_t i) {
  int64_t len = p.lens[b];
  len = len < 0 ? 0 : (len > p.Tmax ? p.Tmax : len);
  int64_t vis = len - p.Tq + i + 1;
  return vis < 0 ? 0 : (vis > len ? len : vis);
}

// Merges online-softmax state (om, ol, oa) into (m, l, a); maxima are in the
// log2 domain.
__device__ __forceinline__ void merge_state(float& m, float& l, float (&a)[8], float om, float ol,
                                            const float (&oa)[8]) {
  const float M = fmaxf(m, om);
  if (M == -INFINITY) return;  // both empty
  const float f1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
  const float f2 = om == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(om - M);
  l = l * f1 + ol * f2;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = a[e] * f1 + oa[e] * f2;
  m = M;
}

// NW waves per block, UN key steps in flight per wave.  NEW (Tq == 1): the
// step's own K/V row comes in beside the cache as key lens[b] - 1; the block
// whose key range holds that key scores it from the new rows and stores it
// into the cache, so the append costs no launch of its own.
template <typename T, int D, bool VEC, int NW, int UN, bool NEW>
__global__ void __launch_bounds__(64 * NW) decode_attn(DArgs p) {
  constexpr int LPK = D / 8;           // lanes per key
  constexpr int KPS = 64 / LPK;        // keys per wave step
  constexpr int BS = NW * KPS * UN;    // keys per block iteration
  __shared__ float sm_acc[NW][D];
  __shared__ float sm_m[NW], sm_l[NW];

  if ((int)blockIdx.y >= p.pf.first) {
    prefetch_lines(p.pf, (int64_t)blockIdx.y - p.pf.first);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane / LPK, sub = lane % LPK;
  const int s = blockIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t i = row % p.Tq, bh = row / p.Tq;
  const int64_t h = bh % p.H, b = bh / p.H;
  const int64_t j_lo = (int64_t)s * p.chunk;

  // Scores are kept in the log2 domain (scale * log2(e) folded into one
  // multiply) so every exponential is one v_exp_f32.
  Raw8<T, VEC> qr;
  qr.load((const T*)p.q + b * p.q_sb + h * p.q_sh + i * p.q_st + sub * 8);
  const float c2 = p.scale * 1.4426950408889634f;
  const T* K = (const T*)p.k + b * p.k_sb + h * p.k_sh + sub * 8;
  const T* V = (const T*)p.v + b * p.v_sb + h * p.v_sh + sub * 8;
  const int tmax = (int)p.Tmax, kst = (int)p.k_st, vst = (int)p.v_st;
  int jnew = -1;  // NEW: cache row of the new K/V row, -1 for none

  // Raw K/V rows of one iteration, clamped into the cache (always legal) and
  // masked when scored.
  Raw8<T, VEC> kr[UN], vr[UN];
  auto load_range = [&](int64_t base, int u0, int u1, int rows) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      if (u < u0 || u >= u1) continue;
      const int j = (int)base + (u * NW + w) * KPS + g;
      const int jc = j < rows ? j : rows - 1;
      kr[u].load(K + jc * kst);   // 32-bit offsets: Tmax * stride < 2^31 (checked on the host)
      vr[u].load(V + jc * vst);
    }
  };
  auto load_iter = [&](int64_t base) __attribute__((always_inline)) { load_range(base, 0, UN, tmax); };
  // The first half of the first iteration's batches go out before the
  // sequence length is read, so that the two latencies overlap; the second
  // half after it, clamped to the last scored row, so that rows past the
  // context (up to Tmax) are not fetched from HBM (C4 decode step at context
  // 513-640: 1.2556 -> 1.2450 ms against loading every batch up to Tmax
  // first; issuing 1, 2, 3 or 4 of the 6 batches early measured the same).
  constexpr int UE = UN >= 2 ? UN / 2 : UN;
  load_range(j_lo, 0, UE, tmax);
  const int64_t vis = visible_keys(p, b, i);
  int64_t j_hi = j_lo + p.chunk < vis ? j_lo + p.chunk : vis;
  if constexpr (NEW) {
    // The new row is key lens[b] - 1, the last visible one.  A length
    // outside [1, Tmax] names no cache row: the new row is then neither
    // scored nor stored (kv_write drops such rows) and attention sees the
    // cache as it is.  Otherwise the loop stops short of it.
    const int64_t lb = p.lens[b];
    jnew = (lb >= 1 && lb <= p.Tmax) ? (int)lb - 1 : -1;
    if (jnew >= 0 && j_hi > jnew) j_hi = jnew;
  }
  if constexpr (UE < UN) {
    // the later batches: rows past the scored range re-read its last row
    const int rows = j_hi > 0 ? (int)j_hi : 1;
    load_range(j_lo, UE, UN, rows < tmax ? rows : tmax);
  }
  float m = -INFINITY, l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;

  for (int64_t base = j_lo; base < j_hi; base += BS) {
    // the iteration's scores, then one online-softmax rescale for all of them
    const int64_t lim = j_hi - base;
    float sc[UN];
    float mx = m;
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const float d = group_sum<LPK>(dot8(qr, kr[u]));
      sc[u] = (u * NW + w) * KPS + g < lim ? d * c2 : -INFINITY;
      mx = fmaxf(mx, sc[u]);
    }
    const float alpha = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mx);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      // A masked key (past the visible length, or a clamped address) adds
      // nothing, whatever its cache row holds: a NaN or Inf left in an
      // unused row must not reach the output through 0 * v.
      const bool live = sc[u] != -INFINITY;
      const float pe = live ? __builtin_amdgcn_exp2f(sc[u] - mx) : 0.f;
      l += pe;
      float vx[8];
      vr[u].to_float(vx);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = live ? fmaf(pe, vx[e], acc[e]) : acc[e];
    }
    m = mx;
    if (base + BS < j_hi) load_iter(base + BS);
  }

  if constexpr (NEW) {
    // The block whose key range holds the new row: key group 0 of wave 0
    // adds it as one more online-softmax term, and its lanes (8 dims each)
    // store it into the cache.  No wave reads cache row jnew unmasked, so
    // the store races with nothing that counts.
    if (w == 0 && jnew >= j_lo && jnew < j_lo + p.chunk) {
      Raw8<T, VEC> knr, vnr;
      knr.load((const T*)p.kn + b * p.kn_sb + h * p.kn_sh + sub * 8);
      vnr.load((const T*)p.vn + b * p.vn_sb + h * p.vn_sh + sub * 8);
      const float d = group_sum<LPK>(dot8(qr, knr)) * c2;
      if (g == 0) {
        const float M = fmaxf(m, d);
        const float f1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
        const float f2 = __builtin_amdgcn_exp2f(d - M);
        float vx[8];
        vnr.to_float(vx);
        l = l * f1 + f2;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = acc[e] * f1 + f2 * vx[e];
        m = M;
        knr.store((T*)K + (int64_t)jnew * kst);
        vnr.store((T*)V + (int64_t)jnew * vst);
      }
    }
  }

  // the wave's KPS key groups meet by xor shuffles over the group bits of
  // the lane id, then the NW waves through LDS
#pragma unroll
  for (int x = LPK; x < 64; x <<= 1) {
    const float om = __shfl_xor(m, x, 64), ol = __shfl_xor(l, x, 64);
    float oa[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) oa[e] = __shfl_xor(acc[e], x, 64);
    merge_state(m, l, acc, om, ol, oa);
  }
  if (g == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm_acc[w][sub * 8 + e] = acc[e];
    if (sub == 0) { sm_m[w] = m; sm_l[w] = l; }
  }
  __syncthreads();
  if (tid >= D) return;

  float M = -INFINITY;
#pragma unroll
  for (int x = 0; x < NW; ++x) M = fmaxf(M, sm_m[x]);
  float L = 0.f, A = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int x = 0; x < NW; ++x) {
      const float mx = sm_m[x];
      const float f = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mx - M);
      L += sm_l[x] * f;
      A += sm_acc[x][tid] * f;
    }
  }
  if (p.splits == 1) {
    T* O = (T*)p.o + b * p.o_sb + h * p.o_sh + i * p.o_st;
    O[tid] = from_f<T>(L > 0.f ? A / L : 0.f);
  } else {
    float* P = p.part + (row * p.splits + s) * (D + 2);
    P[tid] = A;
    if (tid == 0) { P[D] = M; P[D + 1] = L; }
  }
}

// One block of D threads per row: merges the row's split partials.
template <typename T, int D>
__global__ void __launch_bounds__(128) decode_merge(DArgs p) {
  const int64_t row = blockIdx.x;
  const int64_t i = row % p.Tq, bh = row / p.Tq;
  const int64_t h = bh % p.H, b = bh / p.H;
  const int t = threadIdx.x;
  const float* P = p.part + row * p.splits * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < p.splits; ++s) M = fmaxf(M, P[s * (D + 2) + D]);
  float L = 0.f, A = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < p.splits; ++s) {
      const float ms = P[s * (D + 2) + D];
      const float f = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - M);
      L += P[s * (D + 2) + D + 1] * f;
      A += P[s * (D + 2) + t] * f;
    }
  }
  T* O = (T*)p.o + b * p.o_sb + h * p.o_sh + i * p.o_st;
  O[t] = from_f<T>(L > 0.f ? A / L : 0.f);
}

// dst rows [pos[b] + t] of the cache = src rows t, as raw elements of E;
// blockIdx.y picks one of `pairs` (cache, rows) pairs of the same shape.
template <typename E>
struct KvArgs {
  E* c[2];
  const E* x[2];
  int64_t cs[2][3], xs[2][3];  // (batch, head, token) strides in E elements
  const int32_t* pos;
  int64_t H, T, D, Tmax, n;
};

template <typename E>
__global__ void __launch_bounds__(256) kv_write_kernel(KvArgs<E> a) {
  const int j = blockIdx.y;
  E* __restrict__ c = a.c[j];
  const E* __restrict__ x = a.x[j];
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = idx % a.D, r = idx / a.D;
    const int64_t t = r % a.T, bh = r / a.T;
    const int64_t h = bh % a.H, b = bh / a.H;
    const int64_t dt = (int64_t)a.pos[b] + t;
    if (dt < 0 || dt >= a.Tmax) continue;  // rows past the cache's capacity are dropped
    c[b * a.cs[j][0] + h * a.cs[j][1] + dt * a.cs[j][2] + d] = x[b * a.xs[j][0] + h * a.xs[j][1] + t * a.xs[j][2] + d];
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T, int D, bool NEW>
void launch_decode_n(const DArgs& p0, bool vec, int64_t rows, bool whole, hipStream_t s) {
  DArgs p = p0;
  p.pf.first = 0x7fffffff;
  // a whole-row launch leaves CUs idle: blocks past the rows read ahead
  // what the graph walk asked this launch to
  if (whole && p.splits == 1) p.pf = make_prefetch((int)rows, 64 * kDWavesWhole);
  const dim3 grid((unsigned)p.splits, (unsigned)(rows + (whole && p.splits == 1 ? p.pf.blocks : 0)));
  constexpr int NWW = kDWavesWhole, UW = kDUnrollWhole, NWS = kDWavesSplit, US = kDUnrollSplit;
  // 6 key steps per wave when that covers the whole cache in one iteration
  constexpr int UW6 = kDUnrollWhole6;
  const bool one_pass = p.Tmax <= (int64_t)NWW * (64 / (D / 8)) * UW6;
  if (whole && one_pass) {
    if (vec) hipLaunchKernelGGL((decode_attn<T, D, true, NWW, UW6, NEW>), grid, dim3(64 * NWW), 0, s, p);
    else hipLaunchKernelGGL((decode_attn<T, D, false, NWW, UW6, NEW>), grid, dim3(64 * NWW), 0, s, p);
  } else if (whole) {
    if (vec) hipLaunchKernelGGL((decode_attn<T, D, true, NWW, UW, NEW>), grid, dim3(64 * NWW), 0, s, p);
    else hipLaunchKernelGGL((decode_attn<T, D, false, NWW, UW, NEW>), grid, dim3(64 * NWW), 0, s, p);
  } else {
    if (vec) hipLaunchKernelGGL((decode_attn<T, D, true, NWS, US, NEW>), grid, dim3(64 * NWS), 0, s, p);
    else hipLaunchKernelGGL((decode_attn<T, D, false, NWS, US, NEW>), grid, dim3(64 * NWS), 0, s, p);
  }
  if (p.splits > 1) hipLaunchKernelGGL((decode_merge<T, D>), dim3((unsigned)rows), dim3(D), 0, s, p);
}

template <typename T, int D>
void launch_decode(const DArgs& p, bool vec, int64_t rows, bool whole, hipStream_t s) {
  if (p.kn) launch_decode_n<T, D, true>(p, vec, rows, whole, s);
  else launch_decode_n<T, D, false>(p, vec, rows, whole, s);
}

template <typename E>
void launch_kv_write(const KvWrite& a, int64_t vec, hipStream_t s) {
  // vec = elements of the dtype per E
  KvArgs<E> k{};
  const int pairs = a.cache2 ? 2 : 1;
  for (int j = 0; j < pairs; ++j) {
    k.c[j] = (E*)(j ? a.cache2 : a.cache);
    k.x[j] = (const E*)(j ? a.src2 : a.src);
    const int64_t* cs = j ? a.c2s : a.cs;
    const int64_t* xs = j ? a.x2s : a.xs;
    for (int i = 0; i < 3; ++i) {
      k.cs[j][i] = cs[i] / vec;
      k.xs[j][i] = xs[i] / vec;
    }
  }
  k.pos = a.pos;
  k.H = a.H; k.T = a.T; k.D = a.D / vec; k.Tmax = a.Tmax;
  k.n = a.B * a.H * a.T * k.D;
  int64_t g = (k.n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL((kv_write_kernel<E>), dim3((unsigned)g, (unsigned)pairs), dim3(256), 0, s, k);
}

}  // namespace

bool decode_attention_supported(const DecodeAttn& a) {
  return (a.D == 32 || a.D == 64 || a.D == 128) &&
         (a.dt == DType::F32 || a.dt == DType::F16 || a.dt == DType::BF16);
}

// Launch-shape override for tuning sweeps: APPLEGPU_DECODE_ATTN=whole, or
// split:<n> (n key splits of 4-wave blocks); unset = the heuristic below.
static int decode_forced_splits() {
  static int v = [] {
    const char* e = getenv("APPLEGPU_DECODE_ATTN");
    if (!e) return 0;
    if (!strcmp(e, "whole")) return -1;
    if (!strncmp(e, "split:", 6)) return atoi(e + 6) > 0 ? atoi(e + 6) : 0;
    return 0;
  }();
  return v;
}

static bool decode_whole(const DecodeAttn& a) {
  const int f = decode_forced_splits();
  if (f == -1) return true;
  if (f > 0) return false;
  return a.B * a.H * a.Tq >= kDRowsWhole;
}

int decode_attention_splits(const DecodeAttn& a, int64_t* chunk) {
  const int64_t rows = a.B * a.H * a.Tq;
  if (decode_whole(a)) {
    *chunk = a.Tmax;
    return 1;
  }
  // keys per block iteration of the split kernel, as in decode_attn
  const int64_t bs = (int64_t)kDWavesSplit * (64 / (a.D / 8)) * kDUnrollSplit;
  // aim for >= 2048 blocks over the 256 CUs, with at least one block
  // iteration per split
  int64_t want = rows >= 2048 ? 1 : (2048 + rows - 1) / rows;
  if (decode_forced_splits() > 0) want = decode_forced_splits();
  const int64_t max_splits = (a.Tmax + bs - 1) / bs;
  if (want > max_splits) want = max_splits;
  if (want < 1) want = 1;
  int64_t c = (a.Tmax + want - 1) / want;
  c = (c + bs - 1) / bs * bs;
  *chunk = c;
  return (int)((a.Tmax + c - 1) / c);
}

size_t decode_attention_ws_bytes(const DecodeAttn& a) {
  int64_t chunk;
  const int splits = decode_attention_splits(a, &chunk);
  if (splits <= 1) return 0;
  return (size_t)(a.B * a.H * a.Tq) * splits * (a.D + 2) * sizeof(float);
}

void decode_attention(const DecodeAttn& a, void* ws, hipStream_t s) {
  if (!decode_attention_supported(a)) fail("decode_attention: head dim %lld not supported", (long long)a.D);
  if (a.Tmax <= 0) fail("decode_attention: empty cache");
  if (a.Tmax * (a.k_st > a.v_st ? a.k_st : a.v_st) >= (int64_t)1 << 31)
    fail("decode_attention: cache rows of one head span more than 2^31 elements");
  const int64_t rows = a.B * a.H * a.Tq;
  if (rows == 0) return;
  if (rows > 0x7fffffffLL) fail("decode_attention: too many rows");
  DArgs p{};
  p.q = a.q; p.k = a.k; p.v = a.v; p.o = a.o;
  p.lens = a.lens;
  p.H = a.H; p.Tq = a.Tq; p.Tmax = a.Tmax;
  p.q_sb = a.q_sb; p.q_sh = a.q_sh; p.q_st = a.q_st;
  p.k_sb = a.k_sb; p.k_sh = a.k_sh; p.k_st = a.k_st;
  p.v_sb = a.v_sb; p.v_sh = a.v_sh; p.v_st = a.v_st;
  p.o_sb = a.o_sb; p.o_sh = a.o_sh; p.o_st = a.o_st;
  p.scale = a.scale;
  if (a.kn) {
    if (a.Tq != 1 || !a.vn) fail("decode_attention: appending new K/V rows needs one query row per sequence");
    p.kn = a.kn; p.vn = a.vn;
    p.kn_sb = a.kn_sb; p.kn_sh = a.kn_sh; p.vn_sb = a.vn_sb; p.vn_sh = a.vn_sh;
  }
  int64_t chunk;
  p.splits = decode_attention_splits(a, &chunk);
  p.chunk = (int)chunk;
  if (p.splits > 1) {
    if (!ws) fail("decode_attention: split-KV workspace missing");
    p.part = (float*)ws;
  }
  // 16-byte loads need every row of q, K and V 16-byte aligned
  const size_t es = dtype_size(a.dt);
  auto al = [&](const void* ptr, int64_t s0, int64_t s1, int64_t s2) {
    return al16(ptr) && (s0 * es) % 16 == 0 && (s1 * es) % 16 == 0 && (s2 * es) % 16 == 0;
  };
  const bool vec = al(a.q, a.q_sb, a.q_sh, a.q_st) && al(a.k, a.k_sb, a.k_sh, a.k_st) &&
                   al(a.v, a.v_sb, a.v_sh, a.v_st) &&
                   (!a.kn || (al(a.kn, a.kn_sb, a.kn_sh, 0) && al(a.vn, a.vn_sb, a.vn_sh, 0)));
  AGPU_FLOAT_SWITCH(a.dt, {
    const bool whole = decode_whole(a);
    if (a.D == 32) launch_decode<T, 32>(p, vec, rows, whole, s);
    else if (a.D == 64) launch_decode<T, 64>(p, vec, rows, whole, s);
    else launch_decode<T, 128>(p, vec, rows, whole, s);
  });
  check_launch("decode_attention");
}

void kv_write(const KvWrite& a, hipStream_t s) {
  const int64_t n = a.B * a.H * a.T * a.D;
  if (n == 0) return;
  const size_t es = dtype_size(a.dt);
  // widest element that divides every row and stride of every pair
  auto fits = [&](size_t w) {
    const int64_t v = (int64_t)(w / es);
    if (w < es || w % es) return false;
    auto ok = [&](int64_t x) { return x % v == 0; };
    bool r = ok(a.D);
    for (int j = 0; j < (a.cache2 ? 2 : 1); ++j) {
      const void* c = j ? a.cache2 : a.cache;
      const void* x = j ? a.src2 : a.src;
      const int64_t* cs = j ? a.c2s : a.cs;
      const int64_t* xs = j ? a.x2s : a.xs;
      r = r && ((uintptr_t)c % w) == 0 && ((uintptr_t)x % w) == 0 && ok(cs[0]) && ok(cs[1]) && ok(cs[2]) &&
          ok(xs[0]) && ok(xs[1]) && ok(xs[2]);
    }
    return r;
  };
  if (fits(16)) launch_kv_write<uint4>(a, (int64_t)(16 / es), s);
  else if (fits(8)) launch_kv_write<uint2>(a, (int64_t)(8 / es), s);
  else if (es == 4) launch_kv_write<uint32_t>(a, 1, s);
  else if (es == 2) launch_kv_write<uint16_t>(a, 1, s);
  else if (es == 1) launch_kv_write<uint8_t>(a, 1, s);
  else launch_kv_write<uint2>(a, 1, s);
  check_launch("kv_write");
}

}  // namespace k
}  // namespace agpu
