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
#include "device.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kQT = 16;  // query rows per block
constexpr int kKT = 64;  // keys per LDS tile
constexpr int kTPR = 16; // threads per query row

struct AArgs {
  const void* q; const void* k; const void* v; void* o;
  int64_t H, Tq, Tk;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale;
  int causal;
  int q_tiles;
};

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

}  // namespace

bool attention_supported(const Attn& a) {
  return (a.D == 64 || a.D == 128 || a.D == 32) && (a.dt == DType::F32 || a.dt == DType::F16 || a.dt == DType::BF16);
}

void attention(const Attn& a, hipStream_t s) {
  if (!attention_supported(a)) fail("fused attention: head dim %lld not supported", (long long)a.D);
  if (a.B * a.H * a.Tq == 0) return;
  AArgs p{};
  p.q = a.q; p.k = a.k; p.v = a.v; p.o = a.o;
  p.H = a.H; p.Tq = a.Tq; p.Tk = a.Tk;
  p.q_sb = a.q_sb; p.q_sh = a.q_sh; p.q_st = a.q_st;
  p.k_sb = a.k_sb; p.k_sh = a.k_sh; p.k_st = a.k_st;
  p.v_sb = a.v_sb; p.v_sh = a.v_sh; p.v_st = a.v_st;
  p.o_sb = a.o_sb; p.o_sh = a.o_sh; p.o_st = a.o_st;
  p.scale = a.scale;
  p.causal = a.causal ? 1 : 0;
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
