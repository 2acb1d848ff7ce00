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
// Layout: one 256-thread block owns 64 query rows of one (batch, head); four
// threads share a row.  Thread (r, sub) keeps its query row in registers,
// scores keys sub, sub+4, ..., and accumulates output dims
// {sub*4 + 16*i + 0..3}.  Q, K, V and O are read/written through their own
// (batch, head, token) strides with unit stride along d, so head splits of a
// fused QKV projection and the head-merge transpose cost nothing.
#include "device.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {

constexpr int kQT = 64;  // query rows per block
constexpr int kKT = 64;  // keys per LDS tile

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
  constexpr int KP = D + 4;   // K row pitch (floats), keeps float4 reads conflict-free
  constexpr int PP = kKT + 1; // P row pitch
  constexpr int DO = D / 4;   // output dims per thread
  __shared__ __attribute__((aligned(16))) float Ks[kKT * KP];
  __shared__ __attribute__((aligned(16))) float Vs[kKT * D];
  __shared__ float Ps[kQT * PP];

  const int tid = threadIdx.x;
  const int r = tid >> 2, sub = tid & 3;
  const int64_t bh = blockIdx.x / p.q_tiles;
  const int qt = (int)(blockIdx.x % p.q_tiles);
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q0 = (int64_t)qt * kQT;
  const int64_t qi = q0 + r;
  const bool row_ok = qi < p.Tq;

  const T* Q = (const T*)p.q + b * p.q_sb + h * p.q_sh;
  const T* K = (const T*)p.k + b * p.k_sb + h * p.k_sh;
  const T* V = (const T*)p.v + b * p.v_sb + h * p.v_sh;

  float q[D];
#pragma unroll
  for (int d = 0; d < D; ++d) q[d] = row_ok ? to_f(Q[qi * p.q_st + d]) : 0.f;

  float o[DO];
#pragma unroll
  for (int i = 0; i < DO; ++i) o[i] = 0.f;
  float m = -INFINITY, l = 0.f;

  int64_t kv_end = p.Tk;
  if (p.causal) {
    int64_t last_q = q0 + kQT - 1 < p.Tq - 1 ? q0 + kQT - 1 : p.Tq - 1;
    kv_end = last_q + 1 < p.Tk ? last_q + 1 : p.Tk;
  }

  for (int64_t j0 = 0; j0 < kv_end; j0 += kKT) {
    // stage K and V tiles as fp32
    for (int e = tid; e < kKT * D; e += 256) {
      const int c = e / D, d = e % D;
      const int64_t j = j0 + c;
      const bool ok = j < p.Tk;
      Ks[c * KP + d] = ok ? to_f(K[j * p.k_st + d]) : 0.f;
      Vs[c * D + d] = ok ? to_f(V[j * p.v_st + d]) : 0.f;
    }
    __syncthreads();

    float s[kKT / 4];
    float tmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < kKT / 4; ++jj) {
      const int c = sub + 4 * jj;
      const float* kr = &Ks[c * KP];
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        float4 kv = *(const float4*)&kr[d];
        acc += q[d] * kv.x;
        acc += q[d + 1] * kv.y;
        acc += q[d + 2] * kv.z;
        acc += q[d + 3] * kv.w;
      }
      const int64_t j = j0 + c;
      bool vis = j < p.Tk && (!p.causal || j <= qi);
      s[jj] = vis ? acc * p.scale : -INFINITY;
      tmax = fmaxf(tmax, s[jj]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 1, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 2, 64));
    const float m_new = fmaxf(m, tmax);
    // m_new is finite for every row that has a visible key in this tile or
    // an earlier one; rows with none keep zero weight.
    const float alpha = (m == -INFINITY) ? 0.f : expf(m - m_new);
    float psum = 0.f;
#pragma unroll
    for (int jj = 0; jj < kKT / 4; ++jj) {
      const float pv = (s[jj] == -INFINITY) ? 0.f : expf(s[jj] - m_new);
      psum += pv;
      Ps[r * PP + sub + 4 * jj] = pv;
    }
    psum += __shfl_xor(psum, 1, 64);
    psum += __shfl_xor(psum, 2, 64);
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int i = 0; i < DO; ++i) o[i] *= alpha;
    __syncthreads();

#pragma unroll 4
    for (int c = 0; c < kKT; ++c) {
      const float pv = Ps[r * PP + c];
      const float* vr = &Vs[c * D];
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        float4 vv = *(const float4*)&vr[sub * 4 + 16 * i];
        o[4 * i] += pv * vv.x;
        o[4 * i + 1] += pv * vv.y;
        o[4 * i + 2] += pv * vv.z;
        o[4 * i + 3] += pv * vv.w;
      }
    }
    __syncthreads();
  }

  if (!row_ok) return;
  T* O = (T*)p.o + b * p.o_sb + h * p.o_sh + qi * p.o_st;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int i = 0; i < D / 16; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) O[sub * 4 + 16 * i + e] = from_f<T>(o[4 * i + e] * inv);
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
