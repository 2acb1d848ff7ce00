// Instantiates gemm_mf for fp32 activations times int8 weight codes with a
// per-output-row scale (B(k, n) = q[n][k] * scale[n]): the dequantisation is
// fused into the operand conversion, so W streams from HBM at one byte per
// element (see gemm_kernels.hpp).
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

namespace {
template <bool FAST>
void launch_i8(const GArgs& p, int cfg, bool ak, dim3 grid, hipStream_t s) {
  if (cfg == 0) {
    if (ak) hipLaunchKernelGGL((gemm_mf<float, int8_t, bf16_t, 128, 128, 2, 2, 1, 32, 2, true, true, FAST>), grid,
                               dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemm_mf<float, int8_t, bf16_t, 128, 128, 2, 2, 1, 32, 2, false, true, FAST>), grid,
                            dim3(256), 0, s, p);
  } else if (cfg == 6) {
    if (ak) hipLaunchKernelGGL((gemm_mf<float, int8_t, bf16_t, 64, 64, 2, 2, 1, 64, 2, true, true, FAST>), grid,
                               dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemm_mf<float, int8_t, bf16_t, 64, 64, 2, 2, 1, 64, 2, false, true, FAST>), grid,
                            dim3(256), 0, s, p);
  } else {
    fail("gemm: int8 weights take tile configuration 0 or 6, not %d", cfg);
  }
}
}  // namespace

void launch_mf_f32_i8(const GArgs& p, int cfg, bool ak, bool fast, dim3 grid, hipStream_t s) {
  if (fast) launch_i8<true>(p, cfg, ak, grid, s);
  else launch_i8<false>(p, cfg, ak, grid, s);
}

}  // namespace k
}  // namespace agpu
