// Instantiates the gemm_mf kernels for f16 operands that qualify for the
// unmasked fast loads (see gemm_kernels.hpp).
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

void launch_mf_f16_fast(const GArgs& p, int cfg, bool ak, bool bk, dim3 grid, hipStream_t s) {
  launch_mf<half_t, half_t, true>(p, cfg, ak, bk, grid, s);
}

}  // namespace k
}  // namespace agpu
