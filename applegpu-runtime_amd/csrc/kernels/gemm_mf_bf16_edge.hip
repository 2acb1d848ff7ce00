// Instantiates the gemm_mf kernels for bf16 operands of any shape (masked
// loads for every K slice; see gemm_kernels.hpp), and the bf16 dispatcher.
#include "gemm_kernels.hpp"

namespace agpu {
namespace k {
using namespace dev;

void launch_mf_bf16(const GArgs& p, int cfg, bool ak, bool bk, bool fast, dim3 grid, hipStream_t s) {
  if (fast) launch_mf_bf16_fast(p, cfg, ak, bk, grid, s);
  else launch_mf<bf16_t, bf16_t, false>(p, cfg, ak, bk, grid, s);
}

}  // namespace k
}  // namespace agpu
