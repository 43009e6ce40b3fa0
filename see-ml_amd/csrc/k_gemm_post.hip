// k_gemm_post.hip — GEMM kernel instantiations with an AddBias (and an
// activation) after the fused AddEW: NN, the small tile configs.
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

bool LaunchPostNN(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  return LaunchPostVariant<true, false>(cfg, grid, s, a);
}

}  // namespace gemm
}  // namespace seeml_hip
