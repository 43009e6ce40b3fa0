// k_gemm_grp_nn.hip — GEMM group kernel instantiations: A k-contiguous, B row-contiguous
// (the independent projection GEMMs of a decoder layer in one launch).
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

bool LaunchGroupNN(int cfg, dim3 grid, hipStream_t s, const GemmGroupArgs& g) {
  for (uint32_t j = 0; j < g.count; ++j)
    if (g.m[j].lora_t) return LaunchGroupVariant<false, true>(cfg, grid, s, g);
  return LaunchGroupVariant<false, false>(cfg, grid, s, g);
}

}  // namespace gemm
}  // namespace seeml_hip
