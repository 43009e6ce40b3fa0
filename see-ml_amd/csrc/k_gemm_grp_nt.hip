// k_gemm_grp_nt.hip — GEMM group kernel instantiations: both operands k-contiguous
// (the independent projection GEMMs of a decoder layer in one launch).
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

bool LaunchGroupNT(int cfg, dim3 grid, hipStream_t s, const GemmGroupArgs& g) {
  for (uint32_t j = 0; j < g.count; ++j)
    if (g.m[j].lora_t) return LaunchGroupVariant<true, true>(cfg, grid, s, g);
  return LaunchGroupVariant<true, false>(cfg, grid, s, g);
}

}  // namespace gemm
}  // namespace seeml_hip
