// k_gemm_nn.hip — GEMM kernel instantiations: A k-contiguous, B row-contiguous (GemmNN, GemmAccNN, PV, dS K).
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

void LaunchNN(int cfg, bool vec, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  if (a.lora_t) {  // the host admits only vec, one slice and the LoRA configs
    (void)LaunchLoraVariant<true, false>(cfg, grid, s, a);
    return;
  }
  if (vec && a.out && a.splits == 1) LaunchVariant<true, false, false, true, true, true>(cfg, grid, s, a);
  else if (vec) LaunchVariant<true, false, false, true, true>(cfg, grid, s, a);
  else LaunchVariant<true, false, false, false>(cfg, grid, s, a);
}

}  // namespace gemm
}  // namespace seeml_hip
