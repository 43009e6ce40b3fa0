// k_gemm_nt.hip — GEMM kernel instantiations: both k-contiguous (GemmNT, QK^T, dO V^T).
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

void LaunchNT(int cfg, bool vec, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  if (a.lora_t) {  // the host admits only vec, one slice and the LoRA configs
    (void)LaunchLoraVariant<true, true>(cfg, grid, s, a);
    return;
  }
  if (vec && a.out && a.splits == 1) LaunchVariant<true, true, false, true, true, true>(cfg, grid, s, a);
  else if (vec) LaunchVariant<true, true, false, true, true>(cfg, grid, s, a);
  else LaunchVariant<true, true, false, false>(cfg, grid, s, a);
}

}  // namespace gemm
}  // namespace seeml_hip
