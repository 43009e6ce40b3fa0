// k_gemm_tn.hip — GEMM kernel instantiations: both row-contiguous (GemmTN, P^T dO, dS^T Q).
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

void LaunchTN(int cfg, bool vec, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  if (vec && a.out && a.splits == 1) LaunchVariant<false, false, false, true, true, true>(cfg, grid, s, a);
  else if (vec) LaunchVariant<false, false, false, true, true>(cfg, grid, s, a);
  else LaunchVariant<false, false, false, false>(cfg, grid, s, a);
}

}  // namespace gemm
}  // namespace seeml_hip
