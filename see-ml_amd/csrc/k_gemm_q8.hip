// k_gemm_q8.hip — GEMM kernel instantiations: int8 B (GemmNNQ8 / GemmNTQ8), element loads.
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

void LaunchQ8(int cfg, bool b_kc, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  if (b_kc) LaunchVariant<true, true, true, false>(cfg, grid, s, a);
  else LaunchVariant<true, false, true, false>(cfg, grid, s, a);
}

}  // namespace gemm
}  // namespace seeml_hip
