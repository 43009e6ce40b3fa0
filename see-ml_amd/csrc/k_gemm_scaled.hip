// k_gemm_scaled.hip — GEMM kernel instantiations with a Scale folded into
// one operand's loads: NT with A scaled (dt = (s du) B^T) and TN with B
// scaled (dB = t^T (s du)), on the small tile configs.
#include "k_gemm_kernel.h"

namespace seeml_hip {
namespace gemm {

bool LaunchScaledNT(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  return LaunchScaledVariant<true, true, 1>(cfg, grid, s, a);
}

bool LaunchScaledTN(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  return LaunchScaledVariant<false, false, 2>(cfg, grid, s, a);
}

}  // namespace gemm
}  // namespace seeml_hip
