// GEMM kernel instantiations for f16 activations (the kernel is in kh_gemm_kernel.h).
#include "kh_gemm_kernel.h"

namespace kh {
namespace gemm_detail {

hipError_t launch_gemm_f16(int wf, int epi, const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  return launch_wf<KH_F16>(wf, epi, a, grid_x, tn, st);
}

hipError_t launch_conv_f16(const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  return launch_conv<KH_F16>(a, grid_x, tn, st);
}

}  // namespace gemm_detail
}  // namespace kh
