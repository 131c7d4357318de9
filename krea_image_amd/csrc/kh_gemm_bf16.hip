// GEMM kernel instantiations for bf16 activations (the kernel is in kh_gemm_kernel.h).
#include "kh_gemm_kernel.h"

namespace kh {
namespace gemm_detail {

hipError_t launch_gemm_bf16(int wf, int epi, const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  return launch_wf<KH_BF16>(wf, epi, a, grid_x, tn, st);
}

hipError_t launch_conv_bf16(const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  return launch_conv<KH_BF16>(a, grid_x, tn, st);
}

}  // namespace gemm_detail
}  // namespace kh
