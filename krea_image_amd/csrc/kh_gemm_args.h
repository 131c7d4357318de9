// Shared by the GEMM's host planner (kh_gemm.hip) and its kernel instantiation units (kh_gemm_f16.hip,
// kh_gemm_bf16.hip): tile constants, weight-format codes, the kernel argument block and the launchers.
#pragma once
#include "kh_common.h"

namespace kh {
namespace gemm_detail {

constexpr int BM = 256, BN = 256, BK = 64;
#ifndef KH_GEMM_WAVES
#define KH_GEMM_WAVES 8
#endif
constexpr int WAVES_DEFAULT = KH_GEMM_WAVES;
constexpr int STAGE = BM * BK * 2;  // bytes of one 16-bit 256 x 64 tile
constexpr int X_STAGES = 3, W_STAGES = 2;
constexpr int GROUP_M = 4;  // tile rows per group (measured: 4 edges out 2, 8 and 16 by 1-3 %)

// weight formats; the group formats carry their scale type in the kernel so the K loop has no branches
enum { WF_16 = 0, WF_I8_CHANNEL = 1, WF_I8_GROUP = 2, WF_I8_GROUP_F16 = 3, WF_I8_GROUP_BF16 = 4 };
// flag on an int8 format: the weights are in the packed layout of kh_pack_int8 (each thread's 8 k-rows x 4
// columns contiguous, read with two 16-byte loads instead of eight 4-byte ones)
constexpr int WF_PK = 8;
// internal epilogue: STORE16 followed by the per-head RMSNorm + RoPE of the q and k heads (qk_norm_rope fused;
// GemmArgs qk_*). Needs 256-wide tiles: each wave's 128 columns are then one head.
constexpr int EPI_QKNR = 8;
constexpr bool wide_only(int epi) { return epi == KH_EPI_SWIGLU || epi == EPI_QKNR; }
constexpr bool is_group(int wf) { return wf >= WF_I8_GROUP; }

struct GemmArgs {
  const void* A;
  const void* W;
  const void* S;
  void* C;
  const float* vec;
  int M, N, K, lda, ldw, ldc, gshift, s_dtype;
  int sk_iters;  // stream-K: K steps per workgroup (0 = one tile per workgroup)
  float* ws;     // stream-K partial tiles: 2 slots of BM x BN f32 per workgroup
  int* cnt;      // stream-K arrival counts per tile (zero between launches)
  // implicit 3 x 3 convolution (CONV kernels): A is an NHWC image [pixels, lda] of cv_C channels, the GEMM
  // rows are the cv_H x cv_W output pixels and K runs over (tap, channel) (tools/convert.py:338-344);
  // cv_up: the image is cv_H / 2 x cv_W / 2, nearest-upsampled. cv_cinv = ceil(2^32 / cv_C).
  int cv_C, cv_H, cv_W, cv_up;
  uint32_t cv_cinv;
  // BIAS16 only: C16 = round16(round16(acc + vec) + R) with R 16-bit [M, ldr] (the VAE's residual adds),
  // when R is not null
  const void* R;
  int ldr;
  // cv_sub = 1: the 2x-upsampling 3 x 3 conv as sub-pixel 2 x 2 convs on the cv_H x cv_W low-res image: rows
  // are low-res pixels, K runs over (2 x 2 tap, channel), column n = phase cv_np + co with phase = 2 py + px,
  // and row (i, j) of phase (py, px) is output pixel (2 i + py, 2 j + px) of the 2 cv_H x 2 cv_W image.
  // cv_winv = ceil(2^32 / cv_W).
  int cv_sub, cv_np;
  uint32_t cv_winv;
  // EPI_QKNR: q heads are columns [qk_qoff, + 128 qk_nq), k heads [qk_koff, + 128 qk_nk) (offsets multiples of
  // 128); norm weights qk_wq / qk_wk [128]; RoPE tables [M, 64] (qk_mode 0: adjacent pairs, 1: i with i + 64,
  // 2: none); qk_big >= 0: that head channel goes to qk_qbig [M, nq] / qk_kbig [M, nk] in f32 and is zeroed
  const float *qk_wq, *qk_wk, *qk_cos, *qk_sin;
  float *qk_qbig, *qk_kbig;
  int qk_qoff, qk_nq, qk_koff, qk_nk, qk_mode, qk_big;
  float qk_eps;
  // host-side launch choice, not read by the kernel: K steps ahead that weights are loaded (2, or 3 for the
  // instantiations that have the three-set form; see gemm_kernel's WA)
  int wa = 2;
};
// the weight formats / tile widths with a three-step weight prefetch instantiation (WA = 3): packed int8 with
// per-channel scales, data-parallel; 256-wide tiles only with fp16 activations (the bf16 conversion needs
// the registers the third set would take)
constexpr bool has_wa3(int act, int wf, int tn) {
  return wf == (WF_I8_CHANNEL | WF_PK) && (tn != 256 || act == KH_F16);
}

// launch the GEMM kernel instantiation for (activation type, weight format wf, epilogue epi, tile width tn):
// kh_gemm_f16.hip / kh_gemm_bf16.hip
hipError_t launch_gemm_f16(int wf, int epi, const GemmArgs& a, int grid_x, int tn, hipStream_t st);
hipError_t launch_gemm_bf16(int wf, int epi, const GemmArgs& a, int grid_x, int tn, hipStream_t st);
// the implicit 3 x 3 convolution kernels (16-bit weights, bias epilogue)
hipError_t launch_conv_f16(const GemmArgs& a, int grid_x, int tn, hipStream_t st);
hipError_t launch_conv_bf16(const GemmArgs& a, int grid_x, int tn, hipStream_t st);

}  // namespace gemm_detail
}  // namespace kh
