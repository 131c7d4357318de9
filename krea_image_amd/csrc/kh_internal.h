// Host-side internals of libkh: the error sink of the C ABI and the op entry points behind it.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/kh.h"

namespace kh {

// Error sink of one C-ABI call: formats into the caller's (err, errlen) buffer, like the reference's
// C boundary copies std::exception::what() into `err` (engine/src/pipeline.mm:594-641).
struct Err {
  char* buf;
  int len;
  int fail(const char* fmt, ...) __attribute__((format(printf, 2, 3))) {
    if (buf && len > 0) {
      va_list ap;
      va_start(ap, fmt);
      vsnprintf(buf, (size_t)len, fmt, ap);
      va_end(ap);
    }
    return KH_EINVAL;
  }
  int hip(hipError_t r, const char* what) {
    if (buf && len > 0) snprintf(buf, (size_t)len, "%s: %s", what, hipGetErrorString(r));
    return KH_EHIP;
  }
  void clear() {
    if (buf && len > 0) buf[0] = 0;
  }
};

// Stream-K workspace of a GEMM launch (caller-owned device memory, 256-byte aligned, its counter words zeroed once
// by gemm_workspace_init); a launch without one (or with one too small) runs data-parallel.
struct GemmWs {
  void* p;
  size_t bytes;
};
size_t gemm_workspace_bytes_for(int ctas);
int gemm_plan(int M, int N, int K, int epi, int w16, int ctas, int with_ws, int* out, Err& e);
size_t gemm_workspace_bytes();  // for the current device
int gemm_workspace_init(hipStream_t st, void* ws, size_t bytes, Err& e);
// kh_gemm_ws with the library's static device scratch as the workspace (no allocation)
int gemm_static(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
                int lda, int ldw, int ldc, const void* vec, Err& e);
size_t gemm_static_scratch_bytes();

int pack_int8(hipStream_t st, const void* W, int K, int ldw, void* out, Err& e);
int gemm(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
         int lda, int ldw, int ldc, const void* vec, Err& e, const GemmWs* ws = nullptr);
// the per-head RMSNorm + RoPE of qk_norm_rope fused into a STORE16 GEMM's epilogue
struct QkNormRope {
  const float *wq, *wk, *cosb, *sinb;
  float *qbig, *kbig;
  int q_off, n_q, k_off, n_k, mode, big_dim;
  float eps;
};
int gemm_qk_norm_rope(hipStream_t st, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
                      int lda, int ldw, int ldc, const QkNormRope& q, Err& e, const GemmWs* ws = nullptr);
int conv_up2_subpix(hipStream_t st, const void* x, int ldx, int C, int H, int W, int dtype, const kh_weight& W2, int K,
                    int Np, const float* bias4, void* y, int ldy, Err& e, const GemmWs* ws = nullptr);
int vae_subpix_weights(hipStream_t st, const void* w, int dtype, int Cin, int Cout, void* w2, int Kp, int Np,
                       const float* b, float* b4, Err& e);
int conv3x3(hipStream_t st, const void* x, int ldx, int C, int H, int W, int up, int dtype, const kh_weight& Wt, int K,
            int N, const float* bias, const void* res, void* y, int ldy, Err& e, const GemmWs* ws = nullptr);

int attention(hipStream_t st, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
              int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
              int ldg, const float* QB, const float* KB, Err& e);

int rms_norm(hipStream_t st, const float* x, const float* mul, const float* add, void* y, int out_dtype, int rows,
             int width, int ld_in, int ld_out, float eps, int center, Err& e);
int qk_norm_rope(hipStream_t st, void* qkv, int dtype, const float* wq, const float* wk, const float* cosb,
                 const float* sinb, int rows, int ld, int q_off, int n_q, int k_off, int n_k, float eps, int rope_mode,
                 int big_dim, float* qbig, float* kbig, Err& e);
int gemv(hipStream_t st, const float* x, const kh_weight& W, float* y, int rows, int N, int K, int ldw, int act,
         const float* bias, Err& e);
int make_cond(hipStream_t st, const float* tvec, const float* table, const float* n1, const float* n2, int D,
              float* mods, Err& e);
int make_fin(hipStream_t st, const float* t, const float* lin, const float* nf, int D, float* fin, Err& e);
// copies n <= 256 host floats to dst by a kernel argument (stream-ordered, no staging buffer)
int store_vec(hipStream_t st, const float* host, int n, float* dst, Err& e);
int conditioning(hipStream_t st, const kh_qw* f, int fast, float sigma, float* t, float* tvec, float* work,
                 size_t work_bytes, int* from_table, Err& e);
int gemm_f32(hipStream_t st, const float* A, const float* W, float* C, int M, int N, int K, int lda, int ldw, int ldc,
             int mode, const float* bias, Err& e);
int dit_layer_forward(hipStream_t st, const kh_dit_config& c, const kh_dit_layer& L, const kh_dit_state& s, int R,
                      Err& e);
int dit_forward(hipStream_t st, const kh_dit_config& c, const kh_dit_layer* layers, int n, const kh_dit_state& s,
                int R, Err& e);
int rope_tables(int T, int H, int W, int mode, float* cosb, float* sinb);
int sigmas(int steps, float mu, float* out);
int euler_step(hipStream_t st, float* z, const float* v, long long n, float dt, Err& e);
int cfg_combine(hipStream_t st, float* vc, const float* vn, long long n, float scale, Err& e);

int vae_unpack(hipStream_t st, const float* z, const float* mean, const float* stdv, const float* w, const float* b,
               void* y, int H16, int W16, Err& e);
int vae_im2col(hipStream_t st, const void* x, int ldx, int C, int H, int W, int up, int m0, int rows, void* col,
               int Kpad, Err& e);
int vae_norm_silu(hipStream_t st, const void* x, int ldx, const float* gamma, void* y, int ldy, int P, int C, int silu,
                  Err& e);
int vae_add(hipStream_t st, void* y, const void* a, long long n, Err& e);
int vae_transpose(hipStream_t st, const void* in, int ld, int off, int P, int C, void* out, int ldo, Err& e);
int vae_softmax(hipStream_t st, const float* S, int ld, int rows, int n, float scale, void* Pm, Err& e);
int vae_conv_out(hipStream_t st, const void* x, int ldx, int C, const void* w, const float* bias, void* rgba, int H,
                 int W, Err& e);
int vae_zero(hipStream_t st, void* p, size_t bytes, Err& e);
int vae_pad_weight(hipStream_t st, const void* w, int K, int N, void* out, int Kp, int Np, const float* b, float* bout,
                   Err& e);
size_t vae_workspace_bytes(int H16, int W16);
int vae_decode(hipStream_t st, const kh_qw* f, const float* z, int H16, int W16, void* ws, size_t ws_bytes, void* rgba,
               Err& e);

}  // namespace kh
