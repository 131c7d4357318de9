// The C ABI of libkh (include/kh.h): argument plumbing only; validation and launches live with each op.
#include "kh_internal.h"

extern "C" {

const char* kh_version(void) { return "libkh 0.1 gfx950"; }

int kh_gemm(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N, int K,
            int lda, int ldw, int ldc, const void* vec, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!W) return e.fail("gemm: null weight descriptor");
  return kh::gemm((hipStream_t)stream, epi, A, a_dtype, *W, C, M, N, K, lda, ldw, ldc, vec, e);
}

int kh_gemm_ws(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N, int K,
               int lda, int ldw, int ldc, const void* vec, void* workspace, size_t workspace_bytes, char* err,
               int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!W) return e.fail("gemm: null weight descriptor");
  const kh::GemmWs ws{workspace, workspace_bytes};
  return kh::gemm((hipStream_t)stream, epi, A, a_dtype, *W, C, M, N, K, lda, ldw, ldc, vec, e, &ws);
}

size_t kh_gemm_workspace_bytes(void) { return kh::gemm_workspace_bytes(); }

int kh_gemm_plan(int M, int N, int K, int epi, int w16, int ctas, int with_ws, int* out, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::gemm_plan(M, N, K, epi, w16, ctas, with_ws, out, e);
}

int kh_gemm_static(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N,
                   int K, int lda, int ldw, int ldc, const void* vec, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!W) return e.fail("gemm: null weight descriptor");
  return kh::gemm_static((hipStream_t)stream, epi, A, a_dtype, *W, C, M, N, K, lda, ldw, ldc, vec, e);
}

int kh_gemm_workspace_init(kh_stream stream, void* workspace, size_t workspace_bytes, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::gemm_workspace_init((hipStream_t)stream, workspace, workspace_bytes, e);
}

int kh_pack_int8(kh_stream stream, const void* W, int K, int ldw, void* out, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::pack_int8((hipStream_t)stream, W, K, ldw, out, e);
}

int kh_attention(kh_stream stream, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
                 int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
                 int ldg, const float* QB, const float* KB, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::attention((hipStream_t)stream, Q, K, V, O, dtype, Lq, Lk, heads, ldq, ldk, ldv, ldo, group, causal,
                       q_pos0, G, ldg, QB, KB, e);
}

int kh_rms_norm(kh_stream stream, const float* x, const float* mul, const float* add, void* y, int out_dtype, int rows,
                int width, int ld_in, int ld_out, float eps, int center, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::rms_norm((hipStream_t)stream, x, mul, add, y, out_dtype, rows, width, ld_in, ld_out, eps, center, e);
}

int kh_gemm_qk_norm_rope(kh_stream stream, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N,
                         int K, int lda, int ldw, int ldc, const float* wq, const float* wk, const float* cosb,
                         const float* sinb, int q_off, int n_q, int k_off, int n_k, float eps, int rope_mode,
                         int big_dim, float* qbig, float* kbig, void* workspace, size_t workspace_bytes, char* err,
                         int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!W) return e.fail("gemm_qk_norm_rope: null weight descriptor");
  const kh::QkNormRope q{wq, wk, cosb, sinb, qbig, kbig, q_off, n_q, k_off, n_k, rope_mode, big_dim, eps};
  const kh::GemmWs ws{workspace, workspace_bytes};
  return kh::gemm_qk_norm_rope((hipStream_t)stream, A, a_dtype, *W, C, M, N, K, lda, ldw, ldc, q, e, &ws);
}

int kh_qk_norm_rope(kh_stream stream, void* qkv, int dtype, const float* wq, const float* wk, const float* cosb,
                    const float* sinb, int rows, int ld, int q_off, int n_q, int k_off, int n_k, float eps,
                    int rope_mode, int big_dim, float* qbig, float* kbig, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::qk_norm_rope((hipStream_t)stream, qkv, dtype, wq, wk, cosb, sinb, rows, ld, q_off, n_q, k_off, n_k, eps,
                          rope_mode, big_dim, qbig, kbig, e);
}

int kh_gemv(kh_stream stream, const float* x, const kh_weight* W, float* y, int rows, int N, int K, int ldw, int act,
            const float* bias, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!W) return e.fail("gemv: null weight descriptor");
  return kh::gemv((hipStream_t)stream, x, *W, y, rows, N, K, ldw, act, bias, e);
}

int kh_make_cond(kh_stream stream, const float* tvec, const float* table, const float* n1, const float* n2, int D,
                 float* mods, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::make_cond((hipStream_t)stream, tvec, table, n1, n2, D, mods, e);
}

int kh_make_fin(kh_stream stream, const float* t, const float* lin, const float* nf, int D, float* fin, char* err,
                int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::make_fin((hipStream_t)stream, t, lin, nf, D, fin, e);
}

int kh_conditioning(kh_stream stream, const kh_qw* cond, int fast, float sigma, float* t, float* tvec, float* work,
                    size_t work_bytes, int* from_table, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::conditioning((hipStream_t)stream, cond, fast, sigma, t, tvec, work, work_bytes, from_table, e);
}

int kh_gemm_f32(kh_stream stream, const float* A, const float* W, float* C, int M, int N, int K, int lda, int ldw,
                int ldc, int mode, const float* bias, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::gemm_f32((hipStream_t)stream, A, W, C, M, N, K, lda, ldw, ldc, mode, bias, e);
}

int kh_rope_tables(int T, int H, int W, int mode, float* cosb, float* sinb) {
  return kh::rope_tables(T, H, W, mode, cosb, sinb);
}

int kh_sigmas(int steps, float mu, float* out) { return kh::sigmas(steps, mu, out); }

int kh_euler_step(kh_stream stream, float* z, const float* v, long long n, float dt, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::euler_step((hipStream_t)stream, z, v, n, dt, e);
}

int kh_cfg_combine(kh_stream stream, float* vc, const float* vn, long long n, float scale, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::cfg_combine((hipStream_t)stream, vc, vn, n, scale, e);
}

int kh_dit_layer_forward(kh_stream stream, const kh_dit_config* cfg, const kh_dit_layer* layer,
                         const kh_dit_state* state, int rows, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!cfg || !layer || !state) return e.fail("dit: null config / layer / state");
  return kh::dit_layer_forward((hipStream_t)stream, *cfg, *layer, *state, rows, e);
}

int kh_dit_forward(kh_stream stream, const kh_dit_config* cfg, const kh_dit_layer* layers, int n_layers,
                   const kh_dit_state* state, int rows, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!cfg || !state) return e.fail("dit: null config / state");
  return kh::dit_forward((hipStream_t)stream, *cfg, layers, n_layers, *state, rows, e);
}

/* ---- VAE decoder ---- */
int kh_vae_conv3x3(kh_stream stream, const void* x, int ldx, int C, int H, int W, int up, int dtype, const kh_weight* Wt,
                   int K, int N, const float* bias, const void* res, void* y, int ldy, void* workspace,
                   size_t workspace_bytes, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!Wt) return e.fail("conv3x3: null weight descriptor");
  const kh::GemmWs ws{workspace, workspace_bytes};
  return kh::conv3x3((hipStream_t)stream, x, ldx, C, H, W, up, dtype, *Wt, K, N, bias, res, y, ldy, e, &ws);
}

int kh_vae_subpix_weights(kh_stream stream, const void* W, int dtype, int Cin, int Cout, void* W2, int K, int Np,
                          const float* bias, float* bias4, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_subpix_weights((hipStream_t)stream, W, dtype, Cin, Cout, W2, K, Np, bias, bias4, e);
}

int kh_vae_conv_up2(kh_stream stream, const void* x, int ldx, int C, int H, int W, int dtype, const kh_weight* W2, int K,
                    int Np, const float* bias4, void* y, int ldy, void* workspace, size_t workspace_bytes, char* err,
                    int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!W2) return e.fail("conv_up2: null weight descriptor");
  const kh::GemmWs ws{workspace, workspace_bytes};
  return kh::conv_up2_subpix((hipStream_t)stream, x, ldx, C, H, W, dtype, *W2, K, Np, bias4, y, ldy, e, &ws);
}

int kh_vae_im2col(kh_stream stream, const void* x, int ldx, int C, int H, int W, int up, int m0, int rows, void* col,
                  int Kpad, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_im2col((hipStream_t)stream, x, ldx, C, H, W, up, m0, rows, col, Kpad, e);
}

int kh_vae_norm_silu(kh_stream stream, const void* x, int ldx, const float* gamma, void* y, int ldy, int P, int C,
                     int silu, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_norm_silu((hipStream_t)stream, x, ldx, gamma, y, ldy, P, C, silu, e);
}

int kh_vae_unpack(kh_stream stream, const float* z, const float* mean, const float* stdv, const float* w,
                  const float* b, void* y, int H16, int W16, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_unpack((hipStream_t)stream, z, mean, stdv, w, b, y, H16, W16, e);
}

int kh_vae_softmax(kh_stream stream, const float* S, int ld, int rows, int n, float scale, void* P, char* err,
                   int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_softmax((hipStream_t)stream, S, ld, rows, n, scale, P, e);
}

int kh_vae_conv_out(kh_stream stream, const void* x, int ldx, int C, const void* w, const float* bias, void* rgba,
                    int H, int W, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_conv_out((hipStream_t)stream, x, ldx, C, w, bias, rgba, H, W, e);
}

size_t kh_vae_workspace_bytes(int H16, int W16) { return kh::vae_workspace_bytes(H16, W16); }

int kh_vae_decode(kh_stream stream, const kh_qw* vae, const float* z, int H16, int W16, void* workspace,
                  size_t workspace_bytes, void* rgba, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::vae_decode((hipStream_t)stream, vae, z, H16, W16, workspace, workspace_bytes, rgba, e);
}

}  // extern "C"
