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

int kh_attention(kh_stream stream, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
                 int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
                 int ldg, const float* QB, const float* KB, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  return kh::attention((hipStream_t)stream, Q, K, V, O, dtype, Lq, Lk, heads, ldq, ldk, ldv, ldo, group, causal,
                       q_pos0, G, ldg, QB, KB, e);
}

}  // extern "C"
