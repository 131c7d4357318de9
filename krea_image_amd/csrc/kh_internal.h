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

int gemm(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
         int lda, int ldw, int ldc, const void* vec, Err& e);

int attention(hipStream_t st, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
              int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
              int ldg, const float* QB, const float* KB, Err& e);

}  // namespace kh
