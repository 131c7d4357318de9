/* libkh: MI355X (gfx950) drop-in for the per-op GPU API of the shinoss/krea_image engine on the DiT
 * weight-GEMM hot path.
 *
 * The reference engine's op layer is the Objective-C++ class krea::Metal (engine/src/metal.h:44-167); its
 * callers (DiT::lin_qkvg / lin_o / lin_mlp / attend / layer, engine/src/model.mm:282-385) encode ops into
 * one command stream. libkh exports the same ops as a C ABI over HIP streams: plain pointers to device
 * memory, sizes and strides, no exceptions across the boundary. Every entry point returns 0 on success,
 * KH_EINVAL for an argument the op does not support (nothing is launched) or KH_EHIP when HIP reports a
 * launch error; `err` (if non-NULL) receives a NUL-terminated message of at most errlen bytes, the
 * convention of the reference's C ABI (engine/src/krea.h:57-73, engine/src/pipeline.mm:594-641).
 *
 * Ops are asynchronous on `stream` (a hipStream_t; NULL = the null stream) and never allocate.
 */
#ifndef KH_H
#define KH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kh_stream; /* hipStream_t */

enum { KH_OK = 0, KH_EINVAL = -1, KH_EHIP = -2 };

/* element types */
enum { KH_F32 = 0, KH_F16 = 1, KH_BF16 = 2, KH_I8 = 3 };

/* GEMM epilogues: engine/src/metal.h:37-38 (enum class Epi) and engine/kernels/gemm.metal:28-37.
 * "16" outputs use the activation type (bf16 in the reference engine, fp16 in the benchmark configs). */
enum {
  KH_EPI_STORE16 = 0,    /* C16 = acc                                            (Epi::BF16)      */
  KH_EPI_F32 = 1,        /* C32 = acc                                            (Epi::F32)       */
  KH_EPI_RESID_GATE = 2, /* X32 += vec[n] * acc  (gated residual)                (Epi::ResidGate) */
  KH_EPI_RESID = 3,      /* X32 += acc                                           (Epi::Resid)     */
  KH_EPI_SWIGLU = 4,     /* C16[M, N/2] = silu(gate) * up, 64-column tiles [gate 32 | up 32]      */
  KH_EPI_GELU = 5,       /* C16 = gelu_tanh(acc)                                 (Epi::GELU)      */
  KH_EPI_BIAS16 = 6,     /* C16 = acc + vec[n]                                   (Epi::BiasBF16)  */
  KH_EPI_BIAS_F32 = 7    /* C32 = acc + vec[n]                                   (Epi::BiasF32)   */
};

/* A GEMM weight, input-major Wt[K, N] (row stride ldw), the layout tools/convert.py:117-130 writes.
 * Replaces struct krea::Weight {Tensor w, s; bool q8;} (engine/src/metal.h:25-29).
 *   w_dtype KH_F16 / KH_BF16: 16-bit weights (must equal the activation type); s unused.
 *   w_dtype KH_I8, group < K: symmetric int8 with scales s[K/group, N] (row stride ldw), dequantized per
 *       element as round16(q * s) like the reference's gemm_*_q8 kernels (group 128 and f32 scales in the
 *       reference's dit_q8.qw, tools/convert.py:92-99).
 *   w_dtype KH_I8, group == K: per-output-channel scales s[N] (fp16 or f32), applied to the fp32
 *       accumulator (q is exact in fp16/bf16), the format of tools/build_ane.py:79-80.
 * s_dtype: KH_F32, KH_F16 or KH_BF16. */
typedef struct kh_weight {
  const void* w;
  const void* s;
  int w_dtype;
  int s_dtype;
  int group;
} kh_weight;

/* acc[M, N] = A[M, K] (a_dtype KH_F16 / KH_BF16, row stride lda) x Wt[K, N], fp32 accumulation, then
 * `epi`. vec: f32 [N] gate (RESID_GATE) or bias (BIAS16 / BIAS_F32), else unused. C row stride ldc in
 * elements of the output type. Constraints: M > 0, N % 64 == 0, K % 64 == 0, int8 group % 64 == 0,
 * 16-byte aligned A / W rows (lda % 8 == 0, ldw % 16 == 0 for int8, % 8 for 16-bit).
 * Replaces krea::Metal::gemm (engine/src/metal.h:66-69, engine/src/metal.mm:146-163). */
int kh_gemm(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N, int K,
            int lda, int ldw, int ldc, const void* vec, char* err, int errlen);

/* Flash attention, head dim 128: O[q, h] = softmax_k(Q[q,h] . K[k, h/group] / sqrt(128) (+ QB[q,h] KB[k,h/group]))
 * V[k, h/group] (* sigmoid(G[q, h]) if G), fp32 scores / softmax / accumulation, P rounded to the 16-bit type
 * before P V. Q [Lq, ldq], K [Lk, ldk], V [Lk, ldv], O [Lq, ldo], G [Lq, ldg] (dtype KH_F16 / KH_BF16), head h at
 * column 128 h (kv head at 128 (h / group)). causal: key k visible to query i iff k <= i + q_pos0. QB [Lq, heads]
 * and KB [Lk, heads / group] (f32, both or neither): the rank-1 score term of a "big" head dimension.
 * Replaces krea::Metal::attention (engine/src/metal.h:86-88, engine/src/metal.mm:193-202). */
int kh_attention(kh_stream stream, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
                 int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
                 int ldg, const float* QB, const float* KB, char* err, int errlen);

/* Library identification (for the loader checks of the host bindings). */
const char* kh_version(void);

#ifdef __cplusplus
}
#endif
#endif
