/* CPU restatement ("oracle") of the shinoss/krea_image dequant-GEMM + DiT-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker / the timed CPU baseline. The product path (libkh.so) never
 * links or calls it.
 *
 * Every function cites the reference file:line whose semantics it restates. Pinning (what checks each
 * function against something other than itself) is listed in the header of oracle.c.
 *
 * dtype codes are the ones of include/kh.h: 0 = f32, 1 = f16, 2 = bf16, 3 = i8.
 */
#ifndef KH_ORACLE_H
#define KH_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar conversions (round to nearest even) */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
void or_to_f32(const void* src, int dtype, float* dst, size_t n);
void or_from_f32(const float* src, int dtype, void* dst, size_t n);

/* tools/convert.py:92-99 (q8): group-symmetric int8 quantizer of an input-major W[K,N] (f32),
 * scale[g,n] = max(amax over the group's `group` rows, 1e-12) / 127, q = clamp(rint(w / scale), -127, 127).
 * group must divide K. Returns 0, or -1 on a bad shape. */
int or_quant_q8(const float* w, int K, int N, int group, int8_t* q, float* s);
/* tools/build_ane.py:79-80: per-output-channel int8 with an fp16 scale (q computed with the f32 scale). */
int or_quant_q8_channel_f16(const float* w, int K, int N, int8_t* q, uint16_t* s16);
/* tools/convert.py:102-114: gate/up [F, D] rows -> [2F, D] grouped per 64-row tile (32 gate | 32 up), and back.
 * elem = bytes per element (rows are copied as bytes). */
int or_interleave_gate_up(const void* gate, const void* up, int F, int D, int elem, void* out);
int or_deinterleave_gate_up(const void* gu, int F, int D, int elem, void* gate, void* up);

/* engine/kernels/gemm.metal:102-309 (gemm_tiled) + engine/src/metal.mm:146-163 (Metal::gemm):
 *   acc[M,N] = A[M,K] x W~[K,N] in fp32, then the epilogue `epi` (0 STORE16, 1 F32, 2 RESID_GATE,
 *   3 RESID, 4 SWIGLU, 5 GELU, 6 BIAS16, 7 BIAS_F32).
 * W~: w_dtype f16/bf16 -> as stored; w_dtype i8 with group < K -> round16(q * s[k/group, n]) (the Metal
 * kernel's in-tile dequant, gemm.metal:190-196, rounded to the activation type); i8 with group == K ->
 * exact q, and acc is multiplied by s[n] before the epilogue (per-output-channel format).
 * 16-bit outputs use a_dtype. Returns 0, or -1 on an unsupported shape. threads <= 0: all cores. */
int or_gemm(int epi, const void* A, int a_dtype, const void* w, int w_dtype, const void* s, int s_dtype,
            int group, void* C, int M, int N, int K, int lda, int ldw, int ldc, const float* vec, int threads);

/* engine/kernels/gemm.metal:346-371 (gemv_bf16) with an int8/16-bit weight and optional bias:
 * y[r,n] = (y if act&2) + sum_k act1(x[r,k]) W~[k,n] (+ bias[n]); act&1 = SiLU on load. x, y f32. */
int or_gemv(const float* x, const void* w, int w_dtype, const void* s, int s_dtype, int group, float* y, int rows,
            int N, int K, int ldw, int act, const float* bias);
/* engine/src/model.mm:576-581: timestep embedding e[256] of bf16(sigma). */
void or_temb(float sigma, float* e);
/* engine/src/model.mm:340-346: fin[2 D] from t [D], lin [2 D], nf [D]. */
void or_make_fin(const float* t, const float* lin, const float* nf, int D, float* fin);

/* engine/src/model.mm:317-347 (DiT::make_cond), one layer: v_j = tvec[j*D + k] (+ table[j*D + k]);
 * mods = [n1 (1 + v0), v1, v2, n2 (1 + v3), v4, v5]. */
void or_make_cond(const float* tvec, const float* table, const float* n1, const float* n2, int D, float* mods);

/* engine/kernels/norm.metal:28-55 (rms_norm): y = x * rrms * mul (+ add), rrms = 1/sqrt(mean(x^2) + eps);
 * center = 1 gives the LayerNorm variant (x - mean, variance about the mean). y dtype out_dtype. */
void or_rms_norm(const float* x, const float* mul, const float* add, void* y, int out_dtype, int rows, int width,
                 int ld_in, int ld_out, float eps, int center);

/* engine/kernels/norm.metal:81-134 (qk_norm_rope), in place on a 16-bit fused projection buffer. */
void or_qk_norm_rope(void* qkv, int dtype, const float* wq, const float* wk, const float* cosb, const float* sinb,
                     int rows, int ld, int q_off, int n_q, int k_off, int n_k, float eps, int rope_mode, int big_dim,
                     float* qbig, float* kbig);

/* RoPE tables [rows, 64] (cos, sin) for rows = T text rows + H*W image tokens.
 * mode 0: engine/src/model.mm:290-315 (3 axes, theta 1000, pairs 16/24/24, text rows at (0,0,0)).
 * mode 1: 2-D variant of the benchmark configs: theta 10000, pairs [0,32) by row i, [32,64) by column j,
 *         omega_p = theta^(-2 (p mod 32) / 64). */
void or_rope_tables(int T, int H, int W, int mode, float* cosb, float* sinb);

/* The sampler around the DiT forward (engine/src/pipeline.mm:300-316):
 * or_sigmas: krea_sigmas (engine/src/model.mm:594-602), steps + 1 floats;
 * or_euler_step: z += dt v (engine/kernels/norm.metal:234-238), one fused multiply-add per element;
 * or_cfg_combine: vc = vc + scale (vc - vn) (engine/kernels/norm.metal:259-262), difference then one fma. */
void or_sigmas(int steps, float mu, float* out);
void or_euler_step(float* z, const float* v, long long n, float dt);
void or_cfg_combine(float* vc, const float* vn, long long n, float scale);

/* engine/kernels/attention.metal:131-351 (attention_d128) + engine/src/metal.mm:193-202:
 * O = softmax(Q K^T / sqrt(128) (+ QB KB^T)) V (* sigmoid(G)), head dim 128, GQA group, optional causal
 * mask (key j visible to query i iff j <= i + q_pos0). Scores / softmax in fp32, P rounded to the 16-bit
 * type before P V (attention.metal:272-276), exact running max. */
void or_attention(const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk, int heads, int ldq,
                  int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G, int ldg, const float* QB,
                  const float* KB, int threads);

/* ---- VAE decoder ops (engine/kernels/vae.metal) ---- */
void or_vae_conv(const uint16_t* x, int H, int W, int Cin, int ks, int up, const uint16_t* w, const float* bias,
                 const uint16_t* res, int N, uint16_t* y);
void or_vae_norm_silu(const uint16_t* x, const float* gamma, uint16_t* y, int P, int C, int silu);
void or_vae_unpack(const float* z, const float* mean, const float* stdv, const float* w, const float* b, uint16_t* y,
                   int H16, int W16);
void or_vae_softmax(const float* S, int ld, int rows, int n, float scale, uint16_t* P);
void or_vae_conv_out(const uint16_t* x, int C, const uint16_t* w, const float* bias, uint8_t* rgba, int H, int W);

#ifdef __cplusplus
}
#endif
#endif
