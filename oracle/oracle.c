/* CPU restatement ("oracle") of the shinoss/krea_image dequant-GEMM + DiT-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels of libkh.so and the timed CPU baseline of
 * bench.py. Nothing in the product path links, loads or calls this file.
 *
 * Pinning (tests/test_oracle.py checks each function against something other than itself):
 *   or_f32_to_f16/bf16      numpy float16 casts; torch bfloat16 casts; hand-picked tie cases.
 *   or_quant_q8             closed-form known answers (hand-computed groups), round-half-even ties, and
 *                           numpy restatement of convert.py:92-99 on random data.
 *   or_quant_q8_channel_f16 numpy restatement of build_ane.py:79-80.
 *   or_(de)interleave       round trip, and explicit row map 64t+i <- gate 32t+i, 64t+32+i <- up 32t+i.
 *   or_gemm                 fp64 brute force (numpy) on small shapes for every epilogue and weight format;
 *                           identity-weight and permutation-weight invariants; K-split additivity;
 *                           torch gelu(approximate="tanh") and torch silu for the epilogue functions.
 *   or_gemv                 numpy fp64 matvec; torch silu / gelu(approximate="tanh") for the on-load activations.
 *   or_temb                 closed forms: sigma = 0 gives cos = 1, sin = 0; numpy float64 of the same formula
 *                           at bf16(sigma) (<= 1e-5 absolute); bf16 rounding of sigma checked against torch.
 *   or_make_fin             unit impulses in t and in each lin row: each moves only the fin entries that
 *                           model.mm:340-346 names, by nf[k] or 1 (a lin row swap or dropped term fails).
 *   or_make_cond            unit impulses at tvec[j*D+k] (and the table): exactly mods[j][k] moves, by n1[k],
 *                           n2[k] or 1 (model.mm:329-338; row meaning from DiT::layer, model.mm:374-382).
 *   or_rms_norm             numpy fp64; torch layer_norm for center = 1.
 *   or_qk_norm_rope         complex-multiplication form of RoPE (numpy); rotate-half vs pairs equivalence
 *                           under a channel permutation; norm of every head preserved by the rotation.
 *   or_rope_tables          closed form of model.mm:295-315 evaluated at chosen (i, j) positions.
 *   or_attention            torch scaled_dot_product_attention in fp64 (non-causal, causal, GQA); uniform-V
 *                           and one-hot-key invariants; sigmoid gate elementwise.
 *   or_sigmas               closed forms: mu = 0 gives the linear schedule t = 1 - i / steps; endpoints 1 and
 *                           0; strictly decreasing; the logistic identity log(s / (1 - s)) = mu + log(t / (1 - t)).
 *   or_euler_step,          numpy float64 of the update rounded once to f32 (exactly the single rounding of an
 *   or_cfg_combine          fma); dt = 0 / scale = 0 leave the input unchanged.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I8 = 3 };
enum { EPI_STORE16 = 0, EPI_F32, EPI_RESID_GATE, EPI_RESID, EPI_SWIGLU, EPI_GELU, EPI_BIAS16, EPI_BIAS_F32 };

/* ---------------------------------------------------------------------------------------------- */
/* 16-bit float conversions (IEEE binary16 and bfloat16), round to nearest even.                  */

float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ffu;
  float f;
  if (exp == 0) {
    f = ldexpf((float)man, -24); /* zero / subnormal */
    uint32_t u;
    memcpy(&u, &f, 4);
    u |= sign;
    memcpy(&f, &u, 4);
    return f;
  }
  uint32_t u;
  if (exp == 31) u = sign | 0x7f800000u | (man << 13);
  else u = sign | ((exp + 112) << 23) | (man << 13);
  memcpy(&f, &u, 4);
  return f;
}

uint16_t or_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const float a = fabsf(f);
  if (isnan(f)) return sign | 0x7e00u;
  if (a >= 65520.0f) return sign | 0x7c00u; /* rounds to inf */
  if (a < 6.103515625e-05f) {               /* subnormal range: quantum 2^-24 */
    const float q = rintf(a * 16777216.0f);  /* exact scaling, RNE */
    return sign | (uint16_t)q;
  }
  /* normal: keep 10 mantissa bits, RNE on the dropped 13 */
  uint32_t m = u & 0x7fffffffu;
  const uint32_t lsb = (m >> 13) & 1u;
  m += 0xfffu + lsb;
  const uint32_t exp = (m >> 23) - 112;
  return sign | (uint16_t)((exp << 10) | ((m >> 13) & 0x3ffu));
}

float or_bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* engine/src/model.mm:17-24 (bf16_round): add 0x7FFF + lsb, truncate. NaN kept quiet. */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if (isnan(f)) return (uint16_t)((u >> 16) | 0x40u);
  u = u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float round16(float x, int dtype) {
  return dtype == DT_BF16 ? or_bf16_to_f32(or_f32_to_bf16(x)) : or_f16_to_f32(or_f32_to_f16(x));
}

static inline float load_elem(const void* p, int dtype, size_t i) {
  switch (dtype) {
    case DT_F32: return ((const float*)p)[i];
    case DT_F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
    case DT_BF16: return or_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return (float)((const int8_t*)p)[i];
  }
}

static inline void store_elem(void* p, int dtype, size_t i, float v) {
  switch (dtype) {
    case DT_F32: ((float*)p)[i] = v; break;
    case DT_F16: ((uint16_t*)p)[i] = or_f32_to_f16(v); break;
    case DT_BF16: ((uint16_t*)p)[i] = or_f32_to_bf16(v); break;
    default: ((int8_t*)p)[i] = (int8_t)v; break;
  }
}

void or_to_f32(const void* src, int dtype, float* dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = load_elem(src, dtype, i);
}

void or_from_f32(const float* src, int dtype, void* dst, size_t n) {
  for (size_t i = 0; i < n; i++) store_elem(dst, dtype, i, src[i]);
}

/* ---------------------------------------------------------------------------------------------- */
/* Quantizers and the SwiGLU weight interleave.                                                   */

/* tools/convert.py:92-99 */
int or_quant_q8(const float* w, int K, int N, int group, int8_t* q, float* s) {
  if (K <= 0 || N <= 0 || group <= 0 || K % group) return -1;
  for (int g = 0; g < K / group; g++)
    for (int n = 0; n < N; n++) {
      float amax = 0.f;
      for (int r = 0; r < group; r++) amax = fmaxf(amax, fabsf(w[(size_t)(g * group + r) * N + n]));
      const float sc = fmaxf(amax, 1e-12f) / 127.0f;
      s[(size_t)g * N + n] = sc;
      for (int r = 0; r < group; r++) {
        const size_t i = (size_t)(g * group + r) * N + n;
        float v = rintf(w[i] / sc); /* torch.round: half to even (default FP rounding mode) */
        v = fminf(fmaxf(v, -127.f), 127.f);
        q[i] = (int8_t)v;
      }
    }
  return 0;
}

/* tools/build_ane.py:79-80 (per output channel; the scale is stored as fp16, q uses the f32 scale) */
int or_quant_q8_channel_f16(const float* w, int K, int N, int8_t* q, uint16_t* s16) {
  if (K <= 0 || N <= 0) return -1;
  float* s = (float*)malloc(sizeof(float) * (size_t)N);
  if (!s) return -1;
  int rc = or_quant_q8(w, K, N, K, q, s);
  for (int n = 0; n < N; n++) s16[n] = or_f32_to_f16(s[n]);
  free(s);
  return rc;
}

/* tools/convert.py:102-107 */
int or_interleave_gate_up(const void* gate, const void* up, int F, int D, int elem, void* out) {
  if (F % 32) return -1;
  const size_t row = (size_t)D * elem;
  for (int t = 0; t < F / 32; t++)
    for (int i = 0; i < 32; i++) {
      memcpy((char*)out + (size_t)(64 * t + i) * row, (const char*)gate + (size_t)(32 * t + i) * row, row);
      memcpy((char*)out + (size_t)(64 * t + 32 + i) * row, (const char*)up + (size_t)(32 * t + i) * row, row);
    }
  return 0;
}

/* tools/convert.py:110-114 */
int or_deinterleave_gate_up(const void* gu, int F, int D, int elem, void* gate, void* up) {
  if (F % 32) return -1;
  const size_t row = (size_t)D * elem;
  for (int t = 0; t < F / 32; t++)
    for (int i = 0; i < 32; i++) {
      memcpy((char*)gate + (size_t)(32 * t + i) * row, (const char*)gu + (size_t)(64 * t + i) * row, row);
      memcpy((char*)up + (size_t)(32 * t + i) * row, (const char*)gu + (size_t)(64 * t + 32 + i) * row, row);
    }
  return 0;
}

/* ---------------------------------------------------------------------------------------------- */
/* Epilogue math, engine/kernels/common.h:23-29.                                                  */

static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
static inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
static inline float gelu_tanh_f(float x) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
}

/* ---------------------------------------------------------------------------------------------- */
/* GEMM: dequantize W into an f32 panel, convert A, blocked fp32 GEMM, epilogue.                  */

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

/* acc[M,N] (ld N) = Af[M,K] (ld K) x Wf[K,N] (ld N), fp32; rows in blocks of 4, columns of 64, K of 256. */
static void sgemm_blocked(const float* Af, const float* Wf, float* acc, int M, int N, int K) {
  const int MB = 4, NB = 64, KB = 256;
  const int mblocks = (M + MB - 1) / MB, nblocks = (N + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
  for (int nb = 0; nb < nblocks; nb++)
    for (int mb = 0; mb < mblocks; mb++) {
      const int n0 = nb * NB, n1 = n0 + NB < N ? n0 + NB : N;
      const int m0 = mb * MB, m1 = m0 + MB < M ? m0 + MB : M;
      float c[4][64];
      memset(c, 0, sizeof(c));
      for (int k0 = 0; k0 < K; k0 += KB) {
        const int k1 = k0 + KB < K ? k0 + KB : K;
        if (m1 - m0 == 4 && n1 - n0 == 64) {
          for (int k = k0; k < k1; k++) {
            const float* wr = Wf + (size_t)k * N + n0;
            const float a0 = Af[(size_t)(m0 + 0) * K + k], a1 = Af[(size_t)(m0 + 1) * K + k];
            const float a2 = Af[(size_t)(m0 + 2) * K + k], a3 = Af[(size_t)(m0 + 3) * K + k];
            for (int j = 0; j < 64; j++) {
              const float wv = wr[j];
              c[0][j] += a0 * wv;
              c[1][j] += a1 * wv;
              c[2][j] += a2 * wv;
              c[3][j] += a3 * wv;
            }
          }
        } else {
          for (int m = m0; m < m1; m++)
            for (int k = k0; k < k1; k++) {
              const float a = Af[(size_t)m * K + k];
              const float* wr = Wf + (size_t)k * N;
              for (int n = n0; n < n1; n++) c[m - m0][n - n0] += a * wr[n];
            }
        }
      }
      for (int m = m0; m < m1; m++)
        for (int n = n0; n < n1; n++) acc[(size_t)m * N + n] = c[m - m0][n - n0];
    }
}

/* W~ as an f32 panel [K, N] (see the header for the three weight formats) */
static void dequant_panel(const void* w, int w_dtype, const void* s, int s_dtype, int group, int a_dtype, int K, int N,
                          int ldw, float* Wf) {
#pragma omp parallel for schedule(static)
  for (int k = 0; k < K; k++)
    for (int n = 0; n < N; n++) {
      const size_t i = (size_t)k * ldw + n;
      float v = load_elem(w, w_dtype, i);
      if (w_dtype == DT_I8 && group < K) v = round16(v * load_elem(s, s_dtype, (size_t)(k / group) * ldw + n), a_dtype);
      Wf[(size_t)k * N + n] = v;
    }
}

int or_gemm(int epi, const void* A, int a_dtype, const void* w, int w_dtype, const void* s, int s_dtype, int group,
            void* C, int M, int N, int K, int lda, int ldw, int ldc, const float* vec, int threads) {
  if (M <= 0 || N <= 0 || K <= 0 || (a_dtype != DT_F16 && a_dtype != DT_BF16)) return -1;
  if (w_dtype == DT_I8 && (group <= 0 || K % group)) return -1;
  if (w_dtype != DT_I8 && w_dtype != a_dtype) return -1;
  if (epi == EPI_SWIGLU && N % 64) return -1;
  set_threads(threads);
  float* Af = (float*)malloc(sizeof(float) * (size_t)M * K);
  float* Wf = (float*)malloc(sizeof(float) * (size_t)K * N);
  float* acc = (float*)malloc(sizeof(float) * (size_t)M * N);
  if (!Af || !Wf || !acc) {
    free(Af);
    free(Wf);
    free(acc);
    return -1;
  }
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++)
    for (int k = 0; k < K; k++) Af[(size_t)m * K + k] = load_elem(A, a_dtype, (size_t)m * lda + k);
  dequant_panel(w, w_dtype, s, s_dtype, group, a_dtype, K, N, ldw, Wf);
  sgemm_blocked(Af, Wf, acc, M, N, K);
  const int per_channel = (w_dtype == DT_I8 && group == K);

#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++) {
    float* ar = acc + (size_t)m * N;
    if (per_channel)
      for (int n = 0; n < N; n++) ar[n] *= load_elem(s, s_dtype, n);
    const size_t o = (size_t)m * ldc;
    if (epi == EPI_SWIGLU) { /* gemm.metal:262-279 with convert.py:102-107 tile interleave */
      for (int t = 0; t < N / 64; t++)
        for (int i = 0; i < 32; i++)
          store_elem(C, a_dtype, o + 32 * t + i, silu_f(ar[64 * t + i]) * ar[64 * t + 32 + i]);
      continue;
    }
    for (int n = 0; n < N; n++) {
      const float v = ar[n];
      switch (epi) {
        case EPI_STORE16: store_elem(C, a_dtype, o + n, v); break;
        case EPI_F32: ((float*)C)[o + n] = v; break;
        case EPI_RESID_GATE: ((float*)C)[o + n] += v * vec[n]; break;
        case EPI_RESID: ((float*)C)[o + n] += v; break;
        case EPI_GELU: store_elem(C, a_dtype, o + n, gelu_tanh_f(v)); break;
        case EPI_BIAS16: store_elem(C, a_dtype, o + n, v + vec[n]); break;
        case EPI_BIAS_F32: ((float*)C)[o + n] = v + vec[n]; break;
      }
    }
  }
  free(Af);
  free(Wf);
  free(acc);
  return 0;
}

/* ---------------------------------------------------------------------------------------------- */
/* GEMV (adaLN modulation linear) and make_cond.                                                  */

int or_gemv(const float* x, const void* w, int w_dtype, const void* s, int s_dtype, int group, float* y, int rows,
            int N, int K, int ldw, int act, const float* bias) {
  if (rows <= 0 || N <= 0 || K <= 0) return -1;
  if (w_dtype == DT_I8 && (group <= 0 || K % group)) return -1;
  const int per_channel = (w_dtype == DT_I8 && group == K);
  for (int r = 0; r < rows; r++) {
    float* xa = (float*)malloc(sizeof(float) * (size_t)K);
    if (!xa) return -1;
    for (int k = 0; k < K; k++) {
      const float v = x[(size_t)r * K + k];
      xa[k] = (act & 1) ? silu_f(v) : (act & 4) ? gelu_tanh_f(v) : v;
    }
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
      double acc = 0.0;
      for (int k = 0; k < K; k++) {
        float wv = load_elem(w, w_dtype, (size_t)k * ldw + n);
        if (w_dtype == DT_I8 && !per_channel) wv *= load_elem(s, s_dtype, (size_t)(k / group) * ldw + n);
        acc += (double)xa[k] * wv;
      }
      float v = (float)acc;
      if (per_channel) v *= load_elem(s, s_dtype, n);
      if (bias) v += bias[n];
      y[(size_t)r * N + n] = (act & 2) ? y[(size_t)r * N + n] + v : v;
    }
    free(xa);
  }
  return 0;
}

/* Timestep embedding of Conditioning::compute (engine/src/model.mm:576-581): e[i] = cos(ts 1000 f_i),
 * e[128 + i] = sin(ts 1000 f_i), f_i = exp(-log(10000) i / 128), ts = bf16(sigma); float arithmetic as written
 * there. */
void or_temb(float sigma, float* e) {
  const float ts = or_bf16_to_f32(or_f32_to_bf16(sigma));
  for (int i = 0; i < 128; i++) {
    const float f = expf(-logf(10000.0f) * (float)i / 128.0f);
    e[i] = cosf(ts * 1000.0f * f);
    e[128 + i] = sinf(ts * 1000.0f * f);
  }
}

/* engine/src/model.mm:340-346 (the final-norm vectors of DiT::make_cond) */
void or_make_fin(const float* t, const float* lin, const float* nf, int D, float* fin) {
  for (int k = 0; k < D; k++) {
    fin[k] = nf[k] * (1.0f + t[k] + lin[k]);
    fin[D + k] = t[k] + lin[D + k];
  }
}

/* engine/src/model.mm:329-338 */
void or_make_cond(const float* tvec, const float* table, const float* n1, const float* n2, int D, float* mods) {
  for (int k = 0; k < D; k++) {
    float v[6];
    for (int j = 0; j < 6; j++) v[j] = tvec[j * D + k] + (table ? table[j * D + k] : 0.f);
    mods[k] = n1[k] * (1.0f + v[0]);
    mods[D + k] = v[1];
    mods[2 * D + k] = v[2];
    mods[3 * D + k] = n2[k] * (1.0f + v[3]);
    mods[4 * D + k] = v[4];
    mods[5 * D + k] = v[5];
  }
}

/* ---------------------------------------------------------------------------------------------- */
/* Norms and RoPE.                                                                                */

/* engine/kernels/norm.metal:28-55 */
void or_rms_norm(const float* x, const float* mul, const float* add, void* y, int out_dtype, int rows, int width,
                 int ld_in, int ld_out, float eps, int center) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * ld_in;
    double mean = 0.0;
    if (center) {
      for (int c = 0; c < width; c++) mean += xr[c];
      mean /= width;
    }
    double q = 0.0;
    for (int c = 0; c < width; c++) q += ((double)xr[c] - mean) * ((double)xr[c] - mean);
    const float rrms = (float)(1.0 / sqrt(q / width + (double)eps));
    for (int c = 0; c < width; c++) {
      float o = ((float)(xr[c] - mean)) * rrms * mul[c];
      if (add) o += add[c];
      store_elem(y, out_dtype, (size_t)r * ld_out + c, o);
    }
  }
}

/* engine/kernels/norm.metal:81-134 */
void or_qk_norm_rope(void* qkv, int dtype, const float* wq, const float* wk, const float* cosb, const float* sinb,
                     int rows, int ld, int q_off, int n_q, int k_off, int n_k, float eps, int rope_mode, int big_dim,
                     float* qbig, float* kbig) {
  const int heads = n_q + n_k;
#pragma omp parallel for schedule(static)
  for (int u = 0; u < rows * heads; u++) {
    const int row = u / heads, hh = u % heads;
    const int is_q = hh < n_q;
    const int col = is_q ? q_off + hh * 128 : k_off + (hh - n_q) * 128;
    const size_t base = (size_t)row * ld + col;
    const float* w = is_q ? wq : wk;
    float x[128], o[128];
    double ss = 0.0;
    for (int d = 0; d < 128; d++) {
      x[d] = load_elem(qkv, dtype, base + d);
      ss += (double)x[d] * x[d];
    }
    const float rrms = (float)(1.0 / sqrt(ss / 128.0 + (double)eps));
    for (int d = 0; d < 128; d++) x[d] = x[d] * rrms * w[d];
    const float* cr = cosb ? cosb + (size_t)row * 64 : NULL;
    const float* sr = sinb ? sinb + (size_t)row * 64 : NULL;
    if (rope_mode == 0) { /* interleaved pairs (2i, 2i+1) at frequency i */
      for (int i = 0; i < 64; i++) {
        const float c = cr[i], s = sr[i];
        o[2 * i] = x[2 * i] * c - x[2 * i + 1] * s;
        o[2 * i + 1] = x[2 * i] * s + x[2 * i + 1] * c;
      }
    } else if (rope_mode == 1) { /* rotate-half: channel i pairs with i + 64 at frequency i */
      for (int i = 0; i < 64; i++) {
        const float c = cr[i], s = sr[i];
        o[i] = x[i] * c - x[i + 64] * s;
        o[i + 64] = x[i + 64] * c + x[i] * s;
      }
    } else {
      memcpy(o, x, sizeof(o));
    }
    if (big_dim >= 0) {
      if (is_q) qbig[(size_t)row * n_q + hh] = o[big_dim];
      else kbig[(size_t)row * n_k + (hh - n_q)] = o[big_dim];
      o[big_dim] = 0.f;
    }
    for (int d = 0; d < 128; d++) store_elem(qkv, dtype, base + d, o[d]);
  }
}

void or_rope_tables(int T, int H, int W, int mode, float* cosb, float* sinb) {
  double om[64];
  for (int p = 0; p < 64; p++) {
    if (mode == 0) { /* engine/src/model.mm:295-299 */
      const int ax = p < 16 ? 0 : p < 40 ? 1 : 2, k = p - (ax == 0 ? 0 : ax == 1 ? 16 : 40), d = ax == 0 ? 32 : 48;
      om[p] = 1.0 / pow(1000.0, (2.0 * k) / d);
    } else {
      om[p] = 1.0 / pow(10000.0, (2.0 * (p % 32)) / 64.0);
    }
  }
  const int R = T + H * W;
  for (int r = 0; r < R; r++) {
    const int k = r - T;
    const double pi = r < T ? 0 : k / W, pj = r < T ? 0 : k % W;
    for (int p = 0; p < 64; p++) {
      double a;
      if (mode == 0) a = (p < 16 ? 0.0 : p < 40 ? pi : pj) * om[p];
      else a = (p < 32 ? pi : pj) * om[p];
      cosb[(size_t)r * 64 + p] = (float)cos(a);
      sinb[(size_t)r * 64 + p] = (float)sin(a);
    }
  }
}

/* ---------------------------------------------------------------------------------------------- */
/* Attention.                                                                                     */

void or_attention(const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk, int heads, int ldq,
                  int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G, int ldg, const float* QB,
                  const float* KB, int threads) {
  set_threads(threads);
  const int kvh_n = heads / group;
  const float scale = (float)(1.0 / sqrt(128.0));
  /* K and V of every kv head to f32 once */
  float* Kf = (float*)malloc(sizeof(float) * (size_t)Lk * kvh_n * 128);
  float* Vf = (float*)malloc(sizeof(float) * (size_t)Lk * kvh_n * 128);
  if (!Kf || !Vf) {
    free(Kf);
    free(Vf);
    return;
  }
#pragma omp parallel for schedule(static)
  for (int j = 0; j < Lk; j++)
    for (int c = 0; c < kvh_n * 128; c++) {
      Kf[(size_t)j * kvh_n * 128 + c] = load_elem(K, dtype, (size_t)j * ldk + c);
      Vf[(size_t)j * kvh_n * 128 + c] = load_elem(V, dtype, (size_t)j * ldv + c);
    }
#pragma omp parallel for schedule(dynamic, 4)
  for (int u = 0; u < Lq * heads; u++) {
    const int i = u / heads, h = u % heads, kvh = h / group;
    float q[128], o[128];
    for (int d = 0; d < 128; d++) q[d] = load_elem(Q, dtype, (size_t)i * ldq + h * 128 + d);
    float* sc = (float*)malloc(sizeof(float) * (size_t)Lk);
    float mx = -INFINITY;
    int kend = Lk;
    if (causal) kend = i + q_pos0 + 1 < Lk ? i + q_pos0 + 1 : Lk;
    for (int j = 0; j < kend; j++) {
      const float* kr = Kf + (size_t)j * kvh_n * 128 + kvh * 128;
      float s = 0.f;
      for (int d = 0; d < 128; d++) s += q[d] * kr[d];
      if (QB && KB) s += QB[(size_t)i * heads + h] * KB[(size_t)j * kvh_n + kvh];
      sc[j] = s * scale;
      mx = fmaxf(mx, sc[j]);
    }
    for (int d = 0; d < 128; d++) o[d] = 0.f;
    float l = 0.f;
    for (int j = 0; j < kend; j++) {
      const float p = expf(sc[j] - mx);
      l += p;
      const float pr = round16(p, dtype);
      const float* vr = Vf + (size_t)j * kvh_n * 128 + kvh * 128;
      for (int d = 0; d < 128; d++) o[d] += pr * vr[d];
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    for (int d = 0; d < 128; d++) {
      float g = 1.f;
      if (G && ldg > 0) g = sigmoid_f(load_elem(G, dtype, (size_t)i * ldg + h * 128 + d));
      store_elem(O, dtype, (size_t)i * ldo + h * 128 + d, o[d] * inv * g);
    }
    free(sc);
  }
  free(Kf);
  free(Vf);
}

/* ---------------------------------------------------------------------------------------------- */
/* VAE decoder ops (engine/kernels/vae.metal), NHWC bf16 activations [pixel, channel].            */

/* vconv (vae.metal:5-128): out[p, n] = bf16(bias[n] + sum_{tap, ci} in[src(p, tap), ci] * Wt[tap*Cin + ci, n]
 * (+ res[p, n])), fp32 accumulation; ks = 1 or 3 (zero padding ks / 2); up = 1: the input is H/2 x W/2,
 * nearest-upsampled. The residual joins the fp32 sum before the single 16-bit rounding. */
void or_vae_conv(const uint16_t* x, int H, int W, int Cin, int ks, int up, const uint16_t* w, const float* bias,
                 const uint16_t* res, int N, uint16_t* y) {
  const int Win = up ? W / 2 : W;
  float* wf = (float*)malloc((size_t)ks * ks * Cin * N * sizeof(float));
  for (size_t i = 0; i < (size_t)ks * ks * Cin * N; i++) wf[i] = or_bf16_to_f32(w[i]);
#pragma omp parallel for schedule(static)
  for (int p = 0; p < H * W; p++) {
    const int py = p / W, px = p % W;
    float acc[1024];
    for (int n0 = 0; n0 < N; n0 += 1024) {  /* output channels in blocks of 1024 */
      const int nb = N - n0 < 1024 ? N - n0 : 1024;
      for (int n = 0; n < nb; n++) acc[n] = 0.f;
      for (int tap = 0; tap < ks * ks; tap++) {
        int sy = py + (ks == 3 ? tap / 3 - 1 : 0), sx = px + (ks == 3 ? tap % 3 - 1 : 0);
        if (sy < 0 || sy >= H || sx < 0 || sx >= W) continue;
        if (up) {
          sy >>= 1;
          sx >>= 1;
        }
        const uint16_t* xi = x + ((size_t)sy * Win + sx) * Cin;
        const float* wt = wf + (size_t)tap * Cin * N + n0;
        for (int ci = 0; ci < Cin; ci++) {
          const float a = or_bf16_to_f32(xi[ci]);
          const float* wr = wt + (size_t)ci * N;
          for (int n = 0; n < nb; n++) acc[n] += a * wr[n];
        }
      }
      for (int n = 0; n < nb; n++) {
        float v = acc[n] + bias[n0 + n];
        if (res) v += or_bf16_to_f32(res[(size_t)p * N + n0 + n]);
        y[(size_t)p * N + n0 + n] = or_f32_to_bf16(v);
      }
    }
  }
  free(wf);
}

/* vae_norm_silu (vae.metal:588-621): y = x * sqrt(C) / max(||x||, 1e-12) * gamma, SiLU optional. */
void or_vae_norm_silu(const uint16_t* x, const float* gamma, uint16_t* y, int P, int C, int silu) {
#pragma omp parallel for schedule(static)
  for (int p = 0; p < P; p++) {
    const uint16_t* xr = x + (size_t)p * C;
    float ss = 0.f;
    for (int c = 0; c < C; c++) {
      const float v = or_bf16_to_f32(xr[c]);
      ss += v * v;
    }
    const float scale = sqrtf((float)C) / fmaxf(sqrtf(ss), 1e-12f);
    for (int c = 0; c < C; c++) {
      float t = or_bf16_to_f32(xr[c]) * scale * gamma[c];
      if (silu) t = silu_f(t);
      y[(size_t)p * C + c] = or_f32_to_bf16(t);
    }
  }
}

/* vae_unpack_pq (vae.metal:690-712) */
void or_vae_unpack(const float* z, const float* mean, const float* stdv, const float* w, const float* b, uint16_t* y,
                   int H16, int W16) {
  const int W2 = 2 * W16;
  for (int pix = 0; pix < 4 * H16 * W16; pix++) {
    const int yy = pix / W2, xx = pix % W2;
    const float* zt = z + (size_t)((yy >> 1) * W16 + (xx >> 1)) * 64 + (yy & 1) * 2 + (xx & 1);
    float u[16];
    for (int c = 0; c < 16; c++) u[c] = zt[c * 4] * stdv[c] + mean[c];
    for (int o = 0; o < 16; o++) {
      float acc = b[o];
      for (int c = 0; c < 16; c++) acc += w[c * 16 + o] * u[c];
      y[(size_t)pix * 16 + o] = or_f32_to_bf16(acc);
    }
  }
}

/* softmax_rows (vae.metal:727-757): P[r, :n] = bf16(softmax(S[r, :n] * scale)) */
void or_vae_softmax(const float* S, int ld, int rows, int n, float scale, uint16_t* P) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) {
    const float* s = S + (size_t)r * ld;
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, s[i] * scale);
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += expf(s[i] * scale - mx);
    const float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) P[(size_t)r * ld + i] = or_f32_to_bf16(expf(s[i] * scale - mx) * inv);
  }
}

/* vae_conv_out_rgba (vae.metal:759-785) */
void or_vae_conv_out(const uint16_t* x, int C, const uint16_t* w, const float* bias, uint8_t* rgba, int H, int W) {
#pragma omp parallel for schedule(static)
  for (int pix = 0; pix < H * W; pix++) {
    const int y = pix / W, xx = pix % W;
    float acc[4] = {bias[0], bias[1], bias[2], bias[3]};
    for (int tap = 0; tap < 9; tap++) {
      const int sy = y + tap / 3 - 1, sx = xx + tap % 3 - 1;
      if (sy < 0 || sy >= H || sx < 0 || sx >= W) continue;
      const uint16_t* ip = x + ((size_t)sy * W + sx) * C;
      const uint16_t* wp = w + (size_t)tap * C * 4;
      for (int c = 0; c < C; c++)
        for (int k = 0; k < 4; k++) acc[k] += or_bf16_to_f32(ip[c]) * or_bf16_to_f32(wp[(size_t)c * 4 + k]);
    }
    for (int k = 0; k < 4; k++) {
      float a = fminf(fmaxf(acc[k], -1.f), 1.f);
      a = rintf(fminf(fmaxf(a * 0.5f + 0.5f, 0.f), 1.f) * 255.f);
      rgba[(size_t)pix * 4 + k] = (uint8_t)a;
    }
  }
}

/* ---------------------------------------------------------------------------------------------- */
/* Sampler: engine/src/model.mm:594-602 (krea_sigmas), engine/kernels/norm.metal:234-238 (euler_step) and
 * 259-262 (cfg_combine).                                                                          */

void or_sigmas(int steps, float mu, float* out) {
  const double e = exp((double)mu);
  for (int i = 0; i <= steps; i++) {
    const double t = 1.0 - (double)i / steps;
    out[i] = t <= 0 ? 0.0f : (float)(e / (e + (1.0 / t - 1.0)));
  }
}

void or_euler_step(float* z, const float* v, long long n, float dt) {
  for (long long i = 0; i < n; i++) z[i] = fmaf(dt, v[i], z[i]);
}

void or_cfg_combine(float* vc, const float* vn, long long n, float scale) {
  for (long long i = 0; i < n; i++) vc[i] = fmaf(scale, vc[i] - vn[i], vc[i]);
}
