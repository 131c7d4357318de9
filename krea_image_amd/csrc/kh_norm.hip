// The DiT ops either side of the GEMMs on MI355X (gfx950): modulated RMSNorm / LayerNorm, per-head QK
// RMSNorm + RoPE, the adaLN modulation GEMV (SiLU on load, int8 weights), the modulation vectors, and the
// small fp32 GEMM of the patch embed / final projection. All are HBM-bound elementwise or GEMV work: one
// pass over their data with 16-byte vector accesses, reductions in registers / LDS, no MFMA.
#include "kh_common.h"
#include "kh_internal.h"

namespace kh {

namespace {

// ---- sum over a wave64 (DPP / permute shuffles) ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ------------------------------------------------------------------------------------------------------
// Row norm with modulation: engine/kernels/norm.metal:28-55. y = (x - mu) * rrms * mul (+ add), mu = 0 for
// RMSNorm (center = 0) or the row mean for LayerNorm (center = 1); fp32 math, one rounding at the store.
// One 256-thread workgroup per row; the row (<= 16 KB of f32) stays in registers between the passes.
template <int OUT, bool CENTER, bool ADD>
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ mul,
                                                       const float* __restrict__ add, void* __restrict__ y,
                                                       int width, int ld_in, int ld_out, float eps) {
  __shared__ float red[2][4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const f32x4* xr = (const f32x4*)(x + (size_t)row * ld_in);
  const int n4 = width / 4;
  constexpr int MAXV = 8;  // float4 per thread: width <= 8192
  f32x4 v[MAXV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; i++) {
    const int c = tid + i * 256;
    v[i] = c < n4 ? xr[c] : (f32x4){0.f, 0.f, 0.f, 0.f};
    s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
  }
  float mu = 0.f;
  if (CENTER) {
    s = wave_sum(s);
    if ((tid & 63) == 0) red[0][tid >> 6] = s;
    __syncthreads();
    mu = (red[0][0] + red[0][1] + red[0][2] + red[0][3]) / (float)width;
  }
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; i++) {
    const int c = tid + i * 256;
    if (c < n4)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float d = v[i][e] - mu;
        q += d * d;
      }
  }
  q = wave_sum(q);
  if ((tid & 63) == 0) red[1][tid >> 6] = q;
  __syncthreads();
  const float rrms = rsqrtf((red[1][0] + red[1][1] + red[1][2] + red[1][3]) / (float)width + eps);
  const f32x4* mv = (const f32x4*)mul;
  const f32x4* av = (const f32x4*)add;
#pragma unroll
  for (int i = 0; i < MAXV; i++) {
    const int c = tid + i * 256;
    if (c >= n4) continue;
    const f32x4 mm = mv[c];
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = (v[i][e] - mu) * rrms * mm[e];
    if (ADD) o += av[c];
    if constexpr (OUT == KH_F32) {
      ((f32x4*)((float*)y + (size_t)row * ld_out))[c] = o;
    } else {
      ((u32x2*)((uint16_t*)y + (size_t)row * ld_out))[c] =
          (u32x2){(uint32_t)to16<OUT>(o[0]) | ((uint32_t)to16<OUT>(o[1]) << 16),
                  (uint32_t)to16<OUT>(o[2]) | ((uint32_t)to16<OUT>(o[3]) << 16)};
    }
  }
}

// ------------------------------------------------------------------------------------------------------
// Per-head RMSNorm (weight [128]) + RoPE, in place on a 16-bit fused projection buffer:
// engine/kernels/norm.metal:81-134. One wave per (row, head); lane i owns the two channels of rotation
// pair i: (2i, 2i + 1) for rope_mode 0 (interleaved pairs), (i, i + 64) for rope_mode 1 (rotate-half) and
// for rope_mode 2 (no rotation). cos / sin: f32 [rows, 64]. big_dim >= 0: that dimension's rotated value
// goes to qbig [rows, n_q] / kbig [rows, n_k] in f32 and is zeroed in the buffer.
template <int DT>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(uint16_t* __restrict__ qkv, const float* __restrict__ wq,
                                                           const float* __restrict__ wk, const float* __restrict__ cosb,
                                                           const float* __restrict__ sinb, int rows, int ld, int q_off,
                                                           int n_q, int k_off, int n_k, float eps, int rope_mode,
                                                           int big_dim, float* __restrict__ qbig,
                                                           float* __restrict__ kbig) {
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int heads = n_q + n_k;
  const int row = unit / heads, hh = unit % heads;
  if (row >= rows) return;
  const bool is_q = hh < n_q;
  const int col = is_q ? q_off + hh * 128 : k_off + (hh - n_q) * 128;
  uint16_t* base = qkv + (size_t)row * ld + col;
  const float* w = is_q ? wq : wk;
  const int c0 = rope_mode == 0 ? 2 * lane : lane, c1 = rope_mode == 0 ? 2 * lane + 1 : lane + 64;
  float x0, x1;
  if (rope_mode == 0) {
    const uint32_t pr = *(const uint32_t*)(base + c0);
    x0 = from16<DT>((uint16_t)pr);
    x1 = from16<DT>((uint16_t)(pr >> 16));
  } else {
    x0 = from16<DT>(base[c0]);
    x1 = from16<DT>(base[c1]);
  }
  const float rrms = rsqrtf(wave_sum(x0 * x0 + x1 * x1) * (1.0f / 128.0f) + eps);
  x0 *= rrms * w[c0];
  x1 *= rrms * w[c1];
  float o0 = x0, o1 = x1;
  if (rope_mode != 2) {
    const float c = cosb[(size_t)row * 64 + lane], s = sinb[(size_t)row * 64 + lane];
    o0 = x0 * c - x1 * s;
    o1 = x0 * s + x1 * c;
  }
  if (big_dim >= 0) {
    float* dst = is_q ? qbig + (size_t)row * n_q + hh : kbig + (size_t)row * n_k + (hh - n_q);
    if (c0 == big_dim) {
      *dst = o0;
      o0 = 0.f;
    } else if (c1 == big_dim) {
      *dst = o1;
      o1 = 0.f;
    }
  }
  if (rope_mode == 0) {
    *(uint32_t*)(base + c0) = (uint32_t)to16<DT>(o0) | ((uint32_t)to16<DT>(o1) << 16);
  } else {
    base[c0] = to16<DT>(o0);
    base[c1] = to16<DT>(o1);
  }
}

// ------------------------------------------------------------------------------------------------------
// adaLN modulation GEMV: y[r, n] (+)= sum_k act(x[r, k]) W~[k, n] (+ bias[n]), rows <= 4, x / y f32.
// engine/kernels/gemm.metal:346-371 (gemv_bf16: act bit 0 = SiLU on load, bit 1 = accumulate) with the
// weight formats of kh_gemm. HBM-bound (the int8 weight is read once): grid (N / 256, KSPLIT); each
// workgroup reads a K / KSPLIT x 256 slab with one dword (4 columns) per lane and row, coalesced 256 B per
// wave; its 4 waves split the slab's rows, reduce through LDS and add into y with one f32 atomic per
// column. y is initialised (bias, or 0, or left for accumulation) by gemv_init before the split kernel.
constexpr int GEMV_COLS = 256, GEMV_KSPLIT_MAX = 32;

__global__ void gemv_init(float* y, const float* bias, int rows, int N, int ldy, int accumulate) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  for (int r = 0; r < rows; r++) {
    const float b = bias ? bias[n] : 0.f;
    float* yp = y + (size_t)r * ldy + n;
    *yp = accumulate ? *yp + b : b;
  }
}

template <int WF>  // 0: 16-bit weights (WD = dtype), 1: int8 per-channel, 2: int8 group
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, const void* __restrict__ W,
                                                   const void* __restrict__ S, int s_dtype, int group, int w16_dtype,
                                                   float* __restrict__ y, int rows, int N, int K, int ldw, int ldy,
                                                   int silu, int kchunk) {
  __shared__ float xs[4][1024];        // activated x of this slab (rows x kchunk), kchunk <= 1024
  __shared__ f32x4 part[4][4][64];     // [wave][row][lane]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = blockIdx.x * GEMV_COLS + lane * 4;
  const int k0 = blockIdx.y * kchunk, k1 = min(K, k0 + kchunk);
  for (int i = tid; i < rows * (k1 - k0); i += 256) {
    const int r = i / (k1 - k0), k = i % (k1 - k0);
    float v = x[(size_t)r * K + k0 + k];
    xs[r][k] = silu ? silu_f(v) : v;
  }
  __syncthreads();
  f32x4 acc[4] = {};
  if (n < N) {
    for (int k = k0 + wave; k < k1; k += 4) {
      float w4[4];
      if (WF == 0) {
        const u32x2 raw = *(const u32x2*)((const uint16_t*)W + (size_t)k * ldw + n);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint16_t hbits = (uint16_t)(raw[e >> 1] >> (16 * (e & 1)));
          w4[e] = w16_dtype == KH_BF16 ? from16<KH_BF16>(hbits) : from16<KH_F16>(hbits);
        }
      } else {
        const uint32_t raw = *(const uint32_t*)((const int8_t*)W + (size_t)k * ldw + n);
#pragma unroll
        for (int e = 0; e < 4; e++) w4[e] = (float)(int8_t)(raw >> (8 * e));
        if (WF == 2) {
#pragma unroll
          for (int e = 0; e < 4; e++) w4[e] *= load_scale(S, s_dtype, (size_t)(k / group) * ldw + n + e);
        }
      }
      for (int r = 0; r < rows; r++) {
        const float xv = xs[r][k - k0];
#pragma unroll
        for (int e = 0; e < 4; e++) acc[r][e] += xv * w4[e];
      }
    }
  }
  for (int r = 0; r < rows; r++) part[wave][r][lane] = acc[r];
  __syncthreads();
  if (wave == 0 && n < N) {
    for (int r = 0; r < rows; r++) {
      f32x4 s = part[0][r][lane] + part[1][r][lane] + part[2][r][lane] + part[3][r][lane];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float v = s[e];
        if (WF == 1) v *= load_scale(S, s_dtype, n + e);
        atomicAdd(y + (size_t)r * ldy + n + e, v);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------------
// Modulation vectors of one layer: engine/src/model.mm:329-338 (DiT::make_cond), on the device:
// v_j = tvec[j D + k] (+ table[j D + k]); mods = [n1 (1 + v0), v1, v2, n2 (1 + v3), v4, v5].
__global__ void make_cond_kernel(const float* tvec, const float* table, const float* n1, const float* n2, int D,
                                 float* mods) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= D) return;
  float v[6];
#pragma unroll
  for (int j = 0; j < 6; j++) v[j] = tvec[j * D + k] + (table ? table[j * D + k] : 0.f);
  mods[k] = n1[k] * (1.0f + v[0]);
  mods[D + k] = v[1];
  mods[2 * D + k] = v[2];
  mods[3 * D + k] = n2[k] * (1.0f + v[3]);
  mods[4 * D + k] = v[4];
  mods[5 * D + k] = v[5];
}

// ------------------------------------------------------------------------------------------------------
// fp32 GEMM of the patch embed (64 -> D) and the final projection (D -> 64): engine/kernels/f32gemm.metal
// (gemm_f32w) with its modes bit 0 bias, bit 1 GELU(tanh), bit 2 accumulate. 64 x 64 tiles, 256 threads,
// 4 x 4 outputs per thread, K staged 16 at a time through LDS. Tiny next to the DiT layers.
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ W,
                                                       float* __restrict__ C, const float* __restrict__ bias, int M,
                                                       int N, int K, int lda, int ldw, int ldc, int mode) {
  __shared__ float As[16][64 + 1];
  __shared__ float Ws[16][64];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = tid; i < 16 * 64; i += 256) {
      const int r = i / 16, c = i % 16;  // A tile: 64 rows x 16 k
      const int m = m0 + r, k = k0 + c;
      As[c][r] = (m < M && k < K) ? A[(size_t)m * lda + k] : 0.f;
      const int kr = i / 64, nc = i % 64;  // W tile: 16 k x 64 cols
      Ws[kr][nc] = (k0 + kr < K && n0 + nc < N) ? W[(size_t)(k0 + kr) * ldw + n0 + nc] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = As[k][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = Ws[k][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + tx * 4 + j;
      if (n >= N) continue;
      float v = acc[i][j];
      if (mode & 1) v += bias[n];
      if (mode & 2) v = gelu_tanh_f(v);
      float* cp = C + (size_t)m * ldc + n;
      *cp = (mode & 4) ? *cp + v : v;
    }
  }
}

}  // namespace

int rms_norm(hipStream_t st, const float* x, const float* mul, const float* add, void* y, int out_dtype, int rows,
             int width, int ld_in, int ld_out, float eps, int center, Err& e) {
  if (rows <= 0 || width <= 0) return e.fail("rms_norm: empty shape");
  if (width % 4 || ld_in % 4 || ld_out % 4 || width > 8192) return e.fail("rms_norm: width %d unsupported", width);
  if (!x || !mul || !y) return e.fail("rms_norm: null x / mul / y");
  if (out_dtype != KH_F32 && out_dtype != KH_F16 && out_dtype != KH_BF16) return e.fail("rms_norm: bad out dtype");
  dim3 grid(rows), block(256);
#define KH_RN(OUT, C, A) hipLaunchKernelGGL((rms_norm_kernel<OUT, C, A>), grid, block, 0, st, x, mul, add, y, width, ld_in, ld_out, eps)
#define KH_RN2(OUT)              \
  if (center)                    \
    if (add) KH_RN(OUT, true, true); \
    else KH_RN(OUT, true, false);    \
  else if (add) KH_RN(OUT, false, true); \
  else KH_RN(OUT, false, false);
  if (out_dtype == KH_F32) {
    KH_RN2(KH_F32)
  } else if (out_dtype == KH_F16) {
    KH_RN2(KH_F16)
  } else {
    KH_RN2(KH_BF16)
  }
#undef KH_RN2
#undef KH_RN
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "rms_norm launch");
}

int qk_norm_rope(hipStream_t st, void* qkv, int dtype, const float* wq, const float* wk, const float* cosb,
                 const float* sinb, int rows, int ld, int q_off, int n_q, int k_off, int n_k, float eps, int rope_mode,
                 int big_dim, float* qbig, float* kbig, Err& e) {
  if (dtype != KH_F16 && dtype != KH_BF16) return e.fail("qk_norm_rope: dtype must be f16 or bf16");
  if (rows <= 0 || n_q < 0 || n_k < 0 || n_q + n_k == 0) return e.fail("qk_norm_rope: empty shape");
  if (rope_mode < 0 || rope_mode > 2) return e.fail("qk_norm_rope: bad rope mode %d", rope_mode);
  if (rope_mode != 2 && (!cosb || !sinb)) return e.fail("qk_norm_rope: rope needs cos / sin tables");
  if (!qkv || (n_q && !wq) || (n_k && !wk)) return e.fail("qk_norm_rope: null buffer / weight");
  if (big_dim >= 128 || (big_dim >= 0 && (!qbig || !kbig))) return e.fail("qk_norm_rope: big_dim needs qbig / kbig");
  if (ld % 2 || q_off % 2 || k_off % 2) return e.fail("qk_norm_rope: offsets must be even");
  const long units = (long)rows * (n_q + n_k);
  dim3 grid((unsigned)((units + 3) / 4)), block(256);
  if (dtype == KH_F16)
    hipLaunchKernelGGL(qk_norm_rope_kernel<KH_F16>, grid, block, 0, st, (uint16_t*)qkv, wq, wk, cosb, sinb, rows, ld,
                       q_off, n_q, k_off, n_k, eps, rope_mode, big_dim, qbig, kbig);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<KH_BF16>, grid, block, 0, st, (uint16_t*)qkv, wq, wk, cosb, sinb, rows,
                       ld, q_off, n_q, k_off, n_k, eps, rope_mode, big_dim, qbig, kbig);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "qk_norm_rope launch");
}

int gemv(hipStream_t st, const float* x, const kh_weight& W, float* y, int rows, int N, int K, int ldw, int act,
         const float* bias, Err& e) {
  if (rows <= 0 || rows > 4 || N <= 0 || K <= 0) return e.fail("gemv: rows must be 1..4 and N, K > 0");
  if (N % 4 || ldw % 4 || ldw < N) return e.fail("gemv: N and ldw must be multiples of 4, ldw >= N");
  if (!x || !W.w || !y) return e.fail("gemv: null x / W / y");
  int wf, group = K;
  if (W.w_dtype == KH_I8) {
    if (!W.s) return e.fail("gemv: int8 weights need scales");
    group = W.group <= 0 ? K : W.group;
    if (group > K || K % group) return e.fail("gemv: bad group %d", group);
    wf = group == K ? 1 : 2;
  } else if (W.w_dtype == KH_F16 || W.w_dtype == KH_BF16) {
    wf = 0;
  } else {
    return e.fail("gemv: weight dtype must be int8, f16 or bf16");
  }
  // K split so the grid has >= ~512 workgroups; each slab's x fits the 1024-entry LDS stage
  const int col_blocks = (N + GEMV_COLS - 1) / GEMV_COLS;
  int ksplit = 1;
  while (ksplit < GEMV_KSPLIT_MAX && (col_blocks * ksplit < 512 || (K + ksplit - 1) / ksplit > 1024)) ksplit *= 2;
  int kchunk = (K + ksplit - 1) / ksplit;
  if (kchunk > 1024) return e.fail("gemv: K %d too large", K);
  hipLaunchKernelGGL(gemv_init, dim3((N + 255) / 256), dim3(256), 0, st, y, bias, rows, N, N, (act & 2) ? 1 : 0);
  dim3 grid(col_blocks, (K + kchunk - 1) / kchunk), block(256);
  if (wf == 0)
    hipLaunchKernelGGL(gemv_kernel<0>, grid, block, 0, st, x, W.w, W.s, W.s_dtype, group, W.w_dtype, y, rows, N, K,
                       ldw, N, act & 1, kchunk);
  else if (wf == 1)
    hipLaunchKernelGGL(gemv_kernel<1>, grid, block, 0, st, x, W.w, W.s, W.s_dtype, group, W.w_dtype, y, rows, N, K,
                       ldw, N, act & 1, kchunk);
  else
    hipLaunchKernelGGL(gemv_kernel<2>, grid, block, 0, st, x, W.w, W.s, W.s_dtype, group, W.w_dtype, y, rows, N, K,
                       ldw, N, act & 1, kchunk);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "gemv launch");
}

int make_cond(hipStream_t st, const float* tvec, const float* table, const float* n1, const float* n2, int D,
              float* mods, Err& e) {
  if (D <= 0 || !tvec || !n1 || !n2 || !mods) return e.fail("make_cond: bad arguments");
  hipLaunchKernelGGL(make_cond_kernel, dim3((D + 255) / 256), dim3(256), 0, st, tvec, table, n1, n2, D, mods);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "make_cond launch");
}

int gemm_f32(hipStream_t st, const float* A, const float* W, float* C, int M, int N, int K, int lda, int ldw, int ldc,
             int mode, const float* bias, Err& e) {
  if (M <= 0 || N <= 0 || K <= 0) return e.fail("gemm_f32: empty shape");
  if (!A || !W || !C || ((mode & 1) && !bias)) return e.fail("gemm_f32: null A / W / C (or bias for mode & 1)");
  if (lda < K || ldw < N || ldc < N) return e.fail("gemm_f32: bad strides");
  dim3 grid((N + 63) / 64, (M + 63) / 64), block(256);
  hipLaunchKernelGGL(gemm_f32_kernel, grid, block, 0, st, A, W, C, bias, M, N, K, lda, ldw, ldc, mode);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "gemm_f32 launch");
}

}  // namespace kh
