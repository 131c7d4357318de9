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
          (u32x2){pack16<OUT>(o[0], o[1]),
                  pack16<OUT>(o[2], o[3])};
    }
  }
}

// ------------------------------------------------------------------------------------------------------
// Per-head RMSNorm (weight [128]) + RoPE, in place on a 16-bit fused projection buffer:
// engine/kernels/norm.metal:81-134. 16 lanes per (row, head), 8 consecutive channels (one 16-byte load) per
// lane, 4 heads per wave; the sum of squares is reduced over the 16 lanes. rope_mode 0: interleaved pairs
// (2i, 2i + 1) -- the lane's 4 pairs are local; rope_mode 1: rotate-half (i, i + 64) -- the partner channels
// sit in lane ^ 8; rope_mode 2: no rotation. cos / sin: f32 [rows, 64]. big_dim >= 0: that dimension's
// rotated value goes to qbig [rows, n_q] / kbig [rows, n_k] in f32 and is zeroed in the buffer.
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int DT>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(uint16_t* __restrict__ qkv, const float* __restrict__ wq,
                                                           const float* __restrict__ wk, const float* __restrict__ cosb,
                                                           const float* __restrict__ sinb, int rows, int ld, int q_off,
                                                           int n_q, int k_off, int n_k, float eps, int rope_mode,
                                                           int big_dim, float* __restrict__ qbig,
                                                           float* __restrict__ kbig) {
  const long unit = (long)blockIdx.x * 16 + (threadIdx.x >> 4);  // (row, head) pair
  const int sl = threadIdx.x & 15;                                 // lane within the head: channels 8 sl .. 8 sl + 7
  const int heads = n_q + n_k;
  const int row = (int)(unit / heads), hh = (int)(unit % heads);
  const bool valid = row < rows;
  const int rr = valid ? row : rows - 1;
  const bool is_q = hh < n_q;
  const int col = is_q ? q_off + hh * 128 : k_off + (hh - n_q) * 128;
  uint16_t* base = qkv + (size_t)rr * ld + col + sl * 8;
  const float* w = (is_q ? wq : wk) + sl * 8;
  const u32x4 raw = *(const u32x4*)base;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = from16<DT>((uint16_t)(raw[e >> 1] >> (16 * (e & 1))));
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e++) ss += x[e] * x[e];
  const float rrms = rsqrtf(sum16(ss) * (1.0f / 128.0f) + eps);
  const f32x4 w0 = *(const f32x4*)w, w1 = *(const f32x4*)(w + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    x[e] *= rrms * w0[e];
    x[e + 4] *= rrms * w1[e];
  }
  float o[8];
  if (rope_mode == 0) {  // pairs 4 sl .. 4 sl + 3 at frequencies of the same index
    const f32x4 c = *(const f32x4*)(cosb + (size_t)rr * 64 + sl * 4), s = *(const f32x4*)(sinb + (size_t)rr * 64 + sl * 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      o[2 * i] = x[2 * i] * c[i] - x[2 * i + 1] * s[i];
      o[2 * i + 1] = x[2 * i] * s[i] + x[2 * i + 1] * c[i];
    }
  } else if (rope_mode == 1) {  // channel i pairs with i + 64 (lane ^ 8), frequency i % 64
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = __shfl_xor(x[e], 8);
    const int f = (sl & 7) * 8;
    const f32x4 c0 = *(const f32x4*)(cosb + (size_t)rr * 64 + f), c1 = *(const f32x4*)(cosb + (size_t)rr * 64 + f + 4);
    const f32x4 s0 = *(const f32x4*)(sinb + (size_t)rr * 64 + f), s1 = *(const f32x4*)(sinb + (size_t)rr * 64 + f + 4);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float c = e < 4 ? c0[e] : c1[e - 4], s = e < 4 ? s0[e] : s1[e - 4];
      o[e] = sl < 8 ? x[e] * c - y[e] * s : x[e] * c + y[e] * s;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = x[e];
  }
  if (!valid) return;
  if (big_dim >= 0 && big_dim / 8 == sl) {
    const int e = big_dim % 8;
    float v = o[0];
#pragma unroll
    for (int i = 1; i < 8; i++)
      if (i == e) v = o[i];
    if (is_q) qbig[(size_t)row * n_q + hh] = v;
    else kbig[(size_t)row * n_k + (hh - n_q)] = v;
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (i == e) o[i] = 0.f;
  }
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; i++) out[i] = pack16<DT>(o[2 * i], o[2 * i + 1]);
  *(u32x4*)base = out;
}

// ------------------------------------------------------------------------------------------------------
// adaLN modulation GEMV: y[r, n] (+)= sum_k act(x[r, k]) W~[k, n] (+ bias[n]), rows <= 4, x / y f32.
// engine/kernels/gemm.metal:346-371 (gemv_bf16: act bit 0 = SiLU on load, bit 1 = accumulate) with the
// weight formats of kh_gemm. HBM-bound (each weight byte is read once): grid (N / COLS, KSPLIT); a lane owns
// 16 consecutive bytes of a weight row (16 int8 columns, or 8 16-bit ones), so a wave reads 1 KB per row;
// the 4 waves split the slab's rows, each keeping 8 rows' loads in flight, reduce through LDS and add into y
// with one f32 atomic per column. y is initialised (bias, or 0, or kept for accumulation) by gemv_init.
constexpr int GEMV_KSPLIT_MAX = 64;

__global__ void gemv_init(float* y, const float* bias, int rows, int N, int ldy, int accumulate) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  for (int r = 0; r < rows; r++) {
    const float b = bias ? bias[n] : 0.f;
    float* yp = y + (size_t)r * ldy + n;
    *yp = accumulate ? *yp + b : b;
  }
}

// WF 0: 16-bit weights (8 columns per lane), 1: int8 per-channel, 2: int8 group (16 per lane); RMAX: rows the
// instantiation handles (1: the DiT's single conditioning vector, 4: up to four; sizes the accumulators and the
// partial-sum LDS, so the one-row form fits four times as many workgroups per CU)
template <int WF, int RMAX>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, const void* __restrict__ W,
                                                   const void* __restrict__ S, int s_dtype, int group, int w16_dtype,
                                                   float* __restrict__ y, int rows, int N, int K, int ldw, int ldy,
                                                   int silu, int kchunk) {
  constexpr int CPL = WF == 0 ? 8 : 16;  // columns per lane
  constexpr int COLS = 16 * CPL;         // 16 lanes span the block's columns; lane >> 4 picks a row group
  __shared__ float xs[RMAX][512];        // activated x of this slab (rows x kchunk), kchunk <= 512
  __shared__ float part[16][RMAX][COLS]; // [row group][row][column]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = wave * 4 + (lane >> 4);  // 16 row groups
  const int n = blockIdx.x * COLS + (lane & 15) * CPL;
  const int k0 = blockIdx.y * kchunk, k1 = min(K, k0 + kchunk);
  for (int i = tid; i < rows * (k1 - k0); i += 256) {
    const int r = i / (k1 - k0), k = i % (k1 - k0);
    const float v = x[(size_t)r * K + k0 + k];
    xs[r][k] = silu ? silu_f(v) : v;
  }
  __syncthreads();
  float acc[RMAX][CPL];
#pragma unroll
  for (int r = 0; r < RMAX; r++)
#pragma unroll
    for (int c = 0; c < CPL; c++) acc[r][c] = 0.f;
  if (n < N) {
    const char* wp = (const char*)W + ((size_t)n) * (WF == 0 ? 2 : 1);
    const size_t row_bytes = (size_t)ldw * (WF == 0 ? 2 : 1);
    for (int kb = k0 + rg; kb < k1; kb += 16 * 8) {
      u32x4 raw[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int k = kb + 16 * u;
        raw[u] = k < k1 ? *(const u32x4*)(wp + (size_t)k * row_bytes) : (u32x4){0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int k = kb + 16 * u;
        if (k >= k1) break;
        float wv[CPL];
        if (WF == 0) {
#pragma unroll
          for (int c = 0; c < 8; c++) {
            const uint16_t hb = (uint16_t)(raw[u][c >> 1] >> (16 * (c & 1)));
            wv[c] = w16_dtype == KH_BF16 ? from16<KH_BF16>(hb) : from16<KH_F16>(hb);
          }
        } else {
#pragma unroll
          for (int c = 0; c < 16; c++) wv[c] = (float)(int8_t)(raw[u][c >> 2] >> (8 * (c & 3)));
          if (WF == 2) {
            const size_t g = (size_t)(k / group) * ldw + n;
#pragma unroll
            for (int c = 0; c < 16; c++) wv[c] *= load_scale(S, s_dtype, g + c);
          }
        }
#pragma unroll
        for (int r = 0; r < RMAX; r++) {  // static indices keep acc in registers
          if (r >= rows) break;
          const float xv = xs[r][k - k0];
#pragma unroll
          for (int c = 0; c < CPL; c++) acc[r][c] += xv * wv[c];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RMAX; r++) {
    if (r >= rows) break;
#pragma unroll
    for (int c = 0; c < CPL; c++) part[rg][r][(lane & 15) * CPL + c] = acc[r][c];
  }
  __syncthreads();
  for (int i = tid; i < rows * COLS; i += 256) {
    const int r = i / COLS, c = i % COLS;
    const int nc = blockIdx.x * COLS + c;
    if (nc >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int g = 0; g < 16; g++) v += part[g][r][c];
    if (WF == 1) v *= load_scale(S, s_dtype, nc);
    atomicAdd(y + (size_t)r * ldy + nc, v);
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
// Split-K form (gridDim.z > 1, no GELU): each z-slice adds its partial product into C with f32 atomics after
// gemm_f32_init has set C to bias / 0 (or kept it, for accumulate).
__global__ void gemm_f32_init(float* C, const float* bias, int M, int N, int ldc, int mode) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
  if (n >= N) return;
  float* cp = C + (size_t)m * ldc + n;
  const float b = (mode & 1) ? bias[n] : 0.f;
  *cp = (mode & 4) ? *cp + b : b;
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ W,
                                                       float* __restrict__ C, const float* __restrict__ bias, int M,
                                                       int N, int K, int lda, int ldw, int ldc, int mode) {
  const int kz = gridDim.z > 1 ? (K + gridDim.z - 1) / gridDim.z : K;
  const int kbeg = blockIdx.z * kz, kfin = min(K, kbeg + kz);
  __shared__ float As[16][64 + 1];
  __shared__ float Ws[16][64];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = kbeg; k0 < kfin; k0 += 16) {
    for (int i = tid; i < 16 * 64; i += 256) {
      const int r = i / 16, c = i % 16;  // A tile: 64 rows x 16 k
      const int m = m0 + r, k = k0 + c;
      As[c][r] = (m < M && k < kfin) ? A[(size_t)m * lda + k] : 0.f;
      const int kr = i / 64, nc = i % 64;  // W tile: 16 k x 64 cols
      Ws[kr][nc] = (k0 + kr < kfin && n0 + nc < N) ? W[(size_t)(k0 + kr) * ldw + n0 + nc] : 0.f;
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
      float* cp = C + (size_t)m * ldc + n;
      if (gridDim.z > 1) {
        atomicAdd(cp, v);
        continue;
      }
      if (mode & 1) v += bias[n];
      if (mode & 2) v = gelu_tanh_f(v);
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
  if (ld % 8 || q_off % 8 || k_off % 8 || ((uintptr_t)qkv & 15))
    return e.fail("qk_norm_rope: rows and head offsets must be 16-byte aligned");
  const long units = (long)rows * (n_q + n_k);
  dim3 grid((unsigned)((units + 15) / 16)), block(256);
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
  if (ldw < N) return e.fail("gemv: ldw %d < N %d", ldw, N);
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
    return e.fail(W.w_dtype == KH_I8P ? "gemv: packed int8 weights (KH_I8P) are for kh_gemm; pass the KH_I8 layout"
                                      : "gemv: weight dtype must be int8, f16 or bf16");
  }
  // K split so the grid has >= wg_target workgroups; each slab's x fits the 512-entry LDS stage
  const int cols = wf == 0 ? 128 : 256;
  if (N % (wf == 0 ? 8 : 16) || ldw % 16) return e.fail("gemv: N must be a multiple of 16 (8 for 16-bit), ldw of 16");
  const int col_blocks = (N + cols - 1) / cols;
  int ksplit = 1;
  // one-row calls fit six workgroups per CU: more K splits keep more loads in flight (measured at 3072 ->
  // 18432 int8: 512 workgroups 15.1 us, 1024 13.8 us, 2048 14.5 us)
  const int wg_target = rows == 1 ? 1024 : 512;
  while (ksplit < GEMV_KSPLIT_MAX && (col_blocks * ksplit < wg_target || (K + ksplit - 1) / ksplit > 512)) ksplit *= 2;
  const int kchunk = (K + ksplit - 1) / ksplit;
  if (kchunk > 512) return e.fail("gemv: K %d too large", K);
  hipLaunchKernelGGL(gemv_init, dim3((N + 255) / 256), dim3(256), 0, st, y, bias, rows, N, N, (act & 2) ? 1 : 0);
  dim3 grid(col_blocks, (K + kchunk - 1) / kchunk), block(256);
#define KH_GEMV(WF_, R_)                                                                                      \
  hipLaunchKernelGGL((gemv_kernel<WF_, R_>), grid, block, 0, st, x, W.w, W.s, W.s_dtype, group, W.w_dtype, y, rows, \
                     N, K, ldw, N, act & 1, kchunk)
  if (rows == 1) {
    if (wf == 0) KH_GEMV(0, 1);
    else if (wf == 1) KH_GEMV(1, 1);
    else KH_GEMV(2, 1);
  } else {
    if (wf == 0) KH_GEMV(0, 4);
    else if (wf == 1) KH_GEMV(1, 4);
    else KH_GEMV(2, 4);
  }
#undef KH_GEMV
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "gemv launch");
}

// ---- sampler updates over f32 [n]: 4 elements per thread (16-byte accesses when both arrays allow) ----
// MODE 0: z += dt v (euler_step); MODE 1: vc += s (vc - vn) (cfg_combine)
template <int MODE, bool VEC>
__global__ __launch_bounds__(256) void latent_update_kernel(float* __restrict__ y, const float* __restrict__ x,
                                                           long long n, float c) {
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 4;
  auto f = [&](float a, float b) { return MODE == 0 ? fmaf(c, b, a) : fmaf(c, a - b, a); };
  if (VEC && i + 3 < n) {
    f32x4 a = *(const f32x4*)(y + i);
    const f32x4 b = *(const f32x4*)(x + i);
#pragma unroll
    for (int e = 0; e < 4; e++) a[e] = f(a[e], b[e]);
    *(f32x4*)(y + i) = a;
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (i + e < n) y[i + e] = f(y[i + e], x[i + e]);
  }
}

template <int MODE>
static int latent_update(hipStream_t st, float* y, const float* x, long long n, float c, const char* what, Err& e) {
  if (!y || !x) return e.fail("%s: null pointer", what);
  if (n <= 0) return e.fail("%s: n=%lld must be positive", what, n);
  const unsigned blocks = (unsigned)((n + 1023) / 1024);
  if ((((uintptr_t)y | (uintptr_t)x) & 15) == 0)
    hipLaunchKernelGGL((latent_update_kernel<MODE, true>), dim3(blocks), dim3(256), 0, st, y, x, n, c);
  else
    hipLaunchKernelGGL((latent_update_kernel<MODE, false>), dim3(blocks), dim3(256), 0, st, y, x, n, c);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, what);
}

int euler_step(hipStream_t st, float* z, const float* v, long long n, float dt, Err& e) {
  return latent_update<0>(st, z, v, n, dt, "euler_step", e);
}

int cfg_combine(hipStream_t st, float* vc, const float* vn, long long n, float scale, Err& e) {
  return latent_update<1>(st, vc, vn, n, scale, "cfg_combine", e);
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
  // small grids with long K (the D -> 64 head) split K over workgroups; GELU needs the full sum
  int ksplit = 1;
  while (!(mode & 2) && grid.x * grid.y * ksplit < 512 && K / (ksplit * 2) >= 128) ksplit *= 2;
  grid.z = ksplit;
  if (ksplit > 1)
    hipLaunchKernelGGL(gemm_f32_init, dim3((N + 255) / 256, M), dim3(256), 0, st, C, bias, M, N, ldc, mode);
  hipLaunchKernelGGL(gemm_f32_kernel, grid, block, 0, st, A, W, C, bias, M, N, K, lda, ldw, ldc, mode);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "gemm_f32 launch");
}

}  // namespace kh
