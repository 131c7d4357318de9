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
// adaLN / conditioning GEMV: y[r, n] = (y[r, n] if accumulate) + bias[n] + sum_k act(x[r, k]) W~[k, n],
// rows <= 4, x / y f32. engine/kernels/gemm.metal:346-371 (gemv_bf16: act bit 0 = SiLU on load, bit 1 =
// accumulate) and the f32 cblas_sgemv linears of Conditioning::compute (engine/src/model.mm:582-590: the GELU
// between them is applied on load, act bit 2), with the weight formats of kh_gemm plus f32.
// HBM-bound, every weight byte is read once. A workgroup owns a 32-byte column slab of every weight row (32
// int8 / 16 16-bit / 8 f32 columns) over all of K: two lanes of 16 bytes per row, 128 k-groups of contiguous
// rows, 8 rows' loads in flight per lane. The k-groups' partial sums are added through LDS in a fixed order
// (no atomics, no second launch): the same inputs give the same bits on every run. The four slabs of one
// 128-byte line go to workgroups on the same XCD (the dispatcher deals workgroups round-robin to the 8 XCDs,
// each with its own L2), so a line is fetched from HBM once.
constexpr int GEMV_KG = 128;  // k-groups per workgroup (two lanes each)

template <int ACT>
__device__ __forceinline__ float gemv_act(float v) {
  if (ACT == 1) return silu_f(v);
  if (ACT == 4) return gelu_tanh_f(v);
  return v;
}

// WF 0: 16-bit weights, 1: int8 per-channel scales, 2: int8 group scales, 3: f32. RMAX: rows the instantiation
// handles (sizes the accumulators and the LDS; the one-row form fits four times as many workgroups per CU).
template <int WF, int RMAX, int ACT>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, const void* __restrict__ W,
                                                   const void* __restrict__ S, int s_dtype, int group, int w16_dtype,
                                                   const float* __restrict__ bias, float* __restrict__ y, int rows,
                                                   int N, int K, int ldw, int accumulate) {
  constexpr int ES = WF == 3 ? 4 : WF == 0 ? 2 : 1;  // bytes per weight
  constexpr int CPL = 16 / ES;                        // columns per lane
  constexpr int COLS = 2 * CPL;                       // columns per workgroup
  constexpr int OUT = RMAX * COLS;                    // partial sums per k-group
  constexpr int TPO = 256 / OUT;                      // threads per output in the final reduction
  __shared__ float part[GEMV_KG][OUT + 1];
  // gfx950 gives a workgroup up to 160 KiB of LDS; the int8 four-row form uses 128 x 129 x 4 = 66,048 bytes
  // (two workgroups per CU), above the 64 KiB of earlier CDNA parts, so this kernel is gfx950-only as sized
  static_assert(sizeof(part) <= 160 * 1024, "gemv_kernel: partial sums exceed the 160 KiB LDS of a gfx950 CU");
  static_assert(256 % OUT == 0 && GEMV_KG % (256 / OUT) == 0, "gemv_kernel: outputs must split the workgroup");
  const int tid = threadIdx.x, li = tid & 1, kg = tid >> 1;
  const int nblk = gridDim.x;
  const int b = nblk % 8 == 0 ? (int)(blockIdx.x & 7) * (nblk >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int n0 = b * COLS, n = n0 + li * CPL;
  const int kr = (K + GEMV_KG - 1) / GEMV_KG;
  const int k0 = min(K, kg * kr), k1 = min(K, k0 + kr);
  float acc[RMAX][CPL];
#pragma unroll
  for (int r = 0; r < RMAX; r++)
#pragma unroll
    for (int c = 0; c < CPL; c++) acc[r][c] = 0.f;
  if (n < N) {
    const char* wp = (const char*)W + (size_t)n * ES;
    const size_t rb = (size_t)ldw * ES;
    int gcur = -1;
    float sc[CPL];
    for (int kb = k0; kb < k1; kb += 8) {
      u32x4 raw[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int k = kb + u;
        raw[u] = k < k1 ? *(const u32x4*)(wp + (size_t)k * rb) : (u32x4){0u, 0u, 0u, 0u};
      }
      float xa[RMAX][8];  // activated inputs of these 8 rows (loaded while the weights are in flight)
#pragma unroll
      for (int r = 0; r < RMAX; r++)
#pragma unroll
        for (int u = 0; u < 8; u++) xa[r][u] = (r < rows && kb + u < k1) ? x[(size_t)r * K + kb + u] : 0.f;
#pragma unroll
      for (int r = 0; r < RMAX; r++)
#pragma unroll
        for (int u = 0; u < 8; u++) xa[r][u] = gemv_act<ACT>(xa[r][u]);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int k = kb + u;
        if (k >= k1) break;
        float wv[CPL];
        if constexpr (WF == 3) {
          const f32x4 fv = __builtin_bit_cast(f32x4, raw[u]);
#pragma unroll
          for (int c = 0; c < 4; c++) wv[c] = fv[c];
        } else if constexpr (WF == 0) {
#pragma unroll
          for (int c = 0; c < 8; c++) {
            const uint16_t hb = (uint16_t)(raw[u][c >> 1] >> (16 * (c & 1)));
            wv[c] = w16_dtype == KH_BF16 ? from16<KH_BF16>(hb) : from16<KH_F16>(hb);
          }
        } else {
#pragma unroll
          for (int c = 0; c < 16; c++) wv[c] = (float)(int8_t)(raw[u][c >> 2] >> (8 * (c & 3)));
          if (WF == 2) {
            const int g = k / group;
            if (g != gcur) {
              gcur = g;
#pragma unroll
              for (int c = 0; c < 16; c++) sc[c] = load_scale(S, s_dtype, (size_t)g * ldw + n + c);
            }
#pragma unroll
            for (int c = 0; c < 16; c++) wv[c] *= sc[c];
          }
        }
#pragma unroll
        for (int r = 0; r < RMAX; r++) {  // static indices keep acc in registers
          if (r >= rows) break;
          const float xv = xa[r][u];
#pragma unroll
          for (int c = 0; c < CPL; c++) acc[r][c] += xv * wv[c];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RMAX; r++)
#pragma unroll
    for (int c = 0; c < CPL; c++) part[kg][r * COLS + li * CPL + c] = acc[r][c];
  __syncthreads();
  // output o = (row, column) summed by TPO adjacent lanes, each over GEMV_KG / TPO k-groups in order, then a
  // fixed butterfly over those lanes
  const int o = tid / TPO, j = tid % TPO;
  float v = 0.f;
#pragma unroll 4
  for (int i = 0; i < GEMV_KG / TPO; i++) v += part[j * (GEMV_KG / TPO) + i][o];
#pragma unroll
  for (int m = TPO / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  const int r = o / COLS, nc = n0 + o % COLS;
  if (j == 0 && r < rows && nc < N) {
    if (WF == 1) v *= load_scale(S, s_dtype, nc);
    const float bv = bias ? bias[nc] : 0.f;
    float* yp = y + (size_t)r * N + nc;
    *yp = (accumulate ? *yp + bv : bv) + v;
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

// Final-norm vectors of the head from the step's t: engine/src/model.mm:340-346 (the fin half of
// DiT::make_cond): fin[k] = nf[k] (1 + t[k] + lin[k]), fin[D + k] = t[k] + lin[D + k].
__global__ void make_fin_kernel(const float* t, const float* lin, const float* nf, int D, float* fin) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= D) return;
  fin[k] = nf[k] * (1.0f + t[k] + lin[k]);
  fin[D + k] = t[k] + lin[D + k];
}

// A host-computed vector of up to 256 floats passed by value (the timestep embedding of Conditioning::compute)
struct Vec256 {
  float v[256];
};
__global__ void store_vec_kernel(Vec256 src, int n, float* dst) {
  const int i = threadIdx.x;
  if (i < n) dst[i] = src.v[i];
}

// ------------------------------------------------------------------------------------------------------
// fp32 GEMM of the patch embed (64 -> D) and the final projection (D -> 64): engine/kernels/f32gemm.metal
// (gemm_f32w) with its modes bit 0 bias, bit 1 GELU(tanh), bit 2 accumulate. Tiles of 16 TM rows x 64 columns,
// 256 threads, TM x 4 outputs per thread, K staged 16 at a time through LDS, each output summed over all of K
// in order by one thread (no split-K atomics: the results repeat bit for bit). TM = 4 (64-row tiles) unless
// that leaves CUs idle (the D -> 64 head: 64 tiles at 4096 rows), then TM = 1. Tiny next to the DiT layers.
template <int TM>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ W,
                                                       float* __restrict__ C, const float* __restrict__ bias, int M,
                                                       int N, int K, int lda, int ldw, int ldc, int mode) {
  constexpr int BMR = 16 * TM;
  __shared__ float As[16][BMR + 1];
  __shared__ float Ws[16][64];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * BMR, n0 = blockIdx.x * 64;
  float acc[TM][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = tid; i < 16 * BMR; i += 256) {
      const int r = i / 16, c = i % 16;  // A tile: BMR rows x 16 k
      const int m = m0 + r, k = k0 + c;
      As[c][r] = (m < M && k < K) ? A[(size_t)m * lda + k] : 0.f;
    }
    for (int i = tid; i < 16 * 64; i += 256) {
      const int kr = i / 64, nc = i % 64;  // W tile: 16 k x 64 cols
      Ws[kr][nc] = (k0 + kr < K && n0 + nc < N) ? W[(size_t)(k0 + kr) * ldw + n0 + nc] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) {
      float a[TM], b[4];
#pragma unroll
      for (int i = 0; i < TM; i++) a[i] = As[k][ty * TM + i];
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = Ws[k][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int m = m0 + ty * TM + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + tx * 4 + j;
      if (n >= N) continue;
      float v = acc[i][j];
      float* cp = C + (size_t)m * ldc + n;
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
  if (act & ~7) return e.fail("gemv: unknown act bits 0x%x", act);
  if ((act & 1) && (act & 4)) return e.fail("gemv: SiLU and GELU on load are exclusive");
  int wf, group = K;
  if (W.w_dtype == KH_I8) {
    if (!W.s) return e.fail("gemv: int8 weights need scales");
    if (W.s_dtype != KH_F32 && W.s_dtype != KH_F16 && W.s_dtype != KH_BF16) return e.fail("gemv: bad scale dtype");
    group = W.group <= 0 ? K : W.group;
    if (group > K || K % group) return e.fail("gemv: bad group %d", group);
    wf = group == K ? 1 : 2;
  } else if (W.w_dtype == KH_F16 || W.w_dtype == KH_BF16) {
    wf = 0;
  } else if (W.w_dtype == KH_F32) {
    wf = 3;
  } else {
    return e.fail(W.w_dtype == KH_I8P ? "gemv: packed int8 weights (KH_I8P) are for kh_gemm; pass the KH_I8 layout"
                                      : "gemv: weight dtype must be int8, f16, bf16 or f32");
  }
  const int es = wf == 3 ? 4 : wf == 0 ? 2 : 1, cpl = 16 / es;
  if (N % cpl || ((size_t)ldw * es) % 16)
    return e.fail("gemv: N must be a multiple of %d and weight rows 16-byte aligned for this weight type", cpl);
  if (((uintptr_t)W.w & 15)) return e.fail("gemv: W must be 16-byte aligned");
  dim3 grid((unsigned)((N + 2 * cpl - 1) / (2 * cpl))), block(256);
  const int accumulate = (act & 2) ? 1 : 0;
  const int a = act & 5;
#define KH_GEMV(WF_, R_, A_)                                                                                   \
  hipLaunchKernelGGL((gemv_kernel<WF_, R_, A_>), grid, block, 0, st, x, W.w, W.s, W.s_dtype, group, W.w_dtype, \
                     bias, y, rows, N, K, ldw, accumulate)
#define KH_GEMV_A(WF_, R_) \
  do {                     \
    if (a == 1)            \
      KH_GEMV(WF_, R_, 1); \
    else if (a == 4)       \
      KH_GEMV(WF_, R_, 4); \
    else                   \
      KH_GEMV(WF_, R_, 0); \
  } while (0)
#define KH_GEMV_W(R_)     \
  do {                    \
    if (wf == 0)          \
      KH_GEMV_A(0, R_);   \
    else if (wf == 1)     \
      KH_GEMV_A(1, R_);   \
    else if (wf == 2)     \
      KH_GEMV_A(2, R_);   \
    else                  \
      KH_GEMV_A(3, R_);   \
  } while (0)
  if (rows == 1)
    KH_GEMV_W(1);
  else
    KH_GEMV_W(4);
#undef KH_GEMV_W
#undef KH_GEMV_A
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
  const unsigned gx = (unsigned)((N + 63) / 64);
  if ((size_t)gx * ((M + 63) / 64) >= 256)
    hipLaunchKernelGGL(gemm_f32_kernel<4>, dim3(gx, (M + 63) / 64), dim3(256), 0, st, A, W, C, bias, M, N, K, lda, ldw,
                       ldc, mode);
  else
    hipLaunchKernelGGL(gemm_f32_kernel<1>, dim3(gx, (M + 15) / 16), dim3(256), 0, st, A, W, C, bias, M, N, K, lda, ldw,
                       ldc, mode);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "gemm_f32 launch");
}

int make_fin(hipStream_t st, const float* t, const float* lin, const float* nf, int D, float* fin, Err& e) {
  if (D <= 0 || !t || !lin || !nf || !fin) return e.fail("make_fin: null vector or D <= 0");
  hipLaunchKernelGGL(make_fin_kernel, dim3((D + 255) / 256), dim3(256), 0, st, t, lin, nf, D, fin);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "make_fin launch");
}

int store_vec(hipStream_t st, const float* host, int n, float* dst, Err& e) {
  if (n <= 0 || n > 256 || !host || !dst) return e.fail("store_vec: 1..256 values");
  Vec256 v{};
  for (int i = 0; i < n; i++) v.v[i] = host[i];
  hipLaunchKernelGGL(store_vec_kernel, dim3(1), dim3(256), 0, st, v, n, dst);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "store_vec launch");
}

}  // namespace kh
