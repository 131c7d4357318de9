// VAE decoder ops for MI355X (gfx950): the Qwen-Image (Wan 2.1) decoder of the Krea 2 engine, single frame.
//
// Semantics: engine/kernels/vae.metal (vae_unpack_pq 690-712, vconv 5-128 / 162-346, vae_norm_silu 588-668,
// vae_transpose 714-725, softmax_rows 727-757, vae_conv_out_rgba 759-785) as driven by engine/src/vae.mm.
// Activations are NHWC bf16 rows [pixel, channel] with a row stride; weights are the converter's
// implicit-GEMM layout Wt[(ky * 3 + kx) * Cin + ci, co] (tools/convert.py:338-344).
//
// Design: every convolution with a real channel count runs on the GEMM core (16-bit weights, bias
// epilogue): 3 x 3 convs (optionally nearest-2x-upsampled) as an implicit GEMM whose activation DMA
// gathers each (tap, channel) chunk straight from the image (conv3x3 in kh_gemm.hip), 1 x 1 convs as a
// plain GEMM. These kernels are the memory-bound steps around it: the channel RMS norm, the residual add,
// the latent unpack, the mid-block attention's K transpose and row softmax, the 4-channel output conv, and
// an explicit im2col (kept as an exported op: the reference the implicit loader is tested against).
#include "kh_common.h"
#include "kh_internal.h"

namespace kh {

namespace {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

// ---- unpack + de-normalize + post_quant_conv: z f32 [H16 * W16, 64] (features c * 4 + py * 2 + px) ->
//      y bf16 [(2 H16) * (2 W16), 16]; u = z * std + mean, y = W u + b (W f32 [in][out]) ----
__global__ __launch_bounds__(256) void vae_unpack_kernel(const float* __restrict__ z, const float* __restrict__ mean,
                                                        const float* __restrict__ stdv, const float* __restrict__ w,
                                                        const float* __restrict__ b, uint16_t* __restrict__ y, int H16,
                                                        int W16) {
  const int P = 4 * H16 * W16, pix = blockIdx.x * 256 + threadIdx.x;
  if (pix >= P) return;
  const int W2 = 2 * W16, yy = pix / W2, xx = pix % W2;
  const float* zt = z + (size_t)((yy >> 1) * W16 + (xx >> 1)) * 64 + (yy & 1) * 2 + (xx & 1);
  float u[16];
#pragma unroll
  for (int c = 0; c < 16; c++) u[c] = zt[c * 4] * stdv[c] + mean[c];
  uint32_t o[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float a0 = b[2 * k], a1 = b[2 * k + 1];
#pragma unroll
    for (int c = 0; c < 16; c++) {
      a0 += w[c * 16 + 2 * k] * u[c];
      a1 += w[c * 16 + 2 * k + 1] * u[c];
    }
    o[k] = pack16<KH_BF16>(a0, a1);
  }
  u32x4v* yo = (u32x4v*)(y + (size_t)pix * 16);
  yo[0] = (u32x4v){o[0], o[1], o[2], o[3]};
  yo[1] = (u32x4v){o[4], o[5], o[6], o[7]};
}

// ---- im2col of a 3 x 3 conv with zero padding 1, output H x W pixels [m0, m0 + rows), K order
//      (tap, channel), columns [9 C, Kpad) zero. up: the input is H / 2 x W / 2 and nearest-upsampled. One
//      thread per 8 columns (16 bytes) of one pixel. ----
__global__ __launch_bounds__(256) void vae_im2col_kernel(const uint16_t* __restrict__ x, int ldx, int C, int H, int W,
                                                        int up, int m0, int rows, uint16_t* __restrict__ col,
                                                        int Kpad) {
  const int cpr = Kpad / 8;  // 16-byte chunks per panel row
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)rows * cpr) return;
  const int r = (int)(idx / cpr), c8 = (int)(idx % cpr);
  const int k = c8 * 8;
  u32x4v v = {0u, 0u, 0u, 0u};
  if (k < 9 * C) {
    const int tap = k / C, ci = k - tap * C;  // C % 8 == 0: a chunk never straddles two taps
    const int p = m0 + r, py = p / W, px = p % W;
    int sy = py + tap / 3 - 1, sx = px + tap % 3 - 1;
    if (sy >= 0 && sy < H && sx >= 0 && sx < W) {
      const int Win = up ? W / 2 : W;
      if (up) {
        sy >>= 1;
        sx >>= 1;
      }
      v = *(const u32x4v*)(x + ((size_t)sy * Win + sx) * ldx + ci);
    }
  }
  *(u32x4v*)(col + (size_t)r * Kpad + k) = v;
}

// ---- channel RMS norm: y = x * sqrt(C) / max(||x||, 1e-12) * gamma (F.normalize over C, the Wan RMS_norm),
//      optional SiLU; 16 lanes per pixel, 16-byte chunks ----
__global__ __launch_bounds__(256) void vae_norm_silu_kernel(const uint16_t* __restrict__ x, int ldx,
                                                           const float* __restrict__ gamma,
                                                           uint16_t* __restrict__ y, int ldy, int P, int C, int silu) {
  const int q = threadIdx.x & 15;
  const int pix0 = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool valid = pix0 < P;
  const int pix = valid ? pix0 : P - 1;
  const uint16_t* xr = x + (size_t)pix * ldx;
  const int chunks = C / 8;
  float ss = 0.f;
  for (int c = q; c < chunks; c += 16) {
    const u32x4v v = *(const u32x4v*)(xr + c * 8);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float a = bf((uint16_t)v[k]), b = bf((uint16_t)(v[k] >> 16));
      ss += a * a + b * b;
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
  const float scale = sqrtf((float)C) / fmaxf(sqrtf(ss), 1e-12f);
  if (!valid) return;
  uint16_t* yr = y + (size_t)pix * ldy;
  for (int c = q; c < chunks; c += 16) {
    const u32x4v v = *(const u32x4v*)(xr + c * 8);
    u32x4v o;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float a = bf((uint16_t)v[k]) * scale * gamma[c * 8 + 2 * k];
      float b = bf((uint16_t)(v[k] >> 16)) * scale * gamma[c * 8 + 2 * k + 1];
      if (silu) {
        a = silu_f(a);
        b = silu_f(b);
      }
      o[k] = pack16<KH_BF16>(a, b);
    }
    *(u32x4v*)(yr + c * 8) = o;
  }
}

// Register variant for C = 24 L channels with L in {4, 8, 16} (the decoder's 96, 192 and 384): L lanes per
// pixel, 3 chunks of 8 channels per lane (lane q holds chunks q, q + L, q + 2L: consecutive lanes read
// consecutive 16 bytes), so x is read once and every lane is busy; same arithmetic as above.
template <int L>
__global__ __launch_bounds__(256) void vae_norm_silu_reg_kernel(const uint16_t* __restrict__ x, int ldx,
                                                               const float* __restrict__ gamma,
                                                               uint16_t* __restrict__ y, int ldy, int P, int silu) {
  constexpr int CPL = 3, C = 8 * CPL * L;
  const int q = threadIdx.x % L;
  const int pix0 = blockIdx.x * (256 / L) + threadIdx.x / L;
  const bool valid = pix0 < P;
  const int pix = valid ? pix0 : P - 1;
  const uint16_t* xr = x + (size_t)pix * ldx;
  u32x4v v[CPL];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    v[j] = *(const u32x4v*)(xr + (q + L * j) * 8);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float a = bf((uint16_t)v[j][k]), b = bf((uint16_t)(v[j][k] >> 16));
      ss += a * a + b * b;
    }
  }
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, L);
  const float scale = sqrtf((float)C) / fmaxf(sqrtf(ss), 1e-12f);
  if (!valid) return;
  uint16_t* yr = y + (size_t)pix * ldy;
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    const int c = q + L * j;
    const f32x4 g0 = *(const f32x4*)(gamma + c * 8), g1 = *(const f32x4*)(gamma + c * 8 + 4);
    const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
    u32x4v o;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float a = bf((uint16_t)v[j][k]) * scale * g[2 * k];
      float b = bf((uint16_t)(v[j][k] >> 16)) * scale * g[2 * k + 1];
      if (silu) {
        a = silu_f(a);
        b = silu_f(b);
      }
      o[k] = pack16<KH_BF16>(a, b);
    }
    *(u32x4v*)(yr + c * 8) = o;
  }
}

// ---- y[i] += a[i] (bf16, n elements, n % 8 == 0): the residual of the resblocks / attention ----
__global__ __launch_bounds__(256) void vae_add_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ a,
                                                     long long n8) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  u32x4v v = ((const u32x4v*)y)[i];
  const u32x4v w = ((const u32x4v*)a)[i];
#pragma unroll
  for (int k = 0; k < 4; k++)
    v[k] = pack16<KH_BF16>(bf((uint16_t)v[k]) + bf((uint16_t)w[k]), bf((uint16_t)(v[k] >> 16)) + bf((uint16_t)(w[k] >> 16)));
  ((u32x4v*)y)[i] = v;
}

// ---- out[c, p] = in[p, off + c] for p < P, c < C (the attention's K^T), 64 x 64 tiles through LDS ----
__global__ __launch_bounds__(256) void vae_transpose_kernel(const uint16_t* __restrict__ in, int ld, int off, int P,
                                                           int C, uint16_t* __restrict__ out, int ldo) {
  __shared__ uint16_t t[64][66];
  const int p0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int pr = i / 64, cc = i % 64;
    const int p = p0 + pr, c = c0 + cc;
    t[pr][cc] = (p < P && c < C) ? in[(size_t)p * ld + off + c] : (uint16_t)0;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int cr = i / 64, pp = i % 64;
    const int p = p0 + pp, c = c0 + cr;
    if (p < P && c < C) out[(size_t)c * ldo + p] = t[pp][cr];
  }
}

// ---- row softmax: P[r, :n] = bf16(softmax(S[r, :n] * scale)), one workgroup of 256 per row ----
__global__ __launch_bounds__(256) void vae_softmax_kernel(const float* __restrict__ S, int ld, int n, float scale,
                                                         uint16_t* __restrict__ Pm) {
  __shared__ float red[4];
  const float* s = S + (size_t)blockIdx.x * ld;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float mx = -INFINITY;
  for (int i = tid; i < n; i += 256) mx = fmaxf(mx, s[i] * scale);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int i = tid; i < n; i += 256) sum += __expf(s[i] * scale - mx);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  const float inv = 1.0f / (red[0] + red[1] + red[2] + red[3]);
  uint16_t* o = Pm + (size_t)blockIdx.x * ld;
  for (int i = tid; i < n; i += 256) o[i] = to16<KH_BF16>(__expf(s[i] * scale - mx) * inv);
}

// One-read variant for rows of up to 1024 NV values (the mid block's 16384 keys at 1024^2: NV = 16): each
// thread keeps its 4 NV values (float4 loads, 16 KB apart across the workgroup) in registers through the max,
// sum and store phases, so S is read once instead of three times. Needs ld % 4 == 0 and 16-byte aligned S,
// 8-byte aligned Pm.
template <int NV>
__global__ __launch_bounds__(256) void vae_softmax_rows_kernel(const float* __restrict__ S, int ld, int n, float scale,
                                                              uint16_t* __restrict__ Pm) {
  __shared__ float red[2][4];
  const float* s = S + (size_t)blockIdx.x * ld;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  f32x4 v[NV];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = 4 * (tid + 256 * j);
    if (i + 3 < n) {
      v[j] = *(const f32x4*)(s + i);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) v[j][e] = i + e < n ? s[i + e] : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[j][e] *= scale;
      mx = fmaxf(mx, v[j][e]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) red[0][wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[j][e] = __expf(v[j][e] - mx);  // padding: exp(-inf) = 0
      sum += v[j][e];
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  if (lane == 0) red[1][wave] = sum;
  __syncthreads();
  const float inv = 1.0f / (red[1][0] + red[1][1] + red[1][2] + red[1][3]);
  uint16_t* o = Pm + (size_t)blockIdx.x * ld;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = 4 * (tid + 256 * j);
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) h[e] = to16<KH_BF16>(v[j][e] * inv);
    if (i + 3 < n) {
      *(uint2*)(o + i) = make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (i + e < n) o[i + e] = h[e];
    }
  }
}

// ---- final 3 x 3 conv C -> 4 (RGBA; alpha's weights are zero and its bias 1) + clamp(-1, 1) + [0, 255]
//      quantization. A workgroup owns a 16 x 16 pixel tile, one pixel per thread. Per chunk of 32
//      channels it stages the 18 x 18 halo (zero outside the image) and the chunk's weights (f32
//      [tap][channel][4]) in LDS with coalesced loads, then every thread reads its 9 taps from LDS. The halo's
//      pixel stride is 40 channels (80 B): the 16 lanes of one 16-byte LDS read cycle then start on 16
//      distinct 4-bank groups. ----
constexpr int CO_T = 16, CO_HALO = CO_T + 2, CO_CC = 32, CO_PS = 40;
__global__ __launch_bounds__(256) void vae_conv_out_kernel(const uint16_t* __restrict__ x, int ldx, int C,
                                                          const uint16_t* __restrict__ w, const float* __restrict__ bias,
                                                          uint8_t* __restrict__ rgba, int H, int W) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[CO_HALO * CO_HALO * CO_PS];
  __shared__ f32x4 ws[9 * CO_CC];
  const int tiles_x = (W + CO_T - 1) / CO_T;
  const int y0 = (blockIdx.x / tiles_x) * CO_T, x0 = (blockIdx.x % tiles_x) * CO_T;
  const int ty = threadIdx.x / CO_T, tx = threadIdx.x % CO_T;
  const int y = y0 + ty, xx = x0 + tx;
  float acc[4] = {bias[0], bias[1], bias[2], bias[3]};
  for (int c0 = 0; c0 < C; c0 += CO_CC) {
    const int cn = min(CO_CC, C - c0);  // a multiple of 8
    __syncthreads();  // the previous chunk is no longer read
    // halo: CO_HALO^2 pixels x cn / 8 chunks of 16 bytes
    const int gpp = cn / 8;
    for (int i = threadIdx.x; i < CO_HALO * CO_HALO * gpp; i += 256) {
      const int hp = i / gpp, g = i - hp * gpp;
      const int sy = y0 - 1 + hp / CO_HALO, sx = x0 - 1 + hp % CO_HALO;
      u32x4v v = {0u, 0u, 0u, 0u};
      if (sy >= 0 && sy < H && sx >= 0 && sx < W) v = *(const u32x4v*)(x + ((size_t)sy * W + sx) * ldx + c0 + 8 * g);
      *(u32x4v*)(tile + hp * CO_PS + 8 * g) = v;
    }
    for (int i = threadIdx.x; i < 9 * cn; i += 256) {
      const int tap = i / cn, c = i - tap * cn;
      const uint2 wv = *(const uint2*)(w + ((size_t)tap * C + c0 + c) * 4);
      ws[tap * CO_CC + c] = (f32x4){bf((uint16_t)wv.x), bf((uint16_t)(wv.x >> 16)), bf((uint16_t)wv.y),
                                    bf((uint16_t)(wv.y >> 16))};
    }
    __syncthreads();
#pragma unroll
    for (int tap = 0; tap < 9; tap++) {
      const uint16_t* ip = tile + ((ty + tap / 3) * CO_HALO + tx + tap % 3) * CO_PS;
      const f32x4* wp = ws + tap * CO_CC;
      for (int c = 0; c < cn; c += 8) {
        const u32x4v v = *(const u32x4v*)(ip + c);
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const float a = bf((uint16_t)(v[k >> 1] >> (16 * (k & 1))));
          const f32x4 wk = wp[c + k];
          acc[0] += a * wk[0];
          acc[1] += a * wk[1];
          acc[2] += a * wk[2];
          acc[3] += a * wk[3];
        }
      }
    }
  }
  if (y >= H || xx >= W) return;
  uint32_t out = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float a = fminf(fmaxf(acc[k], -1.f), 1.f);
    const float u = rintf(fminf(fmaxf(a * 0.5f + 0.5f, 0.f), 1.f) * 255.f);
    out |= (uint32_t)u << (8 * k);
  }
  ((uint32_t*)rgba)[(size_t)y * W + xx] = out;
}

// ---- zero-padded copy of a weight Wt[K, N] (row stride N) into [Kp, Np], and of a bias [N] into [Np] ----
__global__ __launch_bounds__(256) void vae_pad_weight_kernel(const uint16_t* __restrict__ w, int K, int N,
                                                            uint16_t* __restrict__ out, int Kp, int Np,
                                                            const float* __restrict__ b, float* __restrict__ bout) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < Np && bout) bout[i] = (b && i < N) ? b[i] : 0.f;
  if (i >= (long long)Kp * Np) return;
  const int k = (int)(i / Np), n = (int)(i % Np);
  out[i] = (k < K && n < N) ? w[(size_t)k * N + n] : (uint16_t)0;
}

// ---- sub-pixel weights of a nearest-2x + 3 x 3 conv (engine/kernels/vae.metal:134-160 semantics): for
//      phase (py, px) = (ph >> 1, ph & 1) and 2 x 2 tap t = (r, s), W2[t Cin + ci, ph Np + co] is the sum of the
//      3 x 3 taps (ky, kx) that land on low-res offset (r + py - 1, s + px - 1): rows ky in [0, py] for r = 0,
//      [1 + py, 2] for r = 1 (columns likewise), summed in fp32 in (ky, kx) order, rounded once to 16 bits.
//      Rows >= 4 Cin and columns co >= Cout of each phase are zero; bias4[ph Np + co] = bias[co] (or 0). ----
template <int DT>
__global__ __launch_bounds__(256) void vae_subpix_weights_kernel(const uint16_t* __restrict__ w, int Cin, int Cout,
                                                                 uint16_t* __restrict__ w2, int Kp, int Np,
                                                                 const float* __restrict__ b, float* __restrict__ b4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  const int N4 = 4 * Np;
  if (i < N4 && b4) b4[i] = (b && (int)(i % Np) < Cout) ? b[i % Np] : 0.f;
  if (i >= (long long)Kp * N4) return;
  const int row = (int)(i / N4), col = (int)(i % N4);
  const int ph = col / Np, co = col - ph * Np;
  float acc = 0.f;
  if (row < 4 * Cin && co < Cout) {
    const int t = row / Cin, ci = row - t * Cin, r = t >> 1, sc = t & 1, py = ph >> 1, px = ph & 1;
    const int y0 = r ? 1 + py : 0, y1 = r ? 2 : py, x0 = sc ? 1 + px : 0, x1 = sc ? 2 : px;
    for (int ky = y0; ky <= y1; ky++)
      for (int kx = x0; kx <= x1; kx++) acc += from16<DT>(w[((size_t)(ky * 3 + kx) * Cin + ci) * Cout + co]);
  }
  w2[i] = to16<DT>(acc);
}

// ---- zero n16 16-byte chunks (a kernel, not a memset node, so that a captured decode replays correctly) ----
__global__ __launch_bounds__(256) void vae_zero_kernel(u32x4v* __restrict__ p, long long n16) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += (long long)gridDim.x * 256)
    p[i] = (u32x4v){0u, 0u, 0u, 0u};
}

inline unsigned blocks(long long n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

int vae_unpack(hipStream_t st, const float* z, const float* mean, const float* stdv, const float* w, const float* b,
               void* y, int H16, int W16, Err& e) {
  if (!z || !mean || !stdv || !w || !b || !y) return e.fail("vae_unpack: null pointer");
  if (H16 <= 0 || W16 <= 0) return e.fail("vae_unpack: empty latent %d x %d", H16, W16);
  if ((uintptr_t)y & 15) return e.fail("vae_unpack: y must be 16-byte aligned");
  hipLaunchKernelGGL(vae_unpack_kernel, dim3(blocks(4LL * H16 * W16, 256)), dim3(256), 0, st, z, mean, stdv, w, b,
                     (uint16_t*)y, H16, W16);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_unpack launch");
}

int vae_im2col(hipStream_t st, const void* x, int ldx, int C, int H, int W, int up, int m0, int rows, void* col,
               int Kpad, Err& e) {
  if (!x || !col) return e.fail("vae_im2col: null pointer");
  if (C <= 0 || C % 8 || ldx < C || ldx % 8) return e.fail("vae_im2col: C=%d ldx=%d must be multiples of 8", C, ldx);
  if (H <= 0 || W <= 0 || (up && (H % 2 || W % 2))) return e.fail("vae_im2col: bad size %d x %d (up=%d)", H, W, up);
  if (Kpad < 9 * C || Kpad % 8) return e.fail("vae_im2col: Kpad=%d < 9 C or not a multiple of 8", Kpad);
  if (m0 < 0 || rows <= 0 || m0 + rows > H * W) return e.fail("vae_im2col: rows [%d, %d) outside %d pixels", m0,
                                                              m0 + rows, H * W);
  if (((uintptr_t)x | (uintptr_t)col) & 15) return e.fail("vae_im2col: 16-byte alignment");
  hipLaunchKernelGGL(vae_im2col_kernel, dim3(blocks((long long)rows * (Kpad / 8), 256)), dim3(256), 0, st,
                     (const uint16_t*)x, ldx, C, H, W, up, m0, rows, (uint16_t*)col, Kpad);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_im2col launch");
}

int vae_norm_silu(hipStream_t st, const void* x, int ldx, const float* gamma, void* y, int ldy, int P, int C, int silu,
                  Err& e) {
  if (!x || !gamma || !y) return e.fail("vae_norm_silu: null pointer");
  if (P <= 0 || C <= 0 || C % 8 || ldx < C || ldy < C || ldx % 8 || ldy % 8)
    return e.fail("vae_norm_silu: bad shape P=%d C=%d ldx=%d ldy=%d", P, C, ldx, ldy);
  if (((uintptr_t)x | (uintptr_t)y) & 15) return e.fail("vae_norm_silu: 16-byte alignment");
  const bool g16 = !((uintptr_t)gamma & 15);
  if (g16 && C == 96)
    hipLaunchKernelGGL(vae_norm_silu_reg_kernel<4>, dim3(blocks(P, 64)), dim3(256), 0, st, (const uint16_t*)x, ldx,
                       gamma, (uint16_t*)y, ldy, P, silu);
  else if (g16 && C == 192)
    hipLaunchKernelGGL(vae_norm_silu_reg_kernel<8>, dim3(blocks(P, 32)), dim3(256), 0, st, (const uint16_t*)x, ldx,
                       gamma, (uint16_t*)y, ldy, P, silu);
  else if (g16 && C == 384)
    hipLaunchKernelGGL(vae_norm_silu_reg_kernel<16>, dim3(blocks(P, 16)), dim3(256), 0, st, (const uint16_t*)x, ldx,
                       gamma, (uint16_t*)y, ldy, P, silu);
  else
    hipLaunchKernelGGL(vae_norm_silu_kernel, dim3(blocks(P, 16)), dim3(256), 0, st, (const uint16_t*)x, ldx, gamma,
                       (uint16_t*)y, ldy, P, C, silu);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_norm_silu launch");
}

int vae_add(hipStream_t st, void* y, const void* a, long long n, Err& e) {
  if (!y || !a) return e.fail("vae_add: null pointer");
  if (n <= 0 || n % 8) return e.fail("vae_add: n=%lld must be a positive multiple of 8", n);
  if (((uintptr_t)y | (uintptr_t)a) & 15) return e.fail("vae_add: 16-byte alignment");
  hipLaunchKernelGGL(vae_add_kernel, dim3(blocks(n / 8, 256)), dim3(256), 0, st, (uint16_t*)y, (const uint16_t*)a,
                     n / 8);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_add launch");
}

int vae_transpose(hipStream_t st, const void* in, int ld, int off, int P, int C, void* out, int ldo, Err& e) {
  if (!in || !out) return e.fail("vae_transpose: null pointer");
  if (P <= 0 || C <= 0 || off < 0 || off + C > ld || ldo < P) return e.fail("vae_transpose: bad shape");
  hipLaunchKernelGGL(vae_transpose_kernel, dim3(blocks(P, 64), blocks(C, 64)), dim3(256), 0, st,
                     (const uint16_t*)in, ld, off, P, C, (uint16_t*)out, ldo);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_transpose launch");
}

int vae_softmax(hipStream_t st, const float* S, int ld, int rows, int n, float scale, void* Pm, Err& e) {
  if (!S || !Pm) return e.fail("vae_softmax: null pointer");
  if (rows <= 0 || n <= 0 || n > ld) return e.fail("vae_softmax: bad shape rows=%d n=%d ld=%d", rows, n, ld);
  constexpr int NV = 16;
  if (n <= 1024 * NV && ld % 4 == 0 && !((uintptr_t)S & 15) && !((uintptr_t)Pm & 7))
    hipLaunchKernelGGL(vae_softmax_rows_kernel<NV>, dim3(rows), dim3(256), 0, st, S, ld, n, scale, (uint16_t*)Pm);
  else
    hipLaunchKernelGGL(vae_softmax_kernel, dim3(rows), dim3(256), 0, st, S, ld, n, scale, (uint16_t*)Pm);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_softmax launch");
}

int vae_conv_out(hipStream_t st, const void* x, int ldx, int C, const void* w, const float* bias, void* rgba, int H,
                 int W, Err& e) {
  if (!x || !w || !bias || !rgba) return e.fail("vae_conv_out: null pointer");
  if (C <= 0 || C % 8 || ldx < C || ldx % 8 || H <= 0 || W <= 0) return e.fail("vae_conv_out: bad shape");
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 7) || ((uintptr_t)rgba & 3)) return e.fail("vae_conv_out: alignment");
  const long long tiles = (long long)((H + CO_T - 1) / CO_T) * ((W + CO_T - 1) / CO_T);
  if (tiles >= (1LL << 31)) return e.fail("vae_conv_out: image too large");
  hipLaunchKernelGGL(vae_conv_out_kernel, dim3((unsigned)tiles), dim3(256), 0, st, (const uint16_t*)x,
                     ldx, C, (const uint16_t*)w, bias, (uint8_t*)rgba, H, W);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_conv_out launch");
}

int vae_zero(hipStream_t st, void* p, size_t bytes, Err& e) {
  if (!p || ((uintptr_t)p & 15) || (bytes & 15)) return e.fail("vae_zero: pointer and size must be 16-byte aligned");
  if (!bytes) return KH_OK;
  const long long n16 = (long long)(bytes / 16);
  hipLaunchKernelGGL(vae_zero_kernel, dim3((unsigned)std::min<long long>(blocks(n16, 256), 4096)), dim3(256), 0, st,
                     (u32x4v*)p, n16);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_zero launch");
}

int vae_subpix_weights(hipStream_t st, const void* w, int dtype, int Cin, int Cout, void* w2, int Kp, int Np,
                       const float* b, float* b4, Err& e) {
  if (!w || !w2) return e.fail("vae_subpix_weights: null pointer");
  if (dtype != KH_F16 && dtype != KH_BF16) return e.fail("vae_subpix_weights: dtype must be f16 or bf16");
  if (Cin <= 0 || Cout <= 0 || Kp < 4 * Cin || Np < Cout) return e.fail("vae_subpix_weights: bad shape");
  const long long n = (long long)Kp * 4 * Np;
  if (dtype == KH_BF16)
    hipLaunchKernelGGL(vae_subpix_weights_kernel<KH_BF16>, dim3(blocks(n, 256)), dim3(256), 0, st, (const uint16_t*)w,
                       Cin, Cout, (uint16_t*)w2, Kp, Np, b, b4);
  else
    hipLaunchKernelGGL(vae_subpix_weights_kernel<KH_F16>, dim3(blocks(n, 256)), dim3(256), 0, st, (const uint16_t*)w,
                       Cin, Cout, (uint16_t*)w2, Kp, Np, b, b4);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_subpix_weights launch");
}

int vae_pad_weight(hipStream_t st, const void* w, int K, int N, void* out, int Kp, int Np, const float* b, float* bout,
                   Err& e) {
  if (!w || !out) return e.fail("vae_pad_weight: null pointer");
  if (K <= 0 || N <= 0 || Kp < K || Np < N) return e.fail("vae_pad_weight: bad shape");
  hipLaunchKernelGGL(vae_pad_weight_kernel, dim3(blocks((long long)Kp * Np, 256)), dim3(256), 0, st,
                     (const uint16_t*)w, K, N, (uint16_t*)out, Kp, Np, b, bout);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "vae_pad_weight launch");
}

}  // namespace kh
