// Dequant-GEMM with fused epilogues for MI355X (gfx950): the DiT projections of the Krea 2 engine.
//
//   acc[M, N] = X[M, K] (fp16 / bf16, row-major) x W~[K, N] (W stored input-major int8 or 16-bit), fp32.
//
// Semantics follow engine/kernels/gemm.metal:102-309 (gemm_tiled<EPI, QW, 0, 0>); the design is CDNA4's:
//  * Block tile 256 (n) x 256 (m) x 64 (k), 512 threads = 8 wave64s in a 4 (n) x 2 (m) grid; each wave
//    owns 64 n x 128 m = 2 x 4 MFMA blocks of v_mfma_f32_32x32x16_{f16,bf16}.
//  * The MFMA "A" operand is the weight tile (rows n), "B" the activation tile (columns m), so each lane's
//    accumulator holds 4 consecutive output columns n of one row m: epilogue loads of scale / bias / gate
//    and the 16-bit or f32 stores are 8- or 16-byte vectors.
//  * Both tiles live in LDS as [row][64 k] 16-bit with the 16-byte chunk index XOR-swizzled by (row & 7),
//    so the MFMA operand reads (one ds_read_b128 per lane: 8 consecutive k of one row) are conflict-free.
//  * Weights: each thread loads 8 k-rows x 4 n-columns (a dword per int8 row, coalesced 256 B per wave
//    and row), and converts them to 16-bit while transposing them in registers (v_perm_b32) into four
//    16-byte k-vectors:
//      - int8 per-channel, fp16 activations: 0x6400 | (q ^ 0x80) is the fp16 value 1024 + q + 128, so one
//        packed subtract of 1152 gives q exactly (3 VALU ops per 2 weights); the per-channel scale is
//        applied to the fp32 accumulator in the epilogue (q exact => no dequant rounding at all);
//      - int8 per-channel, bf16 activations: 2^23 + (q ^ 0x80) as f32 minus 2^23 + 128 is exactly q, whose
//        upper 16 bits are its bf16 encoding;
//      - int8 with group scales (the reference's dit_q8 format): round16(fma(q + 128, s, -128 s)), which
//        is the single-rounded f32 product q * s of gemm.metal:190-196 followed by one 16-bit rounding;
//      - 16-bit weights: the same transpose, halfwords only.
//  * Double-buffered LDS (2 x 64 KB): step t+1 is fetched into registers while step t is multiplied, then
//    converted and stored into the other buffer; one workgroup barrier per K step.
//  * Tile order: block ids are first made contiguous per XCD (the dispatcher deals workgroups round-robin
//    to the 8 XCDs, each with its own L2), then walked in groups of 8 tile rows, so co-resident
//    workgroups of one XCD share both X row panels and W column panels in that XCD's L2.
#include "kh_common.h"
#include "kh_internal.h"

namespace kh {

namespace {

constexpr int BM = 256, BN = 256, BK = 64, NTHR = 512;
constexpr int TILE = BM * BK;  // 16-bit elements of one X (or W) tile
constexpr int GROUP_M = 8;

enum { WF_16 = 0, WF_I8_CHANNEL = 1, WF_I8_GROUP = 2 };

struct GemmArgs {
  const void* A;
  const void* W;
  const void* S;
  void* C;
  const float* vec;
  int M, N, K, lda, ldw, ldc, group, s_dtype;
};

template <int ACT>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (ACT == KH_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

// Weight registers of one thread for one K step: 8 k-rows x 4 n-columns.
template <int WF>
struct WRegs;
template <>
struct WRegs<WF_16> {
  u32x2 r[8];
};
template <>
struct WRegs<WF_I8_CHANNEL> {
  uint32_t r[8];
};
template <>
struct WRegs<WF_I8_GROUP> {
  uint32_t r[8];
  float s[4];
};

template <int ACT, int WF>
__device__ __forceinline__ void convert_w(const WRegs<WF>& w, u32x4 (&out)[4]) {
  if constexpr (WF == WF_16) {
    // halfword j of rows 2p (low) and 2p + 1 (high)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t jj = (j & 1) * 2;
      const uint32_t sel = (jj) | ((jj + 1) << 8) | ((jj + 4) << 16) | ((jj + 5) << 24);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t lo = (j < 2) ? w.r[2 * p].x : w.r[2 * p].y;
        const uint32_t hi = (j < 2) ? w.r[2 * p + 1].x : w.r[2 * p + 1].y;
        out[j][p] = __builtin_amdgcn_perm(hi, lo, sel);
      }
    }
  } else if constexpr (WF == WF_I8_CHANNEL && ACT == KH_F16) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t sel = (uint32_t)j | (0x0cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0cu << 24);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t d = __builtin_amdgcn_perm(w.r[2 * p + 1], w.r[2 * p], sel) ^ 0x64806480u;
        const f16x2 h = __builtin_bit_cast(f16x2, d) - (f16x2){(_Float16)1152.0f, (_Float16)1152.0f};
        out[j][p] = __builtin_bit_cast(uint32_t, h);
      }
    }
  } else if constexpr (WF == WF_I8_CHANNEL) {  // bf16 activations
    uint32_t r[8];
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = w.r[i] ^ 0x80808080u;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t sel = (uint32_t)j | (0x0cu << 8) | (0x0cu << 16) | (7u << 24);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const float lo = __builtin_bit_cast(float, __builtin_amdgcn_perm(0x4b000000u, r[2 * p], sel)) - 8388736.0f;
        const float hi = __builtin_bit_cast(float, __builtin_amdgcn_perm(0x4b000000u, r[2 * p + 1], sel)) - 8388736.0f;
        out[j][p] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo),
                                          0x07060302u);
      }
    }
  } else {  // WF_I8_GROUP: round16(q * s), single f32 rounding of the product
    uint32_t r[8];
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = w.r[i] ^ 0x80808080u;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float s = w.s[j], nb = -128.0f * w.s[j];
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const float lo = __builtin_fmaf((float)((r[2 * p] >> (8 * j)) & 0xffu), s, nb);
        const float hi = __builtin_fmaf((float)((r[2 * p + 1] >> (8 * j)) & 0xffu), s, nb);
        out[j][p] = (uint32_t)to16<ACT>(lo) | ((uint32_t)to16<ACT>(hi) << 16);
      }
    }
  }
}

template <int ACT, int WF, int EPI>
__global__ __launch_bounds__(NTHR) void gemm_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2 * TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- tile order (XCD-contiguous, then grouped by GROUP_M tile rows) ----
  const int tiles_n = p.N / BN + (p.N % BN ? 1 : 0), tiles_m = (p.M + BM - 1) / BM;
  const int total = tiles_n * tiles_m;
  int pid = blockIdx.x;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
  const int group_sz = GROUP_M * tiles_n;
  const int first_m = (pid / group_sz) * GROUP_M;
  const int gm = min(GROUP_M, tiles_m - first_m);
  const int in_g = pid % group_sz;
  const int m0 = (first_m + in_g % gm) * BM, n0 = (in_g / gm) * BN;

  // ---- X tile: 4 chunks of 16 B per thread (8 lanes per 128-byte row) ----
  const uint16_t* a_src[4];
  int a_lds[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int cid = tid + r * NTHR, row = cid >> 3, ch = cid & 7;
    const int grow = min(m0 + row, p.M - 1);  // rows >= M are computed from row M-1, never stored
    a_src[r] = (const uint16_t*)p.A + (size_t)grow * p.lda + ch * 8;
    a_lds[r] = row * BK + ((ch ^ (row & 7)) * 8);
  }
  // ---- W tile: k-rows wave*8 .. +7, columns n0 + lane*4 .. +3 ----
  const int wcol = min(n0 + lane * 4, p.N - 4);  // columns >= N (partial last tile) are never stored
  const size_t wrow_bytes = (size_t)p.ldw * (WF == WF_16 ? 2 : 1);
  const char* w_src = (const char*)p.W + (size_t)(wave * 8) * wrow_bytes + (size_t)wcol * (WF == WF_16 ? 2 : 1);
  int w_lds[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int nl = lane * 4 + j;
    w_lds[j] = TILE + nl * BK + ((wave ^ (nl & 7)) * 8);
  }

  u32x4 ra[4];
  WRegs<WF> rw;
  auto load_step = [&](int t) {
    const int k0 = t * BK;
#pragma unroll
    for (int r = 0; r < 4; r++) ra[r] = *(const u32x4*)(a_src[r] + k0);
    const char* ws = w_src + (size_t)k0 * wrow_bytes;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      if constexpr (WF == WF_16)
        rw.r[i] = *(const u32x2*)(ws + (size_t)i * wrow_bytes);
      else
        rw.r[i] = *(const uint32_t*)(ws + (size_t)i * wrow_bytes);
    }
    if constexpr (WF == WF_I8_GROUP) {
      const size_t g = (size_t)(k0 / p.group) * p.ldw + wcol;
#pragma unroll
      for (int j = 0; j < 4; j++) rw.s[j] = load_scale(p.S, p.s_dtype, g + j);
    }
  };
  auto store_step = [&](int buf) {
    uint16_t* L = lds[buf];
#pragma unroll
    for (int r = 0; r < 4; r++) *(u32x4*)(L + a_lds[r]) = ra[r];
    u32x4 wv[4];
    convert_w<ACT, WF>(rw, wv);
#pragma unroll
    for (int j = 0; j < 4; j++) *(u32x4*)(L + w_lds[j]) = wv[j];
  };

  // ---- MFMA operand addressing: wave (wn, wm) owns n [wn*64, +64), m [wm*128, +128) ----
  const int wn = wave & 3, wm = wave >> 2;
  const int l32 = lane & 31, khalf = lane >> 5;
  const int w_frag = TILE + (wn * 64 + l32) * BK;
  const int x_frag = (wm * 128 + l32) * BK;

  f32x16 acc[2][4];
#pragma unroll
  for (int jb = 0; jb < 2; jb++)
#pragma unroll
    for (int ib = 0; ib < 4; ib++) acc[jb][ib] = (f32x16){};

  const int nk = p.K / BK;
  load_step(0);
  store_step(0);
  __syncthreads();
  for (int t = 0; t < nk; t++) {
    const int cur = t & 1;
    if (t + 1 < nk) load_step(t + 1);
    const uint16_t* L = lds[cur];
#pragma unroll
    for (int s = 0; s < BK / 16; s++) {
      const int sw = ((s * 2 + khalf) ^ (lane & 7)) * 8;
      u32x4 wf[2], xf[4];
#pragma unroll
      for (int jb = 0; jb < 2; jb++) wf[jb] = *(const u32x4*)(L + w_frag + jb * 32 * BK + sw);
#pragma unroll
      for (int ib = 0; ib < 4; ib++) xf[ib] = *(const u32x4*)(L + x_frag + ib * 32 * BK + sw);
#pragma unroll
      for (int jb = 0; jb < 2; jb++)
#pragma unroll
        for (int ib = 0; ib < 4; ib++) acc[jb][ib] = mfma32<ACT>(wf[jb], xf[ib], acc[jb][ib]);
    }
    if (t + 1 < nk) store_step(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds, per (jb, ib), row m = m0 + wm*128 + ib*32 + l32 and columns
  //      n = n0 + wn*64 + jb*32 + g*8 + khalf*4 + e  (g = 0..3, e = 0..3) in acc[jb][ib][g*4 + e] ----
  const bool per_channel = (WF == WF_I8_CHANNEL);
#pragma unroll
  for (int jb = 0; jb < 2; jb++) {
    if (EPI == KH_EPI_SWIGLU && jb == 1) break;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int n = n0 + wn * 64 + jb * 32 + g * 8 + khalf * 4;
      if (n >= p.N) continue;
      float sc[4] = {1.f, 1.f, 1.f, 1.f}, sc_up[4] = {1.f, 1.f, 1.f, 1.f}, vv[4] = {0.f, 0.f, 0.f, 0.f};
      if (per_channel) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          sc[e] = load_scale(p.S, p.s_dtype, n + e);
          if (EPI == KH_EPI_SWIGLU) sc_up[e] = load_scale(p.S, p.s_dtype, n + 32 + e);
        }
      }
      if (EPI == KH_EPI_RESID_GATE || EPI == KH_EPI_BIAS16 || EPI == KH_EPI_BIAS_F32) {
        const f32x4 v4 = *(const f32x4*)(p.vec + n);
#pragma unroll
        for (int e = 0; e < 4; e++) vv[e] = v4[e];
      }
#pragma unroll
      for (int ib = 0; ib < 4; ib++) {
        const int m = m0 + wm * 128 + ib * 32 + l32;
        if (m >= p.M) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = acc[jb][ib][g * 4 + e] * sc[e];
        if constexpr (EPI == KH_EPI_SWIGLU) {
          uint16_t h[4];
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = to16<ACT>(silu_f(v[e]) * (acc[1][ib][g * 4 + e] * sc_up[e]));
          const int col = (n / 64) * 32 + (n % 32);
          *(u32x2*)((uint16_t*)p.C + (size_t)m * p.ldc + col) =
              (u32x2){(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
        } else if constexpr (EPI == KH_EPI_STORE16 || EPI == KH_EPI_GELU || EPI == KH_EPI_BIAS16) {
          uint16_t h[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float o = v[e];
            if (EPI == KH_EPI_GELU) o = gelu_tanh_f(o);
            if (EPI == KH_EPI_BIAS16) o += vv[e];
            h[e] = to16<ACT>(o);
          }
          *(u32x2*)((uint16_t*)p.C + (size_t)m * p.ldc + n) =
              (u32x2){(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
        } else {
          f32x4* dst = (f32x4*)((float*)p.C + (size_t)m * p.ldc + n);
          f32x4 o;
          if (EPI == KH_EPI_RESID_GATE || EPI == KH_EPI_RESID) o = *dst;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            if (EPI == KH_EPI_F32) o[e] = v[e];
            else if (EPI == KH_EPI_BIAS_F32) o[e] = v[e] + vv[e];
            else if (EPI == KH_EPI_RESID) o[e] += v[e];
            else o[e] += vv[e] * v[e];
          }
          *dst = o;
        }
      }
    }
  }
}

template <int ACT, int WF>
hipError_t launch_epi(int epi, const GemmArgs& a, hipStream_t st) {
  const int tiles = ((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
  dim3 grid(tiles), block(NTHR);
  switch (epi) {
#define KH_CASE(E)                                                        \
  case E:                                                                 \
    hipLaunchKernelGGL((gemm_kernel<ACT, WF, E>), grid, block, 0, st, a); \
    break;
    KH_CASE(KH_EPI_STORE16)
    KH_CASE(KH_EPI_F32)
    KH_CASE(KH_EPI_RESID_GATE)
    KH_CASE(KH_EPI_RESID)
    KH_CASE(KH_EPI_SWIGLU)
    KH_CASE(KH_EPI_GELU)
    KH_CASE(KH_EPI_BIAS16)
    KH_CASE(KH_EPI_BIAS_F32)
#undef KH_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int ACT>
hipError_t launch_wf(int wf, int epi, const GemmArgs& a, hipStream_t st) {
  if (wf == WF_16) return launch_epi<ACT, WF_16>(epi, a, st);
  if (wf == WF_I8_CHANNEL) return launch_epi<ACT, WF_I8_CHANNEL>(epi, a, st);
  return launch_epi<ACT, WF_I8_GROUP>(epi, a, st);
}

}  // namespace

int gemm(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
         int lda, int ldw, int ldc, const void* vec, Err& e) {
  if (epi < KH_EPI_STORE16 || epi > KH_EPI_BIAS_F32) return e.fail("gemm: unknown epilogue %d", epi);
  if (a_dtype != KH_F16 && a_dtype != KH_BF16) return e.fail("gemm: activations must be f16 or bf16");
  if (M <= 0 || N <= 0 || K <= 0) return e.fail("gemm: empty shape M=%d N=%d K=%d", M, N, K);
  if (N % 64 || K % BK) return e.fail("gemm: unsupported shape N=%d K=%d (need N %% 64 == 0, K %% 64 == 0)", N, K);
  if (!A || !W.w || !C) return e.fail("gemm: null A / W / C");
  if (lda < K || lda % 8) return e.fail("gemm: lda=%d must be >= K and a multiple of 8", lda);
  if (ldw < N) return e.fail("gemm: ldw=%d < N=%d", ldw, N);
  const int out_cols = epi == KH_EPI_SWIGLU ? N / 2 : N;
  if (ldc < out_cols || ldc % 4) return e.fail("gemm: ldc=%d must be >= %d and a multiple of 4", ldc, out_cols);
  const bool needs_vec = epi == KH_EPI_RESID_GATE || epi == KH_EPI_BIAS16 || epi == KH_EPI_BIAS_F32;
  if (needs_vec && !vec) return e.fail("gemm: epilogue %d needs vec", epi);
  int wf;
  int group = 0;
  if (W.w_dtype == KH_I8) {
    if (!W.s) return e.fail("gemm: int8 weights need scales");
    if (W.s_dtype != KH_F32 && W.s_dtype != KH_F16 && W.s_dtype != KH_BF16) return e.fail("gemm: bad scale dtype");
    if (ldw % 16) return e.fail("gemm: int8 ldw=%d must be a multiple of 16", ldw);
    group = W.group <= 0 ? K : W.group;
    if (group >= K) {
      if (group != K) return e.fail("gemm: group %d > K %d", group, K);
      wf = WF_I8_CHANNEL;
    } else {
      if (group % BK || K % group) return e.fail("gemm: int8 group %d must divide K and be a multiple of 64", group);
      wf = WF_I8_GROUP;
    }
  } else {
    if (W.w_dtype != a_dtype) return e.fail("gemm: 16-bit weights must match the activation type");
    if (ldw % 8) return e.fail("gemm: ldw=%d must be a multiple of 8", ldw);
    wf = WF_16;
  }
  GemmArgs a{A, W.w, W.s, C, (const float*)vec, M, N, K, lda, ldw, ldc, group, W.s_dtype};
  hipError_t r = a_dtype == KH_F16 ? launch_wf<KH_F16>(wf, epi, a, st) : launch_wf<KH_BF16>(wf, epi, a, st);
  if (r != hipSuccess) return e.hip(r, "gemm launch");
  return KH_OK;
}

}  // namespace kh
