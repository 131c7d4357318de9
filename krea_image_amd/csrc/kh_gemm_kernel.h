// Dequant-GEMM with fused epilogues for MI355X (gfx950): the DiT projections of the Krea 2 engine.
//
//   acc[M, N] = X[M, K] (fp16 / bf16, row-major) x W~[K, N] (W stored input-major int8 or 16-bit), fp32.
//
// Semantics follow engine/kernels/gemm.metal:102-309 (gemm_tiled<EPI, QW, 0, 0>); the design is CDNA4's:
//  * Block tile 256 (n) x 256 (m) x 64 (k), 512 threads = 8 wave64s (two per SIMD) in a 2 (n) x 4 (m) grid;
//    each wave owns 128 n x 64 m = 4 x 2 MFMA blocks of v_mfma_f32_32x32x16_{f16,bf16}. A 192 (n) x 256 (m)
//    variant (waves 96 n x 64 m) and a 128 (n) one serve shapes that 256-wide tiles would pad or leave CUs
//    idle on (plan_launch in kh_gemm.hip).
//  * The MFMA "A" operand is the weight tile (rows n), "B" the activation tile (columns m), so each lane's
//    accumulator holds 4 consecutive output columns n of one row m: epilogue loads of scale / bias / gate
//    and the 16-bit or f32 stores are 8- or 16-byte vectors.
//  * Both tiles live in LDS as [row][64 k] 16-bit with the 16-byte chunk index XOR-swizzled by swz(row),
//    so the MFMA operand reads (one ds_read_b128 per lane: 8 consecutive k of one row) are conflict-free
//    (gfx950 LDS: 32 banks x 4 B, 8 lanes of a 16-byte access per cycle).
//  * Activations stream global -> LDS by DMA (global_load_lds, no VGPR staging) through a 3-stage ring.
//  * Weights: each thread loads 8 k-rows x 4 n-columns two K steps ahead (a dword per int8 row, coalesced
//    256 B per wave and row, or with WF_PK the same 32 bytes as two 16-byte loads from kh_pack_int8's
//    layout; inline-asm loads with explicit waits), and converts them to 16-bit while
//    transposing them in registers (v_perm_b32) into four 16-byte k-vectors, stored to a 2-stage LDS ring
//    between the MFMA slices:
//      - int8 per-channel, fp16 activations: 0x6400 | (q ^ 0x80) is the fp16 value 1024 + q + 128, so one
//        packed subtract of 1152 gives q exactly (3 VALU ops per 2 weights); the per-channel scale is
//        applied to the fp32 accumulator in the epilogue (q exact => no dequant rounding at all);
//      - int8 per-channel, bf16 activations: 2^23 + (q ^ 0x80) as f32 minus 2^23 + 128 is exactly q, whose
//        upper 16 bits are its bf16 encoding;
//      - int8 with group scales (the reference's dit_q8 format): round16(fma(q + 128, s, -128 s)), which
//        is the single-rounded f32 product q * s of gemm.metal:190-196 followed by one 16-bit rounding;
//      - 16-bit weights: the same transpose, halfwords only.
//    One workgroup barrier per K step; the loop body has no branches.
//  * Tile order: block ids are first made contiguous per XCD (the dispatcher deals workgroups round-robin
//    to the 8 XCDs, each with its own L2), then walked in groups of 4 tile rows, so co-resident
//    workgroups of one XCD share both X row panels and W column panels in that XCD's L2.
//  * Shapes whose tiles would fill under 60 % of a wave of workgroups run stream-K (see plan_launch).
//
// This header holds the kernel and its launch templates; kh_gemm_f16.hip and kh_gemm_bf16.hip instantiate them
// (one translation unit per activation type, compiled in parallel), kh_gemm.hip plans the launches.
#pragma once
#include <type_traits>
#include <utility>

#include "kh_common.h"
#include "kh_gemm_args.h"

namespace kh {

namespace {

using namespace gemm_detail;

// 16 zero bytes in device memory (never written): the source of the activation DMA for the taps of a
// convolution that fall outside the image (zero padding) and for the K padding past 9 C.
__device__ __attribute__((aligned(16))) uint32_t g_zero_chunk[4] = {0u, 0u, 0u, 0u};

// 16-byte chunk XOR of LDS row `row` (rows are 128 bytes = 8 chunks of 8 k). Depends on row & 31 only, is a
// bijection on any 8 consecutive rows (operand reads: 32 consecutive rows per instruction) and on rows
// {j, j+4, ..., j+28} (the weight writes: lane L writes row 4L + j).
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 2)) & 7; }

template <int ACT>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (ACT == KH_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

#ifndef SCHED_FENCE
#define SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)
#endif

// Raw weight registers of one thread for one K step: KR k-rows x 4 n-columns (+ the 4 column scales' raw
// bits for the group format: f32, or f16 / bf16 in the low half).
template <int WF, int KR>
struct WRaw {
  union {
    uint32_t r[KR];
    u32x4 v[KR / 4];  // the packed layout's 16-byte loads
  };
  uint32_t s[4];
};
template <int KR>
struct WRaw<WF_16, KR> {
  u32x2 r[KR];
};

template <int WF>
__device__ __forceinline__ float scale_from_bits(uint32_t b) {
  if constexpr (WF == WF_I8_GROUP) return __builtin_bit_cast(float, b);
  if constexpr (WF == WF_I8_GROUP_BF16) return __builtin_bit_cast(float, b << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// Convert k-rows [8h, 8h+8) of column j to one 16-byte vector of 8 consecutive k (16-bit each).
template <int ACT, int WF, int KR>
__device__ __forceinline__ u32x4 convert_chunk(const WRaw<WF, KR>& w, int j, int h) {
  u32x4 out;
  if constexpr (WF == WF_16) {
    const uint32_t jj = (j & 1) * 2;
    const uint32_t sel = jj | ((jj + 1) << 8) | ((jj + 4) << 16) | ((jj + 5) << 24);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t lo = (j < 2) ? w.r[8 * h + 2 * p].x : w.r[8 * h + 2 * p].y;
      const uint32_t hi = (j < 2) ? w.r[8 * h + 2 * p + 1].x : w.r[8 * h + 2 * p + 1].y;
      out[p] = __builtin_amdgcn_perm(hi, lo, sel);
    }
  } else if constexpr (WF == WF_I8_CHANNEL && ACT == KH_F16) {
    // 0x6400 | (q ^ 0x80) is the fp16 number 1024 + q + 128: one packed subtract of 1152 gives q exactly
    const uint32_t sel = (uint32_t)j | (0x0cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0cu << 24);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t d = __builtin_amdgcn_perm(w.r[8 * h + 2 * p + 1], w.r[8 * h + 2 * p], sel) ^ 0x64806480u;
      const f16x2 v = __builtin_bit_cast(f16x2, d) - (f16x2){(_Float16)1152.0f, (_Float16)1152.0f};
      out[p] = __builtin_bit_cast(uint32_t, v);
    }
  } else if constexpr (WF == WF_I8_CHANNEL) {
    // bf16: the f32 2^23 + (q ^ 0x80) minus 2^23 + 128 is q exactly; its upper half is its bf16 encoding
    const uint32_t sel = (uint32_t)j | (0x0cu << 8) | (0x0cu << 16) | (7u << 24);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t a = w.r[8 * h + 2 * p] ^ 0x80808080u, b = w.r[8 * h + 2 * p + 1] ^ 0x80808080u;
      const float lo = __builtin_bit_cast(float, __builtin_amdgcn_perm(0x4b000000u, a, sel)) - 8388736.0f;
      const float hi = __builtin_bit_cast(float, __builtin_amdgcn_perm(0x4b000000u, b, sel)) - 8388736.0f;
      out[p] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x07060302u);
    }
  } else {
    // group scales: round16(q * s) with the product rounded once in f32: fma(q + 128, s, -128 s)
    const float s = scale_from_bits<WF>(w.s[j]), nb = -128.0f * s;
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t a = w.r[8 * h + 2 * p] ^ 0x80808080u, b = w.r[8 * h + 2 * p + 1] ^ 0x80808080u;
      const float lo = __builtin_fmaf((float)((a >> (8 * j)) & 0xffu), s, nb);
      const float hi = __builtin_fmaf((float)((b >> (8 * j)) & 0xffu), s, nb);
      out[p] = pack16<ACT>(lo, hi);
    }
  }
  return out;
}

// Wave layout of a 256 x 256 block tile with WAVES wave64s: a 2 (n) x WAVES/2 (m) grid, each wave owning
// 128 n x WME m = 4 x IB blocks of 32 x 32. WAVES = 8 runs two waves per SIMD (128 accumulators each), so
// one wave's LDS / memory waits are covered by the other wave's MFMAs.
template <int WAVES>
struct Cfg {
  static constexpr int NTHR = 64 * WAVES;
  static constexpr int WME = BM / (WAVES / 2);  // m extent of a wave
  static constexpr int IB = WME / 32;           // 32-row MFMA blocks per wave
  static constexpr int X_LOADS = 32 / WAVES;    // 1 KB LDS-direct activation loads per thread per K step
  static constexpr int KR = BK / WAVES;         // weight k-rows loaded per thread per K step
  static constexpr int WCH = 4 * (KR / 8);      // converted 16-byte weight chunks per thread per K step
  // loads issued per thread per K step, counted in the waits (a lower bound when group scales are loaded)
  static constexpr int LOADS = X_LOADS + KR;    // + 4 scale loads for the group format
};

// TN: block tile width in n, 256, 192 or 128 (narrow tiles serve N that 256 would pad, e.g. 96 or 384
// channels, and fill a wave of workgroups where 256 would leave CUs idle, e.g. 4096 x 3072 outputs: 16 x 16
// tiles of 192 instead of 16 x 12). The waves' n extent is TN / 2 = JB blocks of 32.
// CONV: the activation tile is gathered from an image as an implicit 3 x 3 convolution (GemmArgs cv_*).
// WFX: weight format, optionally | WF_PK (packed int8 layout).
// WA: K steps ahead that weights are loaded (2 or 3). With 2, the loads issued in step t (activations and
// weights of step t + 2) are waited for at the start of step t + 1: each has one step to land. With 3, the
// weights of step t + 3 go into a third raw register set and the step waits once, at its end, for the loads
// issued one step earlier: activations and weights both get two steps. The same products are summed in the
// same order: results are bitwise equal.
template <int ACT, int WFX, int EPI, int WAVES, bool SK, int TN = BN, bool CONV = false, int WA = 2>
__global__ __launch_bounds__(64 * WAVES, 1) void gemm_kernel(GemmArgs p) {
  constexpr bool PK = (WFX & WF_PK) != 0;
  constexpr int WF = WFX & ~WF_PK;
  static_assert(WA == 2 || (WA == 3 && !SK && !CONV), "three-step weight prefetch: data-parallel GEMMs only");
  static_assert(!PK || (WF != WF_16 && !CONV), "packed layout: int8 weights, plain GEMM");
  using C_ = Cfg<WAVES>;
  static_assert(TN == BN || ((TN == 192 || TN == 128) && !SK && !wide_only(EPI)),
                "narrow tiles (192 / 128): data-parallel, no SwiGLU");
  constexpr int JB = TN / 64, WN = TN / 2;
  constexpr int NTHR = C_::NTHR, IB = C_::IB, X_LOADS = C_::X_LOADS, KR = C_::KR, WCH = C_::WCH;
  // [X stage 0 | X stage 1 | X stage 2 | W stage 0 | W stage 1], 32 KB each
  __shared__ __attribute__((aligned(1024))) char lds[(X_STAGES + W_STAGES) * STAGE];
  typedef __attribute__((address_space(3))) void lds_void;

  // WA = 3 also reads the wave index into a scalar, so wave-uniform values (the LDS DMA destinations in M0,
  // panel offsets) stay on the scalar unit (the two-step instantiations keep their per-lane form)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = WA == 3 ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;

  // ---- work of this workgroup: a range of K steps over the tile sequence. Data-parallel: one whole tile.
  //      Stream-K (sk_iters > 0): sk_iters steps starting at (cta * sk_iters), crossing tile boundaries;
  //      cta ids are made contiguous per XCD so one XCD's workgroups walk neighbouring tiles. ----
  const int tiles_n = (p.N + TN - 1) / TN, tiles_m = (p.M + BM - 1) / BM;
  const int total = tiles_n * tiles_m;
  const int nk = p.K / BK;
  int cta = blockIdx.x, it, it_end;
  if constexpr (SK) {
    cta = (cta % 8) * (gridDim.x / 8) + cta / 8;  // host: gridDim.x % 8 == 0
    it = cta * p.sk_iters;
    it_end = min(it + p.sk_iters, total * nk);
  } else {
    if (total % 8 == 0) cta = (cta % 8) * (total / 8) + cta / 8;
    it = cta * nk;
    it_end = it + nk;
  }
  // tile index -> (m0, n0): walked in groups of GROUP_M tile rows so neighbouring tiles share panels in L2
  const int group_sz = GROUP_M * tiles_n;
  int m0 = 0, n0 = 0, kb = 0;  // current tile and its first K step
  auto set_tile = [&](int tile) {
    const int first_m = (tile / group_sz) * GROUP_M;
    const int gm = min(GROUP_M, tiles_m - first_m);
    const int in_g = tile % group_sz;
    m0 = (first_m + in_g % gm) * BM;
    n0 = (in_g / gm) * TN;
  };

  // ---- X tile (activations) -> LDS directly: instruction r of wave w fills 1 KB block b = WAVES r + w,
  //      i.e. rows 8 WAVES r + 8w + lane/8; lane slot lane & 7 receives logical chunk (lane & 7) ^ swz(row)
  //      (swz of those rows does not depend on r) ----
  const int xrow0 = wave * 8 + (lane >> 3);
  const int xchunk = ((lane & 7) ^ swz(xrow0)) * 8;
  int xoff[X_LOADS];
  int cy[CONV ? X_LOADS : 1], cx[CONV ? X_LOADS : 1];  // CONV: output pixel (row, column) of each load's row
  int sub_py = 0, sub_px = 0;                            // CONV sub-pixel: the tile's phase
  const uint16_t* xbase = (const uint16_t*)p.A;
  auto issue_x_to = [&](int t, int stage) {
    char* dst = lds + stage * STAGE + wave * 1024;
    if constexpr (CONV) {
      // k = (tap, channel) of this lane's 8 columns (C % 8 == 0: never across two taps); taps outside the
      // image and k >= 9 C read the zero chunk
      const uint32_t k = (uint32_t)((kb + t) * BK + xchunk);
      const int tap = (int)__umulhi(k, p.cv_cinv), ci = (int)k - tap * p.cv_C;
      int dy, dx, ntap;
      if (p.cv_sub) {  // 2 x 2 taps at low-res offsets (r + py - 1, s + px - 1)
        dy = (tap >> 1) + sub_py - 1, dx = (tap & 1) + sub_px - 1, ntap = 4;
      } else {
        const int ty = (tap * 11) >> 5;  // tap / 3 for tap < 12
        dy = ty - 1, dx = tap - 3 * ty - 1, ntap = 9;
      }
      const int win = p.cv_up ? p.cv_W >> 1 : p.cv_W;
#pragma unroll
      for (int r = 0; r < X_LOADS; r++) {
        int sy = cy[r] + dy, sx = cx[r] + dx;
        const bool in = tap < ntap && sy >= 0 && sy < p.cv_H && sx >= 0 && sx < p.cv_W;
        sy >>= p.cv_up;
        sx >>= p.cv_up;
        const void* src = in ? (const void*)(xbase + ((size_t)sy * win + sx) * p.lda + ci) : (const void*)g_zero_chunk;
        __builtin_amdgcn_global_load_lds(src, (lds_void*)(dst + r * WAVES * 1024), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int r = 0; r < X_LOADS; r++)
        __builtin_amdgcn_global_load_lds((const void*)(xbase + xoff[r] + (kb + t) * BK),
                                         (lds_void*)(dst + r * WAVES * 1024), 16, 0, 0);
    }
  };

  // ---- W tile: wave w loads k-rows [KR w, KR w + KR), lane columns n0 + 4 wl .. + 3. With TN = 192, lanes
  //      48..63 repeat lanes 32..47, with TN = 128 lanes 32..63 repeat 0..31 (same loads, same LDS writes of
  //      the same values) ----
  const int wl = (TN == 256 || lane < TN / 4) ? lane : lane - (64 - TN / 4);
  constexpr int WB = (WF == WF_16) ? 2 : 1;
  int wcol = 0;  // columns >= N (last tile) are loaded clamped and never stored
  const char* wbase = nullptr;
  const size_t wrow = (size_t)p.ldw * WB;
  auto set_operands = [&]() {
#pragma unroll
    for (int r = 0; r < X_LOADS; r++) {
      const int m = min(m0 + 8 * WAVES * r + xrow0, p.M - 1);
      if constexpr (CONV) {
        cy[r] = m / p.cv_W;
        cx[r] = m - cy[r] * p.cv_W;
      } else {
        xoff[r] = m * p.lda + xchunk;
      }
    }
    if constexpr (CONV) {
      if (p.cv_sub) {
        const int ph = n0 / p.cv_np;  // a tile lies in one phase (TN divides cv_np)
        sub_py = ph >> 1, sub_px = ph & 1;
      }
    }
    wcol = min(n0 + wl * 4, p.N - 4);
    // packed: 8-row panels of 8 ldw bytes, column group c / 4 at 32 (c / 4) = 8 c within the panel
    wbase = (const char*)p.W + ((size_t)(wave * KR) * p.ldw + (PK ? 8 : 1) * wcol) * WB;
  };
  // untracked loads (see vm_load_b32): their waits are the explicit vmcnt of step() / the prologue
  auto issue_w = [&](int t, WRaw<WF, KR>& R) {
    const char* src = wbase + (size_t)((kb + t) * BK) * wrow;
    if constexpr (PK) {
#pragma unroll
      for (int i = 0; i < KR / 8; i++) {  // panel i: rows 8 i .. 8 i + 7 of this thread, 32 contiguous bytes
        R.v[2 * i] = vm_load_b128(src + (size_t)i * 8 * wrow);
        R.v[2 * i + 1] = vm_load_b128(src + (size_t)i * 8 * wrow + 16);
      }
    } else
#pragma unroll
    for (int i = 0; i < KR; i++) {
      if constexpr (WF == WF_16)
        R.r[i] = vm_load_b64(src + i * wrow);
      else
        R.r[i] = vm_load_b32(src + i * wrow);
    }
    if constexpr (is_group(WF)) {
      const size_t g = (size_t)((kb + t) >> p.gshift) * p.ldw + wcol;
      if constexpr (WF == WF_I8_GROUP) {
#pragma unroll
        for (int j = 0; j < 4; j++) R.s[j] = vm_load_b32((const float*)p.S + g + j);
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) R.s[j] = vm_load_u16((const uint16_t*)p.S + g + j);
      }
    }
  };
  // raw(t) has landed: everything but the newest `newer` untracked / DMA loads is complete
  auto ready_w = [&](WRaw<WF, KR>& R, auto newer_c) {
    constexpr int NEWER = decltype(newer_c)::value;
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NEWER));
    if constexpr (PK) {
#pragma unroll
      for (int i = 0; i < KR / 4; i++) vm_ready(R.v[i]);
    } else {
#pragma unroll
      for (int i = 0; i < KR; i++) vm_ready(R.r[i]);
    }
    if constexpr (is_group(WF)) {
#pragma unroll
      for (int j = 0; j < 4; j++) vm_ready(R.s[j]);
    }
  };
  constexpr int H = KR / 8;  // k-chunks (8 rows) per column and thread
  int woff[WCH];  // LDS byte offsets of this thread's converted chunks (column j, half h) in a W stage
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int h = 0; h < H; h++) {
      const int nl = wl * 4 + j;
      woff[j * H + h] = nl * 128 + (((H * wave + h) ^ swz(nl)) * 16);
    }
  auto store_w = [&](const WRaw<WF, KR>& R, int stage, int q) {  // quarter q of the thread's chunks
    char* base = lds + (X_STAGES + stage) * STAGE;
#pragma unroll
    for (int c = q * WCH / 4; c < (q + 1) * WCH / 4; c++)
      *(u32x4*)(base + woff[c]) = convert_chunk<ACT, WF, KR>(R, c / H, c % H);
  };

  // ---- MFMA operands: wave (wn, wm) owns n [WN wn, +WN) x m [WME wm, +WME) = JB x IB blocks of 32 x 32 ----
  const int wn = wave & 1, wm = wave >> 1;
  const int l32 = lane & 31, khalf = lane >> 5;
  const int w_rd = (wn * WN + l32) * 128, x_rd = (wm * C_::WME + l32) * 128;
  int sw[4];
#pragma unroll
  for (int s = 0; s < 4; s++) sw[s] = (((2 * s + khalf) ^ swz(l32)) * 16);

  f32x16 acc[JB][IB];

  auto read_frags = [&](const char* xs, const char* ws, int s, u32x4 (&wf)[JB], u32x4 (&xf)[IB]) {
#pragma unroll
    for (int jb = 0; jb < JB; jb++) wf[jb] = *(const u32x4*)(ws + w_rd + jb * 32 * 128 + sw[s]);
#pragma unroll
    for (int ib = 0; ib < IB; ib++) xf[ib] = *(const u32x4*)(xs + x_rd + ib * 32 * 128 + sw[s]);
  };

  int ns = 0;  // K steps of the current segment
  constexpr int LOADS = (PK ? X_LOADS + KR / 4 : C_::LOADS) + (is_group(WF) ? 4 : 0);
  using NewerT = std::integral_constant<int, LOADS>;

  // One K step: multiply stage t; convert raw(t + 1) into the other W stage between the MFMAs; the loads
  // of step t + 2 (activations straight into LDS, weights into Rl) are in flight meanwhile. Every step is
  // the same code: past the last step the loads re-fetch step nk - 1 into buffers nobody reads (stage
  // (t + 2) % 3 and the W stage of t + 1 are never the stage being multiplied), so the loop has no branches.
  auto step = [&](int t, WRaw<WF, KR>& Rc, WRaw<WF, KR>& Rl) {
    const int tl = min(t + 2, ns - 1);
    issue_x_to(tl, (t + 2) % X_STAGES);
    issue_w(tl, Rl);
    // step t + 1's loads (issued one step ago: its activations into LDS and raw(t + 1) = Rc) have landed
    ready_w(Rc, NewerT{});
    const char* xs = lds + (t % X_STAGES) * STAGE;
    const char* ws = lds + (X_STAGES + (t & 1)) * STAGE;
    u32x4 wf[2][JB], xf[2][IB];
    read_frags(xs, ws, 0, wf[0], xf[0]);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      // Scheduling regions: the next slice's fragment reads are issued first and may not sink past the
      // region end, so they have a whole slice of MFMAs (this wave's and the other wave's on the SIMD) to
      // land; left alone, the scheduler places them ~4 MFMAs before use and then waits for them.
      if (s < 3) read_frags(xs, ws, s + 1, wf[(s + 1) & 1], xf[(s + 1) & 1]);
      SCHED_FENCE();
#pragma unroll
      for (int jb = 0; jb < JB; jb++)
#pragma unroll
        for (int ib = 0; ib < IB; ib++) acc[jb][ib] = mfma32<ACT>(wf[s & 1][jb], xf[s & 1][ib], acc[jb][ib]);
      store_w(Rc, (t + 1) & 1, s);
      SCHED_FENCE();
    }
    lds_barrier();  // this step's converted weights and (waited above) step t + 1's activations are visible
  };

  // WA = 3: multiply stage t; convert raw(t + 1) (Rc, retired at the end of step t - 1) into the other W stage;
  // issue the activations of step t + 2 and the weights of step t + 3 (into Rl); at the end wait for what step
  // t - 1 issued (activations of t + 1, weights of t + 2 in Rn) and tie Rn to that wait.
  auto step3 = [&](int t, WRaw<WF, KR>& Rc, WRaw<WF, KR>& Rn, WRaw<WF, KR>& Rl) {
    issue_x_to(min(t + 2, ns - 1), (t + 2) % X_STAGES);
    issue_w(min(t + 3, ns - 1), Rl);
    const char* xs = lds + (t % X_STAGES) * STAGE;
    const char* ws = lds + (X_STAGES + (t & 1)) * STAGE;
    u32x4 wf[2][JB], xf[2][IB];
    read_frags(xs, ws, 0, wf[0], xf[0]);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if (s < 3) read_frags(xs, ws, s + 1, wf[(s + 1) & 1], xf[(s + 1) & 1]);
      SCHED_FENCE();
#pragma unroll
      for (int jb = 0; jb < JB; jb++)
#pragma unroll
        for (int ib = 0; ib < IB; ib++) acc[jb][ib] = mfma32<ACT>(wf[s & 1][jb], xf[s & 1][ib], acc[jb][ib]);
      store_w(Rc, (t + 1) & 1, s);
      SCHED_FENCE();
    }
    ready_w(Rn, NewerT{});  // step t - 1's group has landed: activations of t + 1 in LDS, weights of t + 2
    lds_barrier();
  };

  bool first_seg = true;
  if (it < it_end) for (;;) {  // segments; uniform: every thread walks the same ones (one when !SK)
  const int tile = it / nk;
  kb = it - tile * nk;
  ns = min(nk - kb, it_end - it);
  set_tile(tile);
  set_operands();
  if (SK && !first_seg) {
    // the previous segment's epilogue stores and LDS reads are done before the pipeline restarts
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
  }
  first_seg = false;
#pragma unroll
  for (int jb = 0; jb < JB; jb++)
#pragma unroll
    for (int ib = 0; ib < IB; ib++) acc[jb][ib] = (f32x16){};

  if constexpr (WA == 2) {
  WRaw<WF, KR> R0, R1;
  issue_x_to(0, 0);
  issue_w(0, R0);
  issue_x_to(min(1, ns - 1), 1);
  issue_w(min(1, ns - 1), R1);
  ready_w(R0, NewerT{});
#pragma unroll
  for (int q = 0; q < 4; q++) store_w(R0, 0, q);
  lds_barrier();
  int t = 0;
  for (; t + 1 < ns; t += 2) {
    step(t, R1, R0);
    step(t + 1, R0, R1);
  }
  if (t < ns) step(t, R1, R0);
  // The last steps' re-fetches must land before the LDS is reused below. The raw registers they target are
  // never read, so they are tied here, after the wait: otherwise the compiler would hand those registers to
  // other values while the (untracked) loads are still in flight and the loads would overwrite them.
  ready_w(R0, std::integral_constant<int, 0>{});
  ready_w(R1, std::integral_constant<int, 0>{});
  } else {
  // groups in issue order: {X(0), W(0), W(1)}, {X(1), W(2)}; the first is waited for (the second, LOADS
  // loads, may stay in flight), then step t issues {X(t + 2), W(t + 3)} and retires {X(t + 1), W(t + 2)}
  WRaw<WF, KR> R0, R1, R2;
  issue_x_to(0, 0);
  issue_w(0, R0);
  issue_w(min(1, ns - 1), R1);
  issue_x_to(min(1, ns - 1), 1);
  issue_w(min(2, ns - 1), R2);
  ready_w(R0, NewerT{});
  ready_w(R1, NewerT{});
#pragma unroll
  for (int q = 0; q < 4; q++) store_w(R0, 0, q);
  lds_barrier();
  int t = 0;
  for (; t + 2 < ns; t += 3) {
    step3(t, R1, R2, R0);
    step3(t + 1, R2, R0, R1);
    step3(t + 2, R0, R1, R2);
  }
  if (t < ns) {  // nested: the second remainder step converts R2, which only the first one's wait retires
    step3(t, R1, R2, R0);
    if (t + 1 < ns) step3(t + 1, R2, R0, R1);
  }
  ready_w(R0, std::integral_constant<int, 0>{});
  ready_w(R1, std::integral_constant<int, 0>{});
  ready_w(R2, std::integral_constant<int, 0>{});
  }
  lds_barrier();

  // ---- stream-K: a tile split over workgroups c0..c1 (K order). Each stores its partial accumulators to
  //      its workspace slot and counts itself in; the last to arrive adds all partials in c0..c1 order
  //      (deterministic whatever the arrival order) and runs the epilogue. No workgroup ever waits. ----
  if constexpr (SK) if (ns != nk) {
    const int c0 = (tile * nk) / p.sk_iters, c1 = (tile * nk + nk - 1) / p.sk_iters;
    // a workgroup has at most two split tiles: slot 2c for its first tile, 2c + 1 for its last
    auto slot = [&](int c) {
      return p.ws + (size_t)(2 * c + (tile == (c * p.sk_iters) / nk ? 0 : 1)) * (BM * BN) + tid * 4;
    };
    // Partials and counts are exchanged device-coherently per access (sc1: through to memory, past both cache
    // levels, as the agent-scope atomics of the memory model are), with no whole-cache write-back or
    // invalidate: the workgroups of one tile may sit on different XCDs, whose L2s are not coherent.
    {
      float* mine = slot(cta);
#pragma unroll
      for (int jb = 0; jb < 4; jb++)
#pragma unroll
        for (int ib = 0; ib < IB; ib++)
#pragma unroll
          for (int g = 0; g < 4; g++)
            st_coherent_b128(mine + (size_t)((jb * IB + ib) * 4 + g) * (NTHR * 4),
                             (f32x4){acc[jb][ib][4 * g], acc[jb][ib][4 * g + 1], acc[jb][ib][4 * g + 2],
                                     acc[jb][ib][4 * g + 3]});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial has reached memory
    lds_barrier();                                      // ... and every thread's
    // the arrival count is broadcast through the (now idle) first LDS word; the epilogue writes there only
    // after its own barrier, which every thread reaches after reading it
    if (tid == 0)
      *(volatile int*)lds = __hip_atomic_fetch_add(p.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();
    if (*(volatile int*)lds != c1 - c0) {
      it += ns;
      if (it >= it_end) break;
      continue;  // another workgroup finishes this tile
    }
    // sum = p_c0 + p_c0+1 + ... in K order (own partial re-read like the others, so the association does
    // not depend on which workgroup arrived last); 8 quads per batch of loads
#pragma unroll
    for (int jb = 0; jb < 4; jb++)
#pragma unroll
      for (int ib = 0; ib < IB; ib++) acc[jb][ib] = (f32x16){};
    for (int c = c0; c <= c1; c++) {
      const float* src = slot(c);
#pragma unroll
      for (int jb = 0; jb < 4; jb++)
#pragma unroll
        for (int u0 = 0; u0 < IB * 4; u0 += 8) {  // 8 accumulator quads per batch of loads
          f32x4 v[8];
          ld_coherent_8x_b128(src + (size_t)(jb * IB * 4 + u0) * (NTHR * 4), NTHR * 4, v);
#pragma unroll
          for (int u = 0; u < 8; u++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[jb][(u0 + u) >> 2][4 * ((u0 + u) & 3) + e] += v[u][e];
        }
    }
    if (tid == 0) __hip_atomic_store(p.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
  }

  // ---- epilogue. The LDS is free after the last barrier: the block's 256 column scales and vec entries
  //      are staged as f32, then the finished values are staged row-major and written out (or, for the
  //      residual epilogues, read-modify-written) with 16-byte vectors covering whole rows of the tile.
  //      Per (jb, ib) the lane holds row m = WME wm + 32 ib + l32 and columns
  //      n = WN wn + 32 jb + 8 g + 4 khalf + e (g, e = 0..3) of the tile in acc[jb][ib][4 g + e]. ----
  constexpr bool OUT16 = (EPI == KH_EPI_STORE16 || EPI == KH_EPI_GELU || EPI == KH_EPI_BIAS16 || EPI == KH_EPI_SWIGLU ||
                          EPI == EPI_QKNR);
  constexpr bool HAS_VEC = (EPI == KH_EPI_RESID_GATE || EPI == KH_EPI_BIAS16 || EPI == KH_EPI_BIAS_F32);
  constexpr int OUT_COLS = (EPI == KH_EPI_SWIGLU) ? TN / 2 : TN;
  constexpr int ELEM = OUT16 ? 2 : 4;
  constexpr int ROW_BYTES = OUT_COLS * ELEM + 16;             // padded staging row
  constexpr int PASS_ROWS = OUT16 ? BM : BM / 2;              // f32 tiles go out in two row halves
  constexpr int SC_OFF = PASS_ROWS * ROW_BYTES;
  static_assert(SC_OFF + 2 * TN * 4 <= (X_STAGES + W_STAGES) * STAGE, "epilogue staging exceeds LDS");
  float* sc_l = (float*)(lds + SC_OFF);
  float* vv_l = sc_l + TN;
  if (tid < TN) {
    const int n = n0 + tid;
    float sv = 1.f, vv = 0.f;
    if (n < p.N) {
      if (WF == WF_I8_CHANNEL) sv = load_scale(p.S, p.s_dtype, n);
      if (HAS_VEC) vv = p.vec[n];
    }
    sc_l[tid] = sv;
    vv_l[tid] = vv;
  }
  lds_barrier();

  if constexpr (EPI == EPI_QKNR) {
    static_assert(TN == 256, "one head per wave");
    // (1) the scaled accumulator rounded to 16 bits: exactly the projection output a separate qk_norm_rope
    //     pass would read (engine/src/model.mm:373-375: EPI_BF16 then qk_norm_rope)
#pragma unroll
    for (int jb = 0; jb < JB; jb++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const f32x4 sc = *(const f32x4*)(sc_l + wn * WN + jb * 32 + g * 8 + khalf * 4);
#pragma unroll
        for (int ib = 0; ib < IB; ib++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            // the f32 product is rounded to 16 bits as in the STORE16 epilogue (the barrier keeps the compiler
            // from fusing multiply and conversion into one mixed-precision FMA, which rounds once)
            float v = acc[jb][ib][g * 4 + e] * sc[e];
            asm volatile("" : "+v"(v));
            acc[jb][ib][g * 4 + e] = from16<ACT>(to16<ACT>(v));
          }
      }
    // (2) q / k heads (engine/kernels/norm.metal:81-134): the wave's 128 columns are one head; this lane holds
    //     64 of a row's channels (c = 32 jb + 8 g + 4 khalf + e), lane ^ 32 the other 64
    const int hc = n0 + wn * WN;
    const bool is_q = hc >= p.qk_qoff && hc < p.qk_qoff + 128 * p.qk_nq;
    const bool is_k = hc >= p.qk_koff && hc < p.qk_koff + 128 * p.qk_nk;
    if (is_q || is_k) {  // wave-uniform
      const float* wv = is_q ? p.qk_wq : p.qk_wk;
      const int head = is_q ? (hc - p.qk_qoff) >> 7 : (hc - p.qk_koff) >> 7;
#pragma unroll
      for (int ib = 0; ib < IB; ib++) {
        const int row = m0 + wm * C_::WME + ib * 32 + l32, rr = min(row, p.M - 1);
        float ss = 0.f;
#pragma unroll
        for (int jb = 0; jb < JB; jb++)
#pragma unroll
          for (int i = 0; i < 16; i++) ss += acc[jb][ib][i] * acc[jb][ib][i];
        ss += __shfl_xor(ss, 32);
        const float rrms = rsqrtf(ss * (1.0f / 128.0f) + p.qk_eps);
#pragma unroll
        for (int jb = 0; jb < JB; jb++)
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const f32x4 w4 = *(const f32x4*)(wv + jb * 32 + g * 8 + khalf * 4);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[jb][ib][g * 4 + e] *= rrms * w4[e];
          }
        const float* cr = p.qk_cos + (size_t)rr * 64;
        const float* sr = p.qk_sin + (size_t)rr * 64;
        if (p.qk_mode == 0) {  // channels (2i, 2i + 1) rotate by frequency i: e = (0, 1), (2, 3)
#pragma unroll
          for (int jb = 0; jb < JB; jb++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
              const int i0 = (jb * 32 + g * 8 + khalf * 4) >> 1;
              const float2 c2 = *(const float2*)(cr + i0), s2 = *(const float2*)(sr + i0);
#pragma unroll
              for (int q2 = 0; q2 < 2; q2++) {
                const float c = q2 ? c2.y : c2.x, sn = q2 ? s2.y : s2.x;
                const float x0 = acc[jb][ib][g * 4 + 2 * q2], x1 = acc[jb][ib][g * 4 + 2 * q2 + 1];
                acc[jb][ib][g * 4 + 2 * q2] = x0 * c - x1 * sn;
                acc[jb][ib][g * 4 + 2 * q2 + 1] = x0 * sn + x1 * c;
              }
            }
        } else if (p.qk_mode == 1) {  // channel i < 64 rotates with i + 64 (block jb + 2), frequency i
#pragma unroll
          for (int jb = 0; jb < 2; jb++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
              const int f = jb * 32 + g * 8 + khalf * 4;
              const f32x4 c4 = *(const f32x4*)(cr + f), s4 = *(const f32x4*)(sr + f);
#pragma unroll
              for (int e = 0; e < 4; e++) {
                const float a = acc[jb][ib][g * 4 + e], b = acc[jb + 2][ib][g * 4 + e];
                acc[jb][ib][g * 4 + e] = a * c4[e] - b * s4[e];
                acc[jb + 2][ib][g * 4 + e] = b * c4[e] + a * s4[e];
              }
            }
        }
        if (p.qk_big >= 0) {  // the big channel leaves the 16-bit tensor for the f32 side buffer
          const int bd = p.qk_big, bjb = bd >> 5, bg = (bd >> 3) & 3, bkh = (bd >> 2) & 1, be = bd & 3;
#pragma unroll
          for (int jb = 0; jb < JB; jb++)
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
              for (int e = 0; e < 4; e++)
                if (jb == bjb && g == bg && e == be && khalf == bkh) {
                  if (row < p.M) {
                    if (is_q) p.qk_qbig[(size_t)row * p.qk_nq + head] = acc[jb][ib][g * 4 + e];
                    else p.qk_kbig[(size_t)row * p.qk_nk + head] = acc[jb][ib][g * 4 + e];
                  }
                  acc[jb][ib][g * 4 + e] = 0.f;
                }
        }
      }
    }
  }

  const int out_n0 = (EPI == KH_EPI_SWIGLU) ? n0 / 2 : n0;
  const int out_N = (EPI == KH_EPI_SWIGLU) ? p.N / 2 : p.N;
  // copy-out geometry: 16-byte chunks, CPR per staged row, consecutive threads along a row
  constexpr int CPR = OUT_COLS * ELEM / 16;
  constexpr int CHUNKS = PASS_ROWS * CPR;
  // WA = 3, residual epilogues: every residual chunk this thread will update in a pass is loaded before the
  // pass stages its tile, so the loads' latency overlaps the staging instead of following it four chunks at
  // a time (the same values are added in the same order: results are bitwise equal)
  constexpr bool RPF = WA == 3 && (EPI == KH_EPI_RESID || EPI == KH_EPI_RESID_GATE) && !CONV;
  constexpr int RPF_N = RPF ? (CHUNKS + NTHR - 1) / NTHR : 1;
  f32x4 xpre[RPF_N];
#pragma unroll
  for (int pass = 0; pass < BM / PASS_ROWS; pass++) {
    if constexpr (RPF) {
      const int grow0 = m0 + pass * PASS_ROWS;
#pragma unroll
      for (int i = 0; i < RPF_N; i++) {
        const int idx = tid + i * NTHR;
        const int r = idx / CPR, c = idx % CPR;
        const int gm_ = grow0 + r, gcol = out_n0 + c * (16 / ELEM);
        if (idx < CHUNKS && gm_ < p.M && gcol < out_N)
          xpre[i] = *(const f32x4*)((const char*)p.C + ((size_t)gm_ * p.ldc + gcol) * ELEM);
      }
    }
    if (PASS_ROWS == BM || (wm * C_::WME) / PASS_ROWS == pass) {
      const int row_base = wm * C_::WME - pass * PASS_ROWS;
#pragma unroll
      for (int jb = 0; jb < JB; jb++) {
        if (EPI == KH_EPI_SWIGLU && (jb & 1)) continue;  // up blocks are consumed with their gate block
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int nl = wn * WN + jb * 32 + g * 8 + khalf * 4;  // tile column of e = 0
          const f32x4 sc = *(const f32x4*)(sc_l + nl);
          f32x4 sc_up = sc, vv = {};
          if (EPI == KH_EPI_SWIGLU) sc_up = *(const f32x4*)(sc_l + nl + 32);
          if (HAS_VEC) vv = *(const f32x4*)(vv_l + nl);
          const int ol = (EPI == KH_EPI_SWIGLU) ? (nl / 64) * 32 + (nl % 32) : nl;  // staged column
#pragma unroll
          for (int ib = 0; ib < IB; ib++) {
            char* dst = lds + (row_base + ib * 32 + l32) * ROW_BYTES + ol * ELEM;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const float v = EPI == EPI_QKNR ? acc[jb][ib][g * 4 + e] : acc[jb][ib][g * 4 + e] * sc[e];
              if (EPI == KH_EPI_SWIGLU) o[e] = silu_fast(v) * (acc[jb + 1][ib][g * 4 + e] * sc_up[e]);
              else if (EPI == KH_EPI_GELU) o[e] = gelu_fast(v);
              else if (EPI == KH_EPI_BIAS16 || EPI == KH_EPI_BIAS_F32) o[e] = v + vv[e];
              else if (EPI == KH_EPI_RESID_GATE) o[e] = v * vv[e];
              else o[e] = v;
            }
            if constexpr (OUT16)
              *(u32x2*)dst = (u32x2){pack16<ACT>(o[0], o[1]),
                                     pack16<ACT>(o[2], o[3])};
            else
              *(f32x4*)dst = (f32x4){o[0], o[1], o[2], o[3]};
          }
        }
      }
    }
    lds_barrier();
    const int grow0 = m0 + pass * PASS_ROWS;
    if constexpr (RPF) {
#pragma unroll
      for (int i = 0; i < RPF_N; i++) {
        const int idx = tid + i * NTHR;
        const int r = idx / CPR, c = idx % CPR;
        const int gm_ = grow0 + r, gcol = out_n0 + c * (16 / ELEM);
        if (idx >= CHUNKS || gm_ >= p.M || gcol >= out_N) continue;
        const f32x4 v = *(const f32x4*)(lds + r * ROW_BYTES + c * 16);
        *(f32x4*)((char*)p.C + ((size_t)gm_ * p.ldc + gcol) * ELEM) = xpre[i] + v;
      }
    } else
#pragma unroll 4
    for (int idx = tid; idx < CHUNKS; idx += NTHR) {
      const int r = idx / CPR, c = idx % CPR;
      const int gm_ = grow0 + r, gcol = out_n0 + c * (16 / ELEM);
      if (gm_ >= p.M || gcol >= out_N) continue;
      const u32x4 v = *(const u32x4*)(lds + r * ROW_BYTES + c * 16);
      size_t orow = (size_t)gm_;
      int ocol = gcol;
      if constexpr (CONV) {
        if (p.cv_sub) {  // low-res pixel (i, j) of phase (py, px) -> output pixel (2 i + py, 2 j + px)
          const int i = (int)__umulhi((uint32_t)gm_, p.cv_winv), j = gm_ - i * p.cv_W;
          orow = (size_t)(2 * i + sub_py) * (2 * p.cv_W) + 2 * j + sub_px;
          ocol = gcol - (2 * sub_py + sub_px) * p.cv_np;
        }
      }
      char* gp = (char*)p.C + (orow * p.ldc + ocol) * ELEM;
      if constexpr (EPI == KH_EPI_RESID || EPI == KH_EPI_RESID_GATE) {
        f32x4 x = *(const f32x4*)gp;
        x += __builtin_bit_cast(f32x4, v);
        *(f32x4*)gp = x;
      } else if (EPI == KH_EPI_BIAS16 && p.R) {
        const u32x4 r = *(const u32x4*)((const uint16_t*)p.R + orow * p.ldr + ocol);
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 4; h++)
          o[h] = pack16<ACT>(from16<ACT>((uint16_t)v[h]) + from16<ACT>((uint16_t)r[h]),
                             from16<ACT>((uint16_t)(v[h] >> 16)) + from16<ACT>((uint16_t)(r[h] >> 16)));
        *(u32x4*)gp = o;
      } else {
        *(u32x4*)gp = v;
      }
    }
    if (pass + 1 < BM / PASS_ROWS) lds_barrier();
  }
  if constexpr (!SK) break;
  it += ns;
  if (it >= it_end) break;
  }  // segments
}

template <int ACT, int WF, int E, int TN, bool CONV>
void launch_dp(const GemmArgs& a, const dim3& grid, const dim3& block, hipStream_t st) {
  if constexpr (!CONV && has_wa3(ACT, WF, TN)) {
    if (a.wa == 3) {
      hipLaunchKernelGGL((gemm_kernel<ACT, WF, E, WAVES_DEFAULT, false, TN, CONV, 3>), grid, block, 0, st, a);
      return;
    }
  }
  hipLaunchKernelGGL((gemm_kernel<ACT, WF, E, WAVES_DEFAULT, false, TN, CONV>), grid, block, 0, st, a);
}

template <int ACT, int WF, int E, bool CONV = false>
void launch_one(const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  const dim3 grid(grid_x), block(64 * WAVES_DEFAULT);
  if (a.sk_iters > 0) {
    hipLaunchKernelGGL((gemm_kernel<ACT, WF, E, WAVES_DEFAULT, true, BN, CONV>), grid, block, 0, st, a);
    return;
  }
  if constexpr (!wide_only(E)) {
    if (tn == 192) {
      launch_dp<ACT, WF, E, 192, CONV>(a, grid, block, st);
      return;
    }
    if constexpr (WF == WF_16) {  // 128-wide tiles: 16-bit weights only (the VAE's narrow channel counts)
      if (tn == 128) {
        launch_dp<ACT, WF, E, 128, CONV>(a, grid, block, st);
        return;
      }
    }
  }
  launch_dp<ACT, WF, E, BN, CONV>(a, grid, block, st);
}

template <int ACT, int WF>
hipError_t launch_epi(int epi, const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  switch (epi) {
    case KH_EPI_STORE16: launch_one<ACT, WF, KH_EPI_STORE16>(a, grid_x, tn, st); break;
    case KH_EPI_F32: launch_one<ACT, WF, KH_EPI_F32>(a, grid_x, tn, st); break;
    case KH_EPI_RESID_GATE: launch_one<ACT, WF, KH_EPI_RESID_GATE>(a, grid_x, tn, st); break;
    case KH_EPI_RESID: launch_one<ACT, WF, KH_EPI_RESID>(a, grid_x, tn, st); break;
    case KH_EPI_SWIGLU: launch_one<ACT, WF, KH_EPI_SWIGLU>(a, grid_x, tn, st); break;
    case KH_EPI_GELU: launch_one<ACT, WF, KH_EPI_GELU>(a, grid_x, tn, st); break;
    case KH_EPI_BIAS16: launch_one<ACT, WF, KH_EPI_BIAS16>(a, grid_x, tn, st); break;
    case KH_EPI_BIAS_F32: launch_one<ACT, WF, KH_EPI_BIAS_F32>(a, grid_x, tn, st); break;
    case EPI_QKNR: launch_one<ACT, WF, EPI_QKNR>(a, grid_x, tn, st); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int ACT>
hipError_t launch_wf(int wf, int epi, const GemmArgs& a, int g, int tn, hipStream_t st) {
  if (wf == WF_16) return launch_epi<ACT, WF_16>(epi, a, g, tn, st);
  if (wf == WF_I8_CHANNEL) return launch_epi<ACT, WF_I8_CHANNEL>(epi, a, g, tn, st);
  if (wf == (WF_I8_CHANNEL | WF_PK)) return launch_epi<ACT, WF_I8_CHANNEL | WF_PK>(epi, a, g, tn, st);
  if (wf == (WF_I8_GROUP | WF_PK)) return launch_epi<ACT, WF_I8_GROUP | WF_PK>(epi, a, g, tn, st);
  if (wf == WF_I8_GROUP) return launch_epi<ACT, WF_I8_GROUP>(epi, a, g, tn, st);
  if (wf == WF_I8_GROUP_F16) return launch_epi<ACT, WF_I8_GROUP_F16>(epi, a, g, tn, st);
  return launch_epi<ACT, WF_I8_GROUP_BF16>(epi, a, g, tn, st);
}

template <int ACT>
hipError_t launch_conv(const GemmArgs& a, int grid_x, int tn, hipStream_t st) {
  launch_one<ACT, WF_16, KH_EPI_BIAS16, true>(a, grid_x, tn, st);
  return hipGetLastError();
}

}  // namespace

}  // namespace kh
