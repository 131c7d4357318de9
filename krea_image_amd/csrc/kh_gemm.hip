// Dequant-GEMM host side: argument checks, launch planning (tile width, stream-K) and dispatch to the kernel
// instantiations (kh_gemm_f16.hip / kh_gemm_bf16.hip; the kernel design is described in kh_gemm_kernel.h).
#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "kh_common.h"
#include "kh_gemm_args.h"
#include "kh_internal.h"

namespace kh {

namespace {

using namespace gemm_detail;

// ---- stream-K workspace: caller-owned device memory (kh_gemm_ws / the DiT and VAE workspaces), never allocated
//      here. Layout: 2 partial-tile slots of BM x BN f32 per workgroup of one wave, then SK_MAX_TILES arrival
//      counters (zero between launches: the finishing workgroup of a tile resets its counter). Launches that
//      share one workspace must be ordered (one stream). ----
constexpr int SK_MAX_TILES = 4096;  // stream-K runs only below 60 % of two waves: < 1.2 x CUs tiles
constexpr int SK_MIN_ITERS = 4;     // below this many K steps per workgroup the partial traffic dominates

std::mutex sk_mu;
std::map<int, int> sk_ctas;  // device -> workgroups of one full wave (one per CU), a multiple of 8

// KH_GEMM_STREAMK=0 keeps every launch data-parallel (read per call, so a host can switch it at run time)
bool sk_enabled() {
  const char* e = getenv("KH_GEMM_STREAMK");
  return !(e && e[0] == '0');
}

// workgroups for a stream-K launch on `dev` (0: unavailable)
int sk_cta_count(int dev) {
  std::lock_guard<std::mutex> lk(sk_mu);
  auto it = sk_ctas.find(dev);
  if (it != sk_ctas.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
  const int c = cus - cus % 8;
  sk_ctas[dev] = c;
  return c;
}

size_t sk_part_bytes(int ctas) { return (size_t)2 * ctas * BM * BN * sizeof(float); }

// KH_GEMM_WAHEAD=3 loads weights three K steps ahead in the instantiations that have that form (has_wa3);
// unset or 2: two steps (read per call)
int wa_choice() {
  const char* e = getenv("KH_GEMM_WAHEAD");
  return e && e[0] == '3' && e[1] == 0 ? 3 : 2;
}

// KH_GEMM_TN192=0 keeps every data-parallel launch on 256-wide tiles (read per call)
bool narrow_enabled() {
  const char* e = getenv("KH_GEMM_TN192");
  return !(e && e[0] == '0');
}

// Tile width and launch. The width is the one that pads N least (ties to the wider: 256, then 192, then
// 128, which only 16-bit-weight GEMMs have: narrow128). With 256-wide tiles the launch is data-parallel
// (one tile per workgroup) unless the tiles fill the last wave of workgroups poorly; then stream-K spreads
// the tiles' K steps evenly over one wave of workgroups. Narrow tiles are data-parallel, unless they fill
// under 60 % of their last wave and 256-wide stream-K needs less work per CU (padded width x tiles / CUs
// against waves x width).
// tn_div > 0: the tile width must divide tn_div (sub-pixel convs: a tile may not straddle two phases).
// ctas: workgroups of one full wave on the device (one per CU, a multiple of 8; 0 if unknown).
void plan_launch_for(GemmArgs& a, int epi, const GemmWs* ws, int ctas, int& grid_x, int& tn, bool narrow128,
                     int tn_div) {
  const int tiles_m = (a.M + BM - 1) / BM;
  const int nk = a.K / BK;
  auto padded = [&](int w) { return (a.N + w - 1) / w * w; };
  tn = BN;
  if (tn_div > 0) {
    tn = tn_div % BN == 0 ? BN : tn_div % 192 == 0 ? 192 : 128;
  } else if (!wide_only(epi) && narrow_enabled()) {
    if (padded(192) < padded(tn)) tn = 192;
    if (narrow128 && padded(128) < padded(tn)) tn = 128;
    if (tn != BN && ctas > 0 && sk_enabled()) {
      const int t = (a.N + tn - 1) / tn * tiles_m, r = (t + ctas - 1) / ctas;
      const double sk_cost = (double)padded(BN) / BN * tiles_m * BN / ctas;
      if ((double)t / ((double)r * ctas) < 0.6 && sk_cost < (double)r * tn) tn = BN;
    }
  }
  const int tiles = ((a.N + tn - 1) / tn) * tiles_m;
  grid_x = tiles;
  a.sk_iters = 0;
  a.ws = nullptr;
  a.cnt = nullptr;
  if (tn != BN || ctas <= 0) return;
  const int rounds = (tiles + ctas - 1) / ctas;
  // Stream-K staggers the workgroups' K offsets, so neighbouring tiles no longer share X / W panels in L2
  // at the same time: measured, it loses to data-parallel launches that fill >= 75 % of their last wave
  // (4608 x 3072 x 3072: 140 vs 103 us) and wins where most CUs would idle (1536 x 3072 x 12288: 156 vs
  // 303 us). It is used below 60 % occupancy.
  if (sk_enabled() && tiles <= SK_MAX_TILES && (double)tiles / ((double)rounds * ctas) < 0.6) {
    const long long iters = (long long)tiles * nk;
    const int per = (int)((iters + ctas - 1) / ctas);
    if (per >= SK_MIN_ITERS && ws && ws->p && ws->bytes >= gemm_workspace_bytes_for(ctas)) {
      a.sk_iters = per;
      a.ws = (float*)ws->p;
      a.cnt = (int*)((char*)ws->p + sk_part_bytes(ctas));
      grid_x = ctas;
      return;
    }
  }
  if (tn_div > 0) return;
  // 192-wide tiles where 256-wide ones leave part of a single wave of workgroups idle and 192-wide ones still
  // fit in one wave (4096 x 3072 outputs: 256 tiles instead of 192; measured 349 -> 326 us at K = 12288).
  // Not where they add a partial wave: at 4608 x 12288 (864 vs 1152 tiles) they measured 390 -> 410 us.
  if (!wide_only(epi) && a.N % 192 == 0 && narrow_enabled() && tiles < ctas) {
    const int tiles192 = (a.N / 192) * tiles_m;
    if (tiles192 > tiles && tiles192 <= ctas) {
      tn = 192;
      grid_x = tiles192;
    }
  }
}

// plan_launch_for on the current device
void plan_launch(GemmArgs& a, int epi, const GemmWs* ws, int& grid_x, int& tn, bool narrow128 = false, int tn_div = 0) {
  int dev = 0;
  const int ctas = hipGetDevice(&dev) == hipSuccess ? sk_cta_count(dev) : 0;
  plan_launch_for(a, epi, ws, ctas, grid_x, tn, narrow128, tn_div);
}

}  // namespace

// The launch kh_gemm / kh_gemm_ws would make for this shape on a device with `ctas` CUs, without a device:
// out = {tile width, workgroups, K steps per workgroup (0: data-parallel)}.
int gemm_plan(int M, int N, int K, int epi, int w16, int ctas, int with_ws, int* out, Err& e) {
  if (epi < KH_EPI_STORE16 || epi > KH_EPI_BIAS_F32) return e.fail("gemm_plan: unknown epilogue %d", epi);
  if (M <= 0 || N <= 0 || K <= 0 || N % 64 || K % BK) return e.fail("gemm_plan: unsupported shape");
  if (ctas <= 0 || ctas % 8) return e.fail("gemm_plan: ctas=%d must be a positive multiple of 8", ctas);
  if (!out) return e.fail("gemm_plan: null out");
  GemmArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, M, N, K, K, N, N, 0, KH_F32, 0, nullptr, nullptr};
  const GemmWs ws{(void*)(uintptr_t)256, gemm_workspace_bytes_for(ctas)};  // never dereferenced
  int grid_x = 0, tn = BN;
  plan_launch_for(a, epi, with_ws ? &ws : nullptr, ctas, grid_x, tn, w16 != 0, 0);
  out[0] = tn;
  out[1] = grid_x;
  out[2] = a.sk_iters;
  return KH_OK;
}

namespace {

int gemm_run(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
             int lda, int ldw, int ldc, const void* vec, const QkNormRope* qk, const GemmWs* ws, Err& e) {
  if (epi < KH_EPI_STORE16 || epi > KH_EPI_BIAS_F32) return e.fail("gemm: unknown epilogue %d", epi);
  if (a_dtype != KH_F16 && a_dtype != KH_BF16) return e.fail("gemm: activations must be f16 or bf16");
  if (M <= 0 || N <= 0 || K <= 0) return e.fail("gemm: empty shape M=%d N=%d K=%d", M, N, K);
  if (N % 64 || K % BK) return e.fail("gemm: unsupported shape N=%d K=%d (need N %% 64 == 0, K %% 64 == 0)", N, K);
  if (!A || !W.w || !C) return e.fail("gemm: null A / W / C");
  if (lda < K || lda % 8) return e.fail("gemm: lda=%d must be >= K and a multiple of 8", lda);
  if (ldw < N) return e.fail("gemm: ldw=%d < N=%d", ldw, N);
  // the activation loader indexes A with 32-bit element offsets (row * lda + k)
  if ((long long)(M - 1) * lda + K >= (1LL << 31))
    return e.fail("gemm: A spans (M - 1) * lda + K = %lld elements, more than 2^31 - 1: split the rows",
                  (long long)(M - 1) * lda + K);
  const int out_cols = epi == KH_EPI_SWIGLU ? N / 2 : N;
  const bool out16 = epi == KH_EPI_STORE16 || epi == KH_EPI_GELU || epi == KH_EPI_BIAS16 || epi == KH_EPI_SWIGLU;
  const int ldc_mult = out16 ? 8 : 4;  // output rows are written in 16-byte vectors
  if (ldc < out_cols || ldc % ldc_mult)
    return e.fail("gemm: ldc=%d must be >= %d and a multiple of %d", ldc, out_cols, ldc_mult);
  if (((uintptr_t)C & 15) || ((uintptr_t)A & 15) || ((uintptr_t)W.w & 15))
    return e.fail("gemm: A, W and C must be 16-byte aligned");
  const bool needs_vec = epi == KH_EPI_RESID_GATE || epi == KH_EPI_BIAS16 || epi == KH_EPI_BIAS_F32;
  if (needs_vec && !vec) return e.fail("gemm: epilogue %d needs vec", epi);
  int wf;
  int group = 0;
  if (W.w_dtype == KH_I8 || W.w_dtype == KH_I8P) {
    if (!W.s) return e.fail("gemm: int8 weights need scales");
    if (W.s_dtype != KH_F32 && W.s_dtype != KH_F16 && W.s_dtype != KH_BF16) return e.fail("gemm: bad scale dtype");
    if (ldw % 16) return e.fail("gemm: int8 ldw=%d must be a multiple of 16", ldw);
    group = W.group <= 0 ? K : W.group;
    if (group >= K) {
      if (group != K) return e.fail("gemm: group %d > K %d", group, K);
      wf = WF_I8_CHANNEL;
    } else {
      if (group % BK || K % group) return e.fail("gemm: int8 group %d must divide K and be a multiple of 64", group);
      if (group & (group - 1)) return e.fail("gemm: int8 group %d must be a power of two", group);
      wf = W.s_dtype == KH_F32 ? WF_I8_GROUP : W.s_dtype == KH_F16 ? WF_I8_GROUP_F16 : WF_I8_GROUP_BF16;
    }
    if (W.w_dtype == KH_I8P) {
      if (wf != WF_I8_CHANNEL && wf != WF_I8_GROUP)
        return e.fail("gemm: packed int8 weights need per-channel scales or f32 group scales");
      wf |= WF_PK;
    }
  } else {
    if (W.w_dtype != a_dtype) return e.fail("gemm: 16-bit weights must match the activation type");
    if (ldw % 8) return e.fail("gemm: ldw=%d must be a multiple of 8", ldw);
    wf = WF_16;
  }
  int gshift = 0;  // log2(group / BK): K step t reads scale row t >> gshift
  while ((BK << gshift) < group) gshift++;
  GemmArgs a{A, W.w, W.s, C, (const float*)vec, M, N, K, lda, ldw, ldc, gshift, W.s_dtype, 0, nullptr, nullptr};
  if (qk) {
    a.qk_wq = qk->wq, a.qk_wk = qk->wk, a.qk_cos = qk->cosb, a.qk_sin = qk->sinb;
    a.qk_qbig = qk->qbig, a.qk_kbig = qk->kbig;
    a.qk_qoff = qk->q_off, a.qk_nq = qk->n_q, a.qk_koff = qk->k_off, a.qk_nk = qk->n_k;
    a.qk_mode = qk->mode, a.qk_big = qk->big_dim, a.qk_eps = qk->eps;
    epi = EPI_QKNR;
  }
  int grid_x = 0, tn = BN;
  if (ws && ws->p && ((uintptr_t)ws->p & 255)) return e.fail("gemm: workspace must be 256-byte aligned");
  plan_launch(a, epi, ws, grid_x, tn, wf == WF_16);
  a.wa = wa_choice();
  hipError_t r = a_dtype == KH_F16 ? launch_gemm_f16(wf, epi, a, grid_x, tn, st)
                                   : launch_gemm_bf16(wf, epi, a, grid_x, tn, st);
  if (r != hipSuccess) return e.hip(r, "gemm launch");
  return KH_OK;
}

}  // namespace

// ---- kh_pack_int8: thread = one (8-row panel, 4-column group): eight 4-byte row reads, one 32-byte write ----
__global__ __launch_bounds__(256) void pack_int8_kernel(const uint8_t* __restrict__ W, int ldw, long long groups,
                                                       uint8_t* __restrict__ out) {
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  const int per_panel = ldw / 4;
  const long long panel = g / per_panel;
  const int cg = (int)(g - panel * per_panel);
  const uint8_t* src = W + (size_t)panel * 8 * ldw + 4 * cg;
  u32x4 a, b;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[i] = *(const uint32_t*)(src + (size_t)i * ldw);
    b[i] = *(const uint32_t*)(src + (size_t)(i + 4) * ldw);
  }
  u32x4* dst = (u32x4*)(out + (size_t)panel * 8 * ldw + 32 * cg);
  dst[0] = a;
  dst[1] = b;
}

int pack_int8(hipStream_t st, const void* W, int K, int ldw, void* out, Err& e) {
  if (!W || !out) return e.fail("pack_int8: null W / out");
  if (K <= 0 || K % 8) return e.fail("pack_int8: K=%d must be a positive multiple of 8", K);
  if (ldw <= 0 || ldw % 16) return e.fail("pack_int8: ldw=%d must be a positive multiple of 16", ldw);
  if (((uintptr_t)W | (uintptr_t)out) & 15) return e.fail("pack_int8: W and out must be 16-byte aligned");
  const size_t bytes = (size_t)K * ldw;
  const uintptr_t w0 = (uintptr_t)W, o0 = (uintptr_t)out;
  if (w0 < o0 + bytes && o0 < w0 + bytes) return e.fail("pack_int8: out overlaps W");
  const long long groups = (long long)(K / 8) * (ldw / 4);
  hipLaunchKernelGGL(pack_int8_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, (const uint8_t*)W, ldw,
                     groups, (uint8_t*)out);
  const hipError_t r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "pack_int8 launch");
}

int gemm(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
         int lda, int ldw, int ldc, const void* vec, Err& e, const GemmWs* ws) {
  return gemm_run(st, epi, A, a_dtype, W, C, M, N, K, lda, ldw, ldc, vec, nullptr, ws, e);
}

size_t gemm_workspace_bytes_for(int ctas) { return ctas > 0 ? sk_part_bytes(ctas) + SK_MAX_TILES * sizeof(int) : 0; }

size_t gemm_workspace_bytes() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  return gemm_workspace_bytes_for(sk_cta_count(dev));
}

__global__ void zero_words_kernel(int* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

int gemm_workspace_init(hipStream_t st, void* ws, size_t bytes, Err& e) {
  int dev = 0;
  hipError_t r = hipGetDevice(&dev);
  if (r != hipSuccess) return e.hip(r, "gemm_workspace_init: no device");
  const int ctas = sk_cta_count(dev);
  const size_t need = gemm_workspace_bytes_for(ctas);
  if (!ws || bytes < need) return e.fail("gemm_workspace_init: workspace %zu bytes < %zu needed", bytes, need);
  if ((uintptr_t)ws & 255) return e.fail("gemm_workspace_init: workspace must be 256-byte aligned");
  // a kernel, not hipMemsetAsync, so the call can sit in a captured graph
  hipLaunchKernelGGL(zero_words_kernel, dim3((SK_MAX_TILES + 255) / 256), dim3(256), 0, st,
                     (int*)((char*)ws + sk_part_bytes(ctas)), SK_MAX_TILES);
  r = hipGetLastError();
  return r == hipSuccess ? KH_OK : e.hip(r, "gemm_workspace_init launch");
}

// ---- kh_gemm_static: kh_gemm_ws on a file-scope device array instead of a caller workspace, for callers that
//      cannot allocate. The array holds the stream-K workspace of one wave of up to STATIC_CTAS workgroups. ----
constexpr int STATIC_CTAS = 256;  // MI355X: 256 CUs
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)2 * STATIC_CTAS * BM * BN * sizeof(float) + SK_MAX_TILES * sizeof(int);
static __device__ __align__(256) unsigned char scratch[STATIC_SCRATCH_BYTES];

namespace {
std::mutex scratch_mu;
std::map<int, void*> scratch_ptr;  // device -> that device's copy of `scratch` (hipGetSymbolAddress)
}  // namespace

size_t gemm_static_scratch_bytes() { return STATIC_SCRATCH_BYTES; }

int gemm_static(hipStream_t st, int epi, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
                int lda, int ldw, int ldc, const void* vec, Err& e) {
  int dev = 0;
  hipError_t r = hipGetDevice(&dev);
  if (r != hipSuccess) return e.hip(r, "gemm_static: no device");
  const size_t need = gemm_workspace_bytes_for(sk_cta_count(dev));
  // a device whose stream-K workspace is larger than the array (more than STATIC_CTAS CUs) runs every shape
  // data-parallel, as kh_gemm_ws does with a NULL or short workspace
  if (need > STATIC_SCRATCH_BYTES) return gemm(st, epi, A, a_dtype, W, C, M, N, K, lda, ldw, ldc, vec, e, nullptr);
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lk(scratch_mu);
    auto it = scratch_ptr.find(dev);
    if (it != scratch_ptr.end()) {
      ptr = it->second;
    } else {
      // first call on this device (it is current): the device address of its copy of the array; the host-side
      // name `scratch` is not a device address and is never passed to a kernel
      r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (r != hipSuccess) return e.hip(r, "gemm_static: hipGetSymbolAddress(scratch)");
      // The counters start at zero: the array is zero-initialised when the code object loads, and every launch
      // leaves them zero. Outside graph capture they are cleared once more and the stream is waited on, so
      // that a first call on another stream cannot overtake the clear. Under capture neither is possible
      // (the fill would be replayed; a wait is illegal) and the load-time zeros stand.
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      r = hipStreamIsCapturing(st, &cs);
      if (r != hipSuccess) return e.hip(r, "gemm_static: hipStreamIsCapturing");
      if (cs == hipStreamCaptureStatusNone) {
        const int rc = gemm_workspace_init(st, ptr, need, e);
        if (rc) return rc;
        r = hipStreamSynchronize(st);
        if (r != hipSuccess) return e.hip(r, "gemm_static: clearing the scratch counters");
      }
      scratch_ptr[dev] = ptr;
    }
  }
  const GemmWs ws{ptr, need};
  return gemm(st, epi, A, a_dtype, W, C, M, N, K, lda, ldw, ldc, vec, e, &ws);
}

int gemm_qk_norm_rope(hipStream_t st, const void* A, int a_dtype, const kh_weight& W, void* C, int M, int N, int K,
                      int lda, int ldw, int ldc, const QkNormRope& q, Err& e, const GemmWs* ws) {
  if (q.mode < 0 || q.mode > 2) return e.fail("gemm_qk_norm_rope: bad rope mode %d", q.mode);
  if (q.mode != 2 && (!q.cosb || !q.sinb)) return e.fail("gemm_qk_norm_rope: rope needs cos / sin tables");
  if (q.n_q < 0 || q.n_k < 0 || q.n_q + q.n_k == 0) return e.fail("gemm_qk_norm_rope: no q / k heads");
  if ((q.n_q && !q.wq) || (q.n_k && !q.wk)) return e.fail("gemm_qk_norm_rope: null norm weight");
  if (q.q_off < 0 || q.k_off < 0 || q.q_off % 128 || q.k_off % 128)
    return e.fail("gemm_qk_norm_rope: head offsets must be multiples of 128 (q %d, k %d)", q.q_off, q.k_off);
  if (q.q_off + 128 * q.n_q > N || q.k_off + 128 * q.n_k > N)
    return e.fail("gemm_qk_norm_rope: heads extend past N = %d", N);
  if (q.big_dim >= 128 || (q.big_dim >= 0 && (!q.qbig || !q.kbig)))
    return e.fail("gemm_qk_norm_rope: big_dim needs qbig / kbig");
  if (((uintptr_t)q.wq | (uintptr_t)q.wk | (uintptr_t)q.cosb | (uintptr_t)q.sinb) & 15)
    return e.fail("gemm_qk_norm_rope: norm weights and tables must be 16-byte aligned");
  return gemm_run(st, KH_EPI_STORE16, A, a_dtype, W, C, M, N, K, lda, ldw, ldc, nullptr, &q, ws, e);
}

}  // namespace kh

namespace kh {

int conv3x3(hipStream_t st, const void* x, int ldx, int C, int H, int W, int up, int dtype, const kh_weight& Wt, int K,
            int N, const float* bias, const void* res, void* y, int ldy, Err& e, const GemmWs* ws) {
  if (dtype != KH_F16 && dtype != KH_BF16) return e.fail("conv3x3: dtype must be f16 or bf16");
  if (!x || !Wt.w || !y || !bias) return e.fail("conv3x3: null x / W / bias / y");
  if (Wt.w_dtype != dtype) return e.fail("conv3x3: weights must be 16-bit of the activation type");
  if (H <= 0 || W <= 0 || C <= 0 || N <= 0) return e.fail("conv3x3: empty shape H=%d W=%d C=%d N=%d", H, W, C, N);
  if (C % 8) return e.fail("conv3x3: C=%d must be a multiple of 8", C);
  if (ldx < C || ldx % 8) return e.fail("conv3x3: ldx=%d must be >= C and a multiple of 8", ldx);
  if (up && (H % 2 || W % 2)) return e.fail("conv3x3: upsampling needs an even output size (%d x %d)", H, W);
  if (K % BK || K < 9 * C) return e.fail("conv3x3: K=%d must be a multiple of 64 and >= 9 C = %d", K, 9 * C);
  if (N % 64) return e.fail("conv3x3: N=%d must be a multiple of 64", N);
  if (ldy < N || ldy % 8) return e.fail("conv3x3: ldy=%d must be >= N and a multiple of 8", ldy);
  if ((long long)H * W >= (1LL << 31)) return e.fail("conv3x3: too many pixels");
  if (((uintptr_t)x | (uintptr_t)Wt.w | (uintptr_t)y | (uintptr_t)res) & 15)
    return e.fail("conv3x3: x, W, res and y must be 16-byte aligned");
  GemmArgs a{x, Wt.w, nullptr, y, bias, H * W, N, K, ldx, N, ldy, 0, KH_F32, 0, nullptr, nullptr,
             C, H, W, up ? 1 : 0, (uint32_t)((((uint64_t)1 << 32) + (uint64_t)C - 1) / (uint64_t)C), res, ldy};
  int grid_x = 0, tn = BN;
  if (ws && ws->p && ((uintptr_t)ws->p & 255)) return e.fail("conv3x3: workspace must be 256-byte aligned");
  plan_launch(a, KH_EPI_BIAS16, ws, grid_x, tn, true);
  const hipError_t r = dtype == KH_F16 ? launch_conv_f16(a, grid_x, tn, st) : launch_conv_bf16(a, grid_x, tn, st);
  if (r != hipSuccess) return e.hip(r, "conv3x3 launch");
  return KH_OK;
}

}  // namespace kh


namespace kh {

int conv_up2_subpix(hipStream_t st, const void* x, int ldx, int C, int H, int W, int dtype, const kh_weight& W2, int K,
                    int Np, const float* bias4, void* y, int ldy, Err& e, const GemmWs* ws) {
  if (dtype != KH_F16 && dtype != KH_BF16) return e.fail("conv_up2: dtype must be f16 or bf16");
  if (!x || !W2.w || !y || !bias4) return e.fail("conv_up2: null x / W2 / bias / y");
  if (W2.w_dtype != dtype) return e.fail("conv_up2: weights must be 16-bit of the activation type");
  if (H <= 0 || W <= 0 || C <= 0 || Np <= 0) return e.fail("conv_up2: empty shape H=%d W=%d C=%d Np=%d", H, W, C, Np);
  if (C % 8) return e.fail("conv_up2: C=%d must be a multiple of 8", C);
  if (ldx < C || ldx % 8) return e.fail("conv_up2: ldx=%d must be >= C and a multiple of 8", ldx);
  if (K % BK || K < 4 * C) return e.fail("conv_up2: K=%d must be a multiple of 64 and >= 4 C = %d", K, 4 * C);
  if (Np % 128 && Np % 192) return e.fail("conv_up2: Np=%d must be a multiple of 128 or 192", Np);
  if (ldy < Np || ldy % 8) return e.fail("conv_up2: ldy=%d must be >= Np and a multiple of 8", ldy);
  if (4LL * H * W >= (1LL << 31) || W >= (1 << 16)) return e.fail("conv_up2: image too large");
  if (((uintptr_t)x | (uintptr_t)W2.w | (uintptr_t)y) & 15) return e.fail("conv_up2: x, W2 and y must be 16-byte aligned");
  GemmArgs a{x, W2.w, nullptr, y, bias4, H * W, 4 * Np, K, ldx, 4 * Np, ldy, 0, KH_F32, 0, nullptr, nullptr,
             C, H, W, 0, (uint32_t)((((uint64_t)1 << 32) + (uint64_t)C - 1) / (uint64_t)C), nullptr, 0};
  a.cv_sub = 1;
  a.cv_np = Np;
  a.cv_winv = (uint32_t)((((uint64_t)1 << 32) + (uint64_t)W - 1) / (uint64_t)W);
  int grid_x = 0, tn = BN;
  if (ws && ws->p && ((uintptr_t)ws->p & 255)) return e.fail("conv_up2: workspace must be 256-byte aligned");
  plan_launch(a, KH_EPI_BIAS16, ws, grid_x, tn, true, Np);
  const hipError_t r = dtype == KH_F16 ? launch_conv_f16(a, grid_x, tn, st) : launch_conv_bf16(a, grid_x, tn, st);
  if (r != hipSuccess) return e.hip(r, "conv_up2 launch");
  return KH_OK;
}

}  // namespace kh
