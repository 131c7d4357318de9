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
 * Ops are asynchronous on `stream` (a hipStream_t; NULL = the null stream). Ops never allocate device memory:
 * what an op needs beyond its inputs and outputs comes from the caller (workspace arguments), as the
 * reference's ops take buffers owned by the model (engine/src/model.mm:251-267).
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
enum { KH_F32 = 0, KH_F16 = 1, KH_BF16 = 2, KH_I8 = 3, KH_I8P = 4 /* int8 in kh_pack_int8's layout */ };

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
 *   w_dtype KH_I8P: int8 as KH_I8 (per-channel scales, or group scales in f32), rearranged by kh_pack_int8;
 *       same results as KH_I8, bitwise. kh_gemm and kh_gemm_qk_norm_rope only (not kh_gemv).
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
 * elements of the output type. Constraints: M > 0, N % 64 == 0, K % 64 == 0, int8 group a power of two
 * >= 64 dividing K, 16-byte aligned A / W rows (lda % 8 == 0, ldw % 16 == 0 for int8, % 8 for 16-bit).
 * kh_gemm launches are data-parallel (one output tile per workgroup); kh_gemm_ws below adds stream-K for shapes
 * that would leave CUs idle. Data-parallel launches may use
 * narrower tiles (not for SWIGLU): 256 x 192 where N pads less to 192 than to 256 (e.g. 384) or where
 * 256-wide tiles fill only part of one wave of workgroups and 192-wide ones still fit in one (4096 x 3072);
 * 256 x 128 for 16-bit weights where N pads less to 128 (e.g. 64, 128). KH_GEMM_TN192=0 keeps 256-wide
 * tiles. Every tile width sums each output's products in the same order: the results are bitwise equal.
 * KH_GEMM_WAHEAD=3 loads packed per-channel int8 weights three K steps ahead instead of two (data-parallel
 * launches; bitwise the same results).
 * Replaces krea::Metal::gemm (engine/src/metal.h:66-69, engine/src/metal.mm:146-163). */
int kh_gemm(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N, int K,
            int lda, int ldw, int ldc, const void* vec, char* err, int errlen);

/* kh_gemm with a stream-K workspace: shapes whose 256 x 256 tiles would fill under 60 % of a wave of workgroups
 * (e.g. 1536 x 12288 outputs on 256 CUs) spread the tiles' K steps over one workgroup per CU; a workgroup that
 * covers part of a tile stores its f32 partial in the workspace and the last to arrive adds the partials in K
 * order (deterministic). workspace: device memory of >= kh_gemm_workspace_bytes() bytes (2 x CUs x 256 KiB of
 * partial slots + 16 KiB of arrival counters), 256-byte aligned, prepared once by kh_gemm_workspace_init (it
 * zeroes the counters; every launch leaves them zero again). Launches that share a workspace must be ordered
 * (one stream). A NULL or smaller workspace, or KH_GEMM_STREAMK=0 in the environment, gives the data-parallel
 * launch of kh_gemm. Stream-K and data-parallel launches of one GEMM agree to fp32 rounding (the K sum is split
 * differently). The workspace is the caller-owned arena the reference's model keeps for its ops
 * (engine/src/model.mm:251-267, engine/src/metal.mm:146-163). */
int kh_gemm_ws(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N, int K,
               int lda, int ldw, int ldc, const void* vec, void* workspace, size_t workspace_bytes, char* err,
               int errlen);
/* Workspace size kh_gemm_ws uses on the current device (0 if no device). */
size_t kh_gemm_workspace_bytes(void);
/* The launch kh_gemm (with_ws 0) or kh_gemm_ws with a full workspace (with_ws 1) makes for an M x N x K GEMM on a
 * device with `ctas` CUs (a positive multiple of 8), computed on the host without a device: out[0] = tile width
 * (256, 192, or 128 for 16-bit weights, w16 = 1), out[1] = workgroups, out[2] = K steps per workgroup (0: one
 * tile per workgroup, data-parallel; > 0: stream-K). No counterpart in the reference, whose Metal::gemm grid is
 * fixed (engine/src/metal.mm:146-163); for tests and for schedulers that size work per launch. */
int kh_gemm_plan(int M, int N, int K, int epi, int w16, int ctas, int with_ws, int* out, char* err, int errlen);
/* Prepares a kh_gemm_ws workspace (a fill kernel on `stream`, so it may be captured in a graph). */
int kh_gemm_workspace_init(kh_stream stream, void* workspace, size_t workspace_bytes, char* err, int errlen);

/* kh_gemm_ws without a workspace argument and without any allocation: the stream-K workspace is a file-scope
 * device array of the library (128 MiB + 16 KiB: one wave of up to 256 workgroups, what MI355X's 256 CUs use),
 * which every GPU the library runs on holds until the process ends, whether or not this entry point is called.
 * No counterpart in the reference; for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops). Same arguments and results as kh_gemm_ws with a workspace (bitwise). A device whose
 * stream-K workspace would exceed the array (more than 256 CUs) runs every shape data-parallel, as kh_gemm_ws
 * does with a short workspace. The first call on a device, outside graph capture, clears the array's counters on
 * `stream` and waits for that stream. All calls on one GPU share its array: calls that may overlap in time on one
 * GPU (other streams, other threads) race, so order them on one stream. */
int kh_gemm_static(kh_stream stream, int epi, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N,
                   int K, int lda, int ldw, int ldc, const void* vec, char* err, int errlen);

/* Load-time rearrangement of int8 weights Wt[K, ldw] (row stride ldw bytes) into the packed layout kh_gemm reads
 * as w_dtype KH_I8P: element (k, n) at byte (k / 8) 8 ldw + 32 (n / 4) + 4 (k % 8) + n % 4, i.e. 8-row panels in
 * which each 4-column group's 8 x 4 bytes are contiguous. A GEMM thread loads one such group per K step (two
 * 16-byte loads instead of eight 4-byte row loads; the bytes it receives are the same). Column views keep
 * working: columns [c0, c0 + N) with c0 % 4 == 0 start at byte 8 c0 of the packed buffer, with the same ldw.
 * K % 8 == 0, ldw % 16 == 0; out holds K ldw bytes and must not overlap W. No counterpart in the reference
 * (its Metal kernels read the input-major layout of tools/convert.py directly). */
int kh_pack_int8(kh_stream stream, const void* W, int K, int ldw, void* out, char* err, int errlen);

/* Flash attention, head dim 128: O[q, h] = softmax_k(Q[q,h] . K[k, h/group] / sqrt(128) (+ QB[q,h] KB[k,h/group]))
 * V[k, h/group] (* sigmoid(G[q, h]) if G), fp32 scores / softmax / accumulation, P rounded to the 16-bit type
 * before P V. Q [Lq, ldq], K [Lk, ldk], V [Lk, ldv], O [Lq, ldo], G [Lq, ldg] (dtype KH_F16 / KH_BF16), head h at
 * column 128 h (kv head at 128 (h / group)). causal: key k visible to query i iff k <= i + q_pos0. QB [Lq, heads]
 * and KB [Lk, heads / group] (f32, both or neither): the rank-1 score term of a "big" head dimension.
 * Workgroups of 8 x 32 queries (4 x 32 with the rank-1 term; KH_ATTN_WAVES=4 / 8 overrides); either size
 * computes the same per-query arithmetic. KH_ATTN_ADDR=1 selects the kernel's scalar-address form (bitwise the
 * same results; used when ldk, ldv <= 2^24).
 * Replaces krea::Metal::attention (engine/src/metal.h:86-88, engine/src/metal.mm:193-202). */
int kh_attention(kh_stream stream, const void* Q, const void* K, const void* V, void* O, int dtype, int Lq, int Lk,
                 int heads, int ldq, int ldk, int ldv, int ldo, int group, int causal, int q_pos0, const void* G,
                 int ldg, const float* QB, const float* KB, char* err, int errlen);

/* Row norm with modulation: y = (x - mu) * rsqrt(mean((x - mu)^2) + eps) * mul (+ add), mu = 0 (center = 0,
 * RMSNorm as in the reference) or the row mean (center = 1, LayerNorm of the benchmark configs); x f32
 * [rows, ld_in], width % 4 == 0, width <= 8192, y in out_dtype (KH_F32 / KH_F16 / KH_BF16).
 * Replaces krea::Metal::rms_norm (engine/src/metal.h:72-74, engine/kernels/norm.metal:28-55). */
int kh_rms_norm(kh_stream stream, const float* x, const float* mul, const float* add, void* y, int out_dtype, int rows,
                int width, int ld_in, int ld_out, float eps, int center, char* err, int errlen);

/* Per-head RMSNorm (f32 weights [128]) + RoPE in place on a 16-bit fused projection buffer [rows, ld]: n_q heads
 * at column q_off, n_k heads at k_off. rope_mode 0: interleaved pairs (2i, 2i+1), 1: rotate-half (i, i+64),
 * 2: none; cos / sin f32 [rows, 64]. big_dim >= 0: that dimension goes to qbig [rows, n_q] / kbig [rows, n_k]
 * (f32) and is zeroed. Replaces krea::Metal::qk_norm_rope (engine/src/metal.h:77-79, norm.metal:81-134). */
int kh_qk_norm_rope(kh_stream stream, void* qkv, int dtype, const float* wq, const float* wk, const float* cosb,
                    const float* sinb, int rows, int ld, int q_off, int n_q, int k_off, int n_k, float eps,
                    int rope_mode, int big_dim, float* qbig, float* kbig, char* err, int errlen);

/* kh_gemm (epilogue STORE16, C 16-bit [M, ldc]) followed by kh_qk_norm_rope on its output rows, fused: the
 * norm and RoPE run in the GEMM epilogue on the 16-bit-rounded projection values (the values the separate
 * pass reads), so the q / k heads never make a round trip through HBM. Arguments as for the two calls, with
 * the projection output C in place of qkv (rows = M, ld = ldc); q_off and k_off multiples of 128; norm
 * weights and tables 16-byte aligned. The per-head sum of squares is added in a different order than the
 * separate pass (results agree to rounding). workspace / workspace_bytes: as for kh_gemm_ws (NULL: data-parallel).
 * Replaces the pair Metal::gemm(Epi::BF16) + Metal::qk_norm_rope of
 * DiT::layer (engine/src/model.mm:373-375). */
int kh_gemm_qk_norm_rope(kh_stream stream, const void* A, int a_dtype, const kh_weight* W, void* C, int M, int N,
                         int K, int lda, int ldw, int ldc, const float* wq, const float* wk, const float* cosb,
                         const float* sinb, int q_off, int n_q, int k_off, int n_k, float eps, int rope_mode,
                         int big_dim, float* qbig, float* kbig, void* workspace, size_t workspace_bytes, char* err,
                         int errlen);

/* adaLN / conditioning GEMV: y[r, n] = (y[r, n] if act & 2) + bias[n] + sum_k act1(x[r, k]) W~[k, n] (bias may be
 * NULL); act & 1 = SiLU on load, act & 4 = GELU(tanh) on load (exclusive); rows 1..4, x [rows, K] / y [rows, N]
 * f32; W as in kh_gemm (int8 per-channel or group, or 16-bit) or f32 (w_dtype KH_F32). N a multiple of 16 (int8),
 * 8 (16-bit) or 4 (f32); weight rows 16-byte aligned. Each output is summed in a fixed order (no atomics): the
 * same inputs give the same bits on every run.
 * Replaces the gemv_bf16 kernel (engine/kernels/gemm.metal:346-371) and the CPU cblas_sgemv of
 * Conditioning::compute (engine/src/model.mm:571-591). */
int kh_gemv(kh_stream stream, const float* x, const kh_weight* W, float* y, int rows, int N, int K, int ldw, int act,
            const float* bias, char* err, int errlen);

/* Modulation vectors of one layer from the adaLN output: engine/src/model.mm:317-347 (DiT::make_cond), on the
 * device. tvec [6 D], table [6 D] or NULL, n1 / n2 [D] -> mods [6 D] = [n1 (1+v0), v1, v2, n2 (1+v3), v4, v5]. */
int kh_make_cond(kh_stream stream, const float* tvec, const float* table, const float* n1, const float* n2, int D,
                 float* mods, char* err, int errlen);

/* Final-norm vectors of the head from the step's t: fin[k] = nf[k] (1 + t[k] + lin[k]), fin[D + k] = t[k] + lin[D + k]
 * (t [D], lin = last.mod [2 D], nf = last.n [D], fin [2 D], all f32). The fin half of DiT::make_cond
 * (engine/src/model.mm:340-346). */
int kh_make_fin(kh_stream stream, const float* t, const float* lin, const float* nf, int D, float* fin, char* err,
                int errlen);

/* fp32 GEMM (patch embed / final projection): C = A[M,K] x W[K,N] with mode bit 0 + bias[N], bit 1 GELU(tanh),
 * bit 2 accumulate into C; every output summed over K in order by one thread (results repeat bit for bit).
 * Replaces krea::Metal::gemm_f32 (engine/src/metal.h:70-71, f32gemm.metal). */
int kh_gemm_f32(kh_stream stream, const float* A, const float* W, float* C, int M, int N, int K, int lda, int ldw,
                int ldc, int mode, const float* bias, char* err, int errlen);

/* RoPE tables on the HOST: cos / sin [T + H*W, 64] f32 for T text rows at the origin and an H x W image grid.
 * mode 0: the reference's 3 axes (theta 1000, pairs 16 / 24 / 24; DiT::set_grid, engine/src/model.mm:290-315);
 * mode 1: 2-D, theta 10000, pairs [0, 32) by row and [32, 64) by column (benchmark configs). */
int kh_rope_tables(int T, int H, int W, int mode, float* cosb, float* sinb);

/* ---- the sampler around the DiT forward (engine/src/pipeline.mm:300-316) ---- */

/* Flow-matching noise levels on the HOST: out[i] = e / (e + (1/t - 1)), e = exp(mu), t = 1 - i / steps, for
 * i = 0 .. steps (out holds steps + 1 floats; out[steps] = 0), computed in double, stored as float.
 * Replaces krea_sigmas (engine/src/model.mm:594-602; the reference's default mu is 1.15, model.h:215). */
int kh_sigmas(int steps, float mu, float* out);

/* Euler step of the latent, z[i] += dt v[i] (f32, n elements, one fused multiply-add per element), dt =
 * sigma[i + 1] - sigma[i]. Replaces Metal::euler_step (engine/src/metal.mm:232-235, norm.metal:234-238). */
int kh_euler_step(kh_stream stream, float* z, const float* v, long long n, float dt, char* err, int errlen);

/* Classifier-free guidance, vc[i] = vc[i] + scale (vc[i] - vn[i]) (f32, n elements, the difference then one
 * fused multiply-add). Replaces the cfg_combine kernel (engine/kernels/norm.metal:259-262,
 * engine/src/pipeline.mm:311-314). */
int kh_cfg_combine(kh_stream stream, float* vc, const float* vn, long long n, float scale, char* err, int errlen);

/* ---- one DiT block on the device: engine/src/model.mm:369-385 (DiT::layer) ---- */
typedef struct kh_dit_config {
  int dim;         /* hidden size D */
  int heads;       /* query heads of 128 */
  int kv_heads;    /* key / value heads (GQA: heads % kv_heads == 0) */
  int ff;          /* MLP hidden units */
  int mlp;         /* 0: GELU(tanh) MLP (up N = ff); 1: SwiGLU (up N = 2 ff, gate|up 64-column tile interleave) */
  int attn_gate;   /* 1: the q|k|v projection also carries a gate block [D]; attention output *= sigmoid(gate) */
  int norm_center; /* 0: RMSNorm pre-norms (reference); 1: LayerNorm pre-norms */
  int rope_mode;   /* kh_qk_norm_rope mode */
  int dtype;       /* activation type KH_F16 / KH_BF16 */
  float eps;       /* norm epsilon (pre-norms and QK norms) */
} kh_dit_config;

typedef struct kh_dit_layer {
  kh_weight qkv;          /* [D, D + 2 kv_heads 128 (+ D gate)]: q | k | v (| gate), convert.py:189-224 layout */
  kh_weight o;            /* [D, D] */
  kh_weight up;           /* [D, ff] (GELU) or [D, 2 ff] interleaved (SwiGLU) */
  kh_weight down;         /* [ff, D] */
  kh_weight ada;          /* adaLN linear [cond_dim, 6 D] (per-layer adaLN, the benchmark configs), or w == NULL */
  const float* ada_bias;  /* [6 D] or NULL */
  const float* mod_table; /* [6 D] per-layer table added to tvec, or NULL. ada.w == NULL and mod_table != NULL:
                             mods = make_cond(state->tvec, mod_table, n1, n2) from the step's shared tvec (the
                             reference, `L{i}.mod`); both NULL: the caller fills state->mods */
  const float* n1;        /* [D] pre-attention norm weight (stored as 1 + w) */
  const float* n2;        /* [D] pre-MLP norm weight */
  const float* qn;        /* [128] q norm weight */
  const float* kn;        /* [128] k norm weight */
  int big_dim;            /* head dimension carried in fp32 (QB / KB), or -1 */
} kh_dit_layer;

typedef struct kh_dit_state { /* device buffers, owned by the caller; rows R = text + image tokens */
  float* x;           /* [R, D] f32 residual stream */
  void* h;            /* [R, D] normalised activations */
  void* qkv;          /* [R, D + 2 kvD (+ D)] */
  void* ao;           /* [R, D] attention output */
  void* mid;          /* [R, ff] MLP hidden */
  float* tvec;        /* [6 D] adaLN output */
  float* mods;        /* [6 D] modulation vectors */
  const float* cond;  /* [cond_dim] conditioning embedding (SiLU applied by the adaLN GEMV) */
  int cond_dim;
  const float* cosb;  /* [R, 64] RoPE tables */
  const float* sinb;
  float* qbig;        /* [R, heads] (layers with big_dim >= 0) */
  float* kbig;        /* [R, kv_heads] */
  void* gemm_ws;      /* kh_gemm_ws workspace for the layer's GEMMs (prepared by kh_gemm_workspace_init), or NULL */
  size_t gemm_ws_bytes;
} kh_dit_state;

/* One layer: adaLN (GEMV + make_cond) -> norm -> qkv GEMM -> QK norm + RoPE -> attention -> O GEMM with gated
 * residual -> norm -> MLP up (GELU / SwiGLU) -> down GEMM with gated residual. Asynchronous on `stream`. */
int kh_dit_layer_forward(kh_stream stream, const kh_dit_config* cfg, const kh_dit_layer* layer,
                         const kh_dit_state* state, int rows, char* err, int errlen);
/* Layers [0, n_layers) in order (engine/src/model.mm:519-525, DiT::run_layers). */
int kh_dit_forward(kh_stream stream, const kh_dit_config* cfg, const kh_dit_layer* layers, int n_layers,
                   const kh_dit_state* state, int rows, char* err, int errlen);

/* ---- packed weight files (.qw) ----
 * Format of tools/convert.py:13-17,49-89: "QWTS" | u32 version | u64 header_len | JSON header | pad | data,
 * tensors 16 KiB aligned. kh_qw_open maps and validates a file (WeightFile::WeightFile,
 * engine/src/weights.mm:16-79); kh_qw_find is WeightFile::info / get (engine/src/weights.mm:88-98); kh_qw_upload copies
 * the data region once into one resident device allocation (replaces the no-copy Metal buffers of
 * weights.mm:59-68; a discrete GPU needs the bytes in HBM). Tensor device address = base + file offset. */
#define KH_QW_MAX_DIMS 8
typedef struct kh_qw kh_qw;
typedef struct kh_qw_tensor {
  const char* name;                 /* valid until kh_qw_close */
  int dtype;                        /* KH_F32 / KH_F16 / KH_BF16 / KH_I8 */
  int ndim;
  int64_t shape[KH_QW_MAX_DIMS];
  size_t offset;                    /* from the data start */
  size_t nbytes;
  const void* host;                 /* into the read-only mapping */
  void* dev;                        /* device copy after kh_qw_upload, else NULL */
} kh_qw_tensor;
/* NULL on error (message in err). */
kh_qw* kh_qw_open(const char* path, char* err, int errlen);
void kh_qw_close(kh_qw* f);                                      /* also frees the device copy */
int kh_qw_count(const kh_qw* f);
unsigned kh_qw_version(const kh_qw* f);
const char* kh_qw_meta(const kh_qw* f);                          /* the header's "meta" object as JSON text */
int kh_qw_at(const kh_qw* f, int i, kh_qw_tensor* out);          /* i-th tensor in name order */
int kh_qw_find(const kh_qw* f, const char* name, kh_qw_tensor* out); /* KH_EINVAL if absent */
/* Synchronous: returns once the data is resident on the current device. Idempotent. */
int kh_qw_upload(kh_qw* f, kh_stream stream, char* err, int errlen);

/* Timestep conditioning of one step: t [D] and tvec [6 D] (f32, device) for noise level sigma from an uploaded
 * cond.qw (tools/convert.py:287-308). Conditioning::get (engine/src/model.mm:545-569): a sigma equal to an
 * entry of the `base.` (fast = 0) or `fast.` (fast = 1) table copies that row; fast = 1 without a match fails
 * (KH_EINVAL: the fast schedule has no computed fallback, as in the reference). Otherwise Conditioning::compute (model.mm:571-591): e = [cos | sin](
 * bf16(sigma) 1000 10000^(-i/128)), i < 128, on the host; then on the device h = tmlp1(e), t = tmlp2(gelu(h)),
 * tvec = tproj(gelu(t)) as f32 GEMVs (kh_gemv, GELU on load). work: device f32 scratch of >= 256 + D floats
 * (unused on a table hit, may be NULL then). A table hit reads only the table tensors (D from `<pre>t`), so a
 * file holding just the tables serves the sigmas they list. *from_table (may be NULL) = 1 on a table hit, else 0. Stream-ordered. */
int kh_conditioning(kh_stream stream, const kh_qw* cond, int fast, float sigma, float* t, float* tvec, float* work,
                    size_t work_bytes, int* from_table, char* err, int errlen);

/* ---- runtime surface around the ops (Metal::alloc / begin / wait, engine/src/metal.h:53-60) ---- */
int kh_stream_create(kh_stream* out, char* err, int errlen);  /* non-blocking stream, default priority */
int kh_stream_destroy(kh_stream s);
int kh_stream_sync(kh_stream s, char* err, int errlen);       /* Metal::wait */
int kh_alloc(void** out, size_t bytes, char* err, int errlen);/* hipMalloc; Metal::alloc */
int kh_free(void* p);
int kh_upload(kh_stream s, void* dst, const void* src, size_t bytes, char* err, int errlen);   /* H2D, synchronous */
int kh_download(kh_stream s, void* dst, const void* src, size_t bytes, char* err, int errlen); /* D2H, synchronous */
int kh_copy(kh_stream s, void* dst, const void* src, size_t bytes, char* err, int errlen);     /* D2D, stream-ordered */

/* ---- VAE decoder (Qwen-Image / Wan 2.1 VAE, single frame), NHWC bf16 activations [pixel, channel] ----
 * The convolutions run on the GEMM core against the converter's Wt[(ky*3+kx)*Cin + ci, co] 16-bit weights
 * (tools/convert.py:338-344); the other calls are the steps around them. */
/* y[p, n] = bias[n] + sum_k x~[p, k] Wt[k, n] (+ res[p, n]): 3x3 convolution, zero padding 1, as an implicit GEMM (the
 * activation tiles are gathered from x per (tap, channel), no im2col panel). x: NHWC [pixels, ldx] with C
 * channels, H x W output pixels (up = 1: x is H/2 x W/2, nearest-upsampled first). Wt [K, N] 16-bit of the
 * activation type (dtype KH_F16 / KH_BF16), rows >= 9 C (up to K, a multiple of 64) are multiplied by zero
 * activations; bias f32 [N]; res (NULL or 16-bit [H W, ldy], the residual, added after the biased output is
 * rounded to 16 bits, then rounded again); y [H W, ldy]. C, ldx, ldy multiples of 8, N of 64; 16-byte aligned.
 * workspace / workspace_bytes: the GEMM's stream-K workspace, as for kh_gemm_ws (NULL: data-parallel).
 * Replaces VAEDecoder::conv mode 3 (engine/src/vae.mm:112-125, kernels/vae.metal vconv3x3). */
int kh_vae_conv3x3(kh_stream stream, const void* x, int ldx, int C, int H, int W, int up, int dtype, const kh_weight* Wt,
                   int K, int N, const float* bias, const void* res, void* y, int ldy, void* workspace,
                   size_t workspace_bytes, char* err, int errlen);
/* Sub-pixel weights of a nearest-2x upsample + 3x3 conv (the reference's vae_subpix_weights,
 * engine/kernels/vae.metal:134-160, driven by engine/src/vae.mm:137-150): W [9 Cin, Cout] 16-bit (dtype) ->
 * W2 [K, 4 Np] with W2[(2r + s) Cin + ci, (2py + px) Np + co] = 16-bit round of the fp32 sum of the 3x3 taps that
 * fall on low-res offset (r + py - 1, s + px - 1); rows >= 4 Cin and columns >= Cout of each phase zero.
 * bias [Cout] f32 (or NULL) -> bias4 [4 Np] (or NULL). K >= 4 Cin, Np >= Cout. */
int kh_vae_subpix_weights(kh_stream stream, const void* W, int dtype, int Cin, int Cout, void* W2, int K, int Np,
                          const float* bias, float* bias4, char* err, int errlen);
/* y = conv3x3(nearest2x(x)) + bias as 4 sub-pixel 2x2 convs in one implicit GEMM (4/9 of the direct form's
 * multiply-adds): x NHWC [H W, ldx] with C channels (the low-res image), W2 / bias4 from
 * kh_vae_subpix_weights, y [2H x 2W pixels, ldy] with Np channels (Np a multiple of 128 or 192); workspace as for
 * kh_vae_conv3x3. Replaces
 * VAEDecoder::conv mode 2 (engine/src/vae.mm:137-150, vconv_up2). */
int kh_vae_conv_up2(kh_stream stream, const void* x, int ldx, int C, int H, int W, int dtype, const kh_weight* W2, int K,
                    int Np, const float* bias4, void* y, int ldy, void* workspace, size_t workspace_bytes, char* err,
                    int errlen);
/* 3x3 (zero padding 1) im2col of output pixels [m0, m0 + rows) of an H x W output: col[r, tap * C + ci],
 * columns [9 C, Kpad) zero; up = 1: x is H/2 x W/2 and nearest-upsampled (the vconv A loader,
 * engine/kernels/vae.metal:11-28). C, ldx, Kpad multiples of 8. */
int kh_vae_im2col(kh_stream stream, const void* x, int ldx, int C, int H, int W, int up, int m0, int rows, void* col,
                  int Kpad, char* err, int errlen);
/* y = x sqrt(C) / max(||x||, 1e-12) * gamma (+ SiLU) per pixel (vae_norm_silu, vae.metal:588-668). */
int kh_vae_norm_silu(kh_stream stream, const void* x, int ldx, const float* gamma, void* y, int ldy, int P, int C,
                     int silu, char* err, int errlen);
/* DiT latent tokens f32 [H16 W16, 64] -> VAE input bf16 [2 H16 x 2 W16, 16]: de-normalize (z std + mean) and
 * post_quant_conv (w f32 [in][out] 16 x 16, b [16]) (vae_unpack_pq, vae.metal:690-712). */
int kh_vae_unpack(kh_stream stream, const float* z, const float* mean, const float* stdv, const float* w,
                  const float* b, void* y, int H16, int W16, char* err, int errlen);
/* P[r, :n] = bf16(softmax(S[r, :n] * scale)) for rows r < rows, row stride ld (softmax_rows, vae.metal:727-757). */
int kh_vae_softmax(kh_stream stream, const float* S, int ld, int rows, int n, float scale, void* P, char* err,
                   int errlen);
/* RGBA8 = quantize(clamp(conv3x3(x, w [9 C, 4] bf16) + bias[4], -1, 1)) (vae_conv_out_rgba, vae.metal:759-785). */
int kh_vae_conv_out(kh_stream stream, const void* x, int ldx, int C, const void* w, const float* bias, void* rgba,
                    int H, int W, char* err, int errlen);
/* Device workspace kh_vae_decode needs for a H16 x W16 latent (0 for an empty one). */
size_t kh_vae_workspace_bytes(int H16, int W16);
/* Full decode (VAEDecoder::run, engine/src/vae.mm:289-337): z f32 [H16 W16, 64] -> rgba uint8 [16 H16 x 16 W16, 4]
 * on the device. Weights come from an uploaded vae.qw (kh_qw_upload), by the converter's tensor names. The
 * workspace (256-byte aligned, >= kh_vae_workspace_bytes) holds every intermediate and the GEMMs' stream-K
 * workspace; nothing is allocated. */
int kh_vae_decode(kh_stream stream, const kh_qw* vae, const float* z, int H16, int W16, void* workspace,
                  size_t workspace_bytes, void* rgba, char* err, int errlen);

/* Library identification (for the loader checks of the host bindings). */
const char* kh_version(void);

#ifdef __cplusplus
}
#endif
#endif
