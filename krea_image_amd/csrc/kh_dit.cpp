// Host-side DiT block orchestration on one HIP stream: engine/src/model.mm:369-385 (DiT::layer) and
// engine/src/model.mm:519-525 (DiT::run_layers), with the adaLN modulation (Conditioning::compute +
// DiT::make_cond, engine/src/model.mm:317-347 and 571-591) moved onto the GPU as a GEMV + make_cond.
// Everything is enqueued asynchronously; nothing allocates (the GEMMs' stream-K workspace is state->gemm_ws).
#include <cmath>

#include "kh_internal.h"

namespace kh {

namespace {

size_t elem_size(int dtype) { return dtype == KH_F32 ? 4 : dtype == KH_I8 ? 1 : 2; }

int check_cfg(const kh_dit_config& c, Err& e) {
  if (c.dim <= 0 || c.dim % 128 || c.heads * 128 != c.dim) return e.fail("dit: dim must be heads * 128");
  if (c.kv_heads <= 0 || c.heads % c.kv_heads) return e.fail("dit: heads %% kv_heads != 0");
  if (c.ff <= 0 || c.ff % 64) return e.fail("dit: ff must be a multiple of 64");
  if (c.mlp != 0 && c.mlp != 1) return e.fail("dit: mlp must be 0 (GELU) or 1 (SwiGLU)");
  if (c.dtype != KH_F16 && c.dtype != KH_BF16) return e.fail("dit: dtype must be f16 or bf16");
  return KH_OK;
}

}  // namespace

int dit_layer_forward(hipStream_t st, const kh_dit_config& c, const kh_dit_layer& L, const kh_dit_state& s, int R,
                      Err& e) {
  int rc = check_cfg(c, e);
  if (rc) return rc;
  if (R <= 0) return e.fail("dit: rows must be > 0");
  if (!s.x || !s.h || !s.qkv || !s.ao || !s.mid || !s.mods) return e.fail("dit: missing state buffer");
  const int D = c.dim, kvD = c.kv_heads * 128;
  const int nqkv = D + 2 * kvD + (c.attn_gate ? D : 0);
  const int nup = c.mlp == 1 ? 2 * c.ff : c.ff;
  const size_t es = elem_size(c.dtype);
  char* qkv = (char*)s.qkv;
  const GemmWs ws{s.gemm_ws, s.gemm_ws_bytes};

  // adaLN: tvec = SiLU(cond) W_ada + b; mods = make_cond(tvec, table, n1, n2)
  if (L.ada.w) {
    if (!s.cond || !s.tvec) return e.fail("dit: adaLN needs state->cond and state->tvec");
    if ((rc = gemv(st, s.cond, L.ada, s.tvec, 1, 6 * D, s.cond_dim, 6 * D, 1, L.ada_bias, e))) return rc;
    if ((rc = make_cond(st, s.tvec, L.mod_table, L.n1, L.n2, D, s.mods, e))) return rc;
  } else if (L.mod_table) {
    // the reference's layout: one tvec per step (Conditioning::compute, model.mm:571-591) shared by all
    // layers, each adding its own table (DiT::make_cond, model.mm:317-347)
    if (!s.tvec) return e.fail("dit: mod_table needs state->tvec");
    if ((rc = make_cond(st, s.tvec, L.mod_table, L.n1, L.n2, D, s.mods, e))) return rc;
  }
  const float* m = s.mods;
  // attention half
  if ((rc = rms_norm(st, s.x, m, m + D, s.h, c.dtype, R, D, D, D, c.eps, c.norm_center, e))) return rc;
  // QKV projection, then the per-head q / k RMSNorm + RoPE as its own HBM-bound pass (model.mm:373-375). The
  // fused form (gemm_qk_norm_rope) measured slower at 4608 rows: 304 us against 264 + 25 us, because the GEMM
  // epilogue runs with the MFMAs idle and its per-row table loads are latency-bound there.
  if ((rc = gemm(st, KH_EPI_STORE16, s.h, c.dtype, L.qkv, s.qkv, R, nqkv, D, D, nqkv, nqkv, nullptr, e, &ws))) return rc;
  if ((rc = qk_norm_rope(st, s.qkv, c.dtype, L.qn, L.kn, s.cosb, s.sinb, R, nqkv, 0, c.heads, D, c.kv_heads, c.eps,
                         c.rope_mode, L.big_dim, s.qbig, s.kbig, e)))
    return rc;
  const bool big = L.big_dim >= 0;
  if ((rc = attention(st, qkv, qkv + D * es, qkv + (D + kvD) * es, s.ao, c.dtype, R, R, c.heads, nqkv, nqkv, nqkv, D,
                      c.heads / c.kv_heads, 0, 0, c.attn_gate ? qkv + (D + 2 * kvD) * es : nullptr,
                      c.attn_gate ? nqkv : 0, big ? s.qbig : nullptr, big ? s.kbig : nullptr, e)))
    return rc;
  if ((rc = gemm(st, KH_EPI_RESID_GATE, s.ao, c.dtype, L.o, s.x, R, D, D, D, D, D, m + 2 * D, e, &ws))) return rc;
  // MLP half
  if ((rc = rms_norm(st, s.x, m + 3 * D, m + 4 * D, s.h, c.dtype, R, D, D, D, c.eps, c.norm_center, e))) return rc;
  if ((rc = gemm(st, c.mlp == 1 ? KH_EPI_SWIGLU : KH_EPI_GELU, s.h, c.dtype, L.up, s.mid, R, nup, D, D, nup, c.ff,
                 nullptr, e, &ws)))
    return rc;
  return gemm(st, KH_EPI_RESID_GATE, s.mid, c.dtype, L.down, s.x, R, D, c.ff, c.ff, D, D, m + 5 * D, e, &ws);
}

int dit_forward(hipStream_t st, const kh_dit_config& c, const kh_dit_layer* layers, int n, const kh_dit_state& s,
                int R, Err& e) {
  if (n < 0 || (n > 0 && !layers)) return e.fail("dit: bad layer list");
  for (int l = 0; l < n; l++) {
    const int rc = dit_layer_forward(st, c, layers[l], s, R, e);
    if (rc) return rc;
  }
  return KH_OK;
}

// krea_sigmas (engine/src/model.mm:594-602)
int sigmas(int steps, float mu, float* out) {
  if (steps <= 0 || !out) return KH_EINVAL;
  const double e = std::exp((double)mu);
  for (int i = 0; i <= steps; i++) {
    const double t = 1.0 - (double)i / steps;
    out[i] = t <= 0 ? 0.0f : (float)(e / (e + (1.0 / t - 1.0)));
  }
  return KH_OK;
}

// RoPE tables of DiT::set_grid: engine/src/model.mm:290-315 (mode 0) and the 2-D variant of the benchmark
// configs (mode 1)
int rope_tables(int T, int H, int W, int mode, float* cosb, float* sinb) {
  if (T < 0 || H < 0 || W < 0 || (mode != 0 && mode != 1) || !cosb || !sinb) return KH_EINVAL;
  double om[64];
  for (int p = 0; p < 64; p++) {
    if (mode == 0) {
      const int ax = p < 16 ? 0 : p < 40 ? 1 : 2, k = p - (ax == 0 ? 0 : ax == 1 ? 16 : 40), d = ax == 0 ? 32 : 48;
      om[p] = 1.0 / std::pow(1000.0, (2.0 * k) / d);
    } else {
      om[p] = 1.0 / std::pow(10000.0, (2.0 * (p % 32)) / 64.0);
    }
  }
  const long R = (long)T + (long)H * W;
  for (long r = 0; r < R; r++) {
    const long k = r - T;
    const double pi = r < T ? 0.0 : (double)(k / W), pj = r < T ? 0.0 : (double)(k % W);
    for (int p = 0; p < 64; p++) {
      const double a = (mode == 0 ? (p < 16 ? 0.0 : p < 40 ? pi : pj) : (p < 32 ? pi : pj)) * om[p];
      cosb[r * 64 + p] = (float)std::cos(a);
      sinb[r * 64 + p] = (float)std::sin(a);
    }
  }
  return KH_OK;
}

}  // namespace kh
