// VAE decoder host loop (engine/src/vae.mm:289-337, VAEDecoder::run) over libkh ops: latent unpack ->
// conv_in -> mid (resblock, attention, resblock) -> 4 up blocks (3 resblocks each, nearest-2x + 3x3 upsampler
// after the first three) -> RMS norm + SiLU -> conv_out -> RGBA8. Weights are read by name from an uploaded
// .qw file (the converter's vae.qw layout, tools/convert.py:347-390). Every buffer, the GEMMs' stream-K
// workspace included, comes from the caller's workspace (kh_vae_workspace_bytes); everything is enqueued on one
// stream.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>

#include "kh_internal.h"

namespace kh {

namespace {

constexpr int OUTS[4] = {384, 384, 192, 96};  // up-block output channels (vae.mm:319)
constexpr int MID_C = 384;
constexpr long long S_CHUNK_BYTES = 1LL << 30;  // attention: f32 S chunk budget (query rows x padded keys)

inline long long ru(long long v, long long a) { return (v + a - 1) / a * a; }
inline int ld_of(int C) { return (int)ru(C, 64); }  // GEMM outputs are padded to 64 columns

// Query rows per attention S chunk: all of them while S fits S_CHUNK_BYTES (16384 at 1024^2), else a multiple of
// 256 (at least 256). Few, tall chunks keep the P V GEMM (rows x 384 outputs, K = all keys) wide enough that
// stream-K splits each tile only a few ways. KH_VAE_QCHUNK overrides (tests of the multi-chunk path).
long long query_chunk(long long P0, long long Pp0) {
  if (const char* e = getenv("KH_VAE_QCHUNK")) {
    const long long q = atoll(e);
    if (q > 0) return std::min(q, P0);
  }
  const long long fit = std::max<long long>(256, S_CHUNK_BYTES / (4 * Pp0) / 256 * 256);
  return std::min(fit, P0);
}

struct Plan {
  long long P0, P3, Pp0, qc;  // VAE-input pixels, output pixels, P0 rounded up to 64, attention query chunk
  size_t act, wpad, bpad, qkv, kt, S, Pm, gws, total;
  size_t off_act[5], off_wpad, off_bpad, off_qkv, off_kt, off_S, off_Pm, off_gws;
};

Plan plan(int H16, int W16) {
  Plan p{};
  p.P0 = 4LL * H16 * W16;
  p.P3 = 64LL * p.P0;  // three 2x upsamplers
  p.Pp0 = ru(p.P0, 64);
  // largest activation: P x padded channels over the stages (P0 x 384, 4 P0 x 384, 16 P0 x 192, 64 P0 x 128)
  const long long a = std::max({p.P0 * MID_C, 4 * p.P0 * 384, 16 * p.P0 * ld_of(192), p.P3 * ld_of(96)});
  p.act = (size_t)ru(a * 2, 256);
  // padded 3 x 3 weights [9 C -> 64, C -> 64] or sub-pixel weights [4 C -> 64, 4 Np] (C <= 384) and biases
  p.wpad = (size_t)ru(16LL * 384 * 384 * 2, 256);
  p.bpad = (size_t)ru(4 * 1152 * 4, 256);
  p.qkv = (size_t)ru(p.Pp0 * 3 * MID_C * 2, 256);
  p.kt = (size_t)ru((long long)MID_C * p.Pp0 * 2, 256);
  p.qc = query_chunk(p.P0, p.Pp0);
  p.S = (size_t)ru(p.qc * p.Pp0 * 4, 256);
  p.Pm = (size_t)ru(p.qc * p.Pp0 * 2, 256);
  size_t off = 0;
  for (int i = 0; i < 5; i++) {
    p.off_act[i] = off;
    off += p.act;
  }
  p.off_wpad = off, off += p.wpad;
  p.off_bpad = off, off += p.bpad;
  p.off_qkv = off, off += p.qkv;
  p.off_kt = off, off += p.kt;
  p.off_S = off, off += p.S;
  p.off_Pm = off, off += p.Pm;
  p.gws = (size_t)ru((long long)gemm_workspace_bytes(), 256);
  p.off_gws = off, off += p.gws;
  p.total = off;
  return p;
}

struct Act {
  uint16_t* p = nullptr;
  int H = 0, W = 0, C = 0, ld = 0;
  int slot = -1;
  long long P() const { return (long long)H * W; }
};

class Decoder {
 public:
  Decoder(hipStream_t st, const kh_qw* f, const Plan& pl, char* ws, Err& e)
      : st_(st), f_(f), pl_(pl), ws_(ws), e_(e), gws_{ws + pl.off_gws, pl.gws} {}

  int run(const float* z, int H16, int W16, void* rgba);

 private:
  hipStream_t st_;
  const kh_qw* f_;
  const Plan& pl_;
  char* ws_;
  Err& e_;
  const GemmWs gws_;  // the GEMMs' stream-K workspace, inside ws_
  bool used_[5] = {false, false, false, false, false};

  int acquire(int H, int W, int C, int ld, Act& a) {
    for (int i = 0; i < 5; i++)
      if (!used_[i]) {
        used_[i] = true;
        a.p = (uint16_t*)(ws_ + pl_.off_act[i]);
        a.H = H, a.W = W, a.C = C, a.ld = ld, a.slot = i;
        return KH_OK;
      }
    return e_.fail("vae: out of activation buffers");
  }
  void release(Act& a) {
    if (a.slot >= 0) used_[a.slot] = false;
    a.slot = -1;
  }
  // device pointer of tensor `name`, checked against its dtype and shape
  int tensor(const std::string& name, int dtype, long long d0, long long d1, const void*& ptr) {
    kh_qw_tensor t;
    if (kh_qw_find(f_, name.c_str(), &t) != KH_OK) return e_.fail("vae: missing tensor %s", name.c_str());
    if (!t.dev) return e_.fail("vae: weight file not uploaded (kh_qw_upload)");
    const long long n = t.ndim == 1 ? t.shape[0] : t.ndim == 2 ? t.shape[0] * t.shape[1] : -1;
    const bool ok = t.dtype == dtype && ((d1 < 0 && t.ndim == 1 && t.shape[0] == d0) ||
                                         (d1 >= 0 && t.ndim == 2 && t.shape[0] == d0 && t.shape[1] == d1));
    if (!ok)
      return e_.fail("vae: tensor %s: dtype %d shape (%lld x %lld, %d dims), expected dtype %d (%lld x %lld)",
                     name.c_str(), t.dtype, (long long)t.shape[0], t.ndim > 1 ? (long long)t.shape[1] : 0LL, t.ndim,
                     dtype, d0, d1);
    (void)n;
    ptr = t.dev;
    return KH_OK;
  }

  // 3 x 3 conv (zero padding 1; up: nearest-2x upsample of x first) x.C -> cout, + bias (+ residual)
  int conv3x3(const Act& x, const std::string& name, int cout, int up, const Act* res, Act& y) {
    int rc;
    const void *w, *b;
    const int K = 9 * x.C, Kp = (int)ru(K, 64), Np = ld_of(cout);
    if ((rc = tensor(name + ".weight", KH_BF16, K, cout, w)) || (rc = tensor(name + ".bias", KH_F32, cout, -1, b)))
      return rc;
    const void* W = w;
    const float* bias = (const float*)b;
    if (up && (Np % 128 == 0 || Np % 192 == 0)) {
      // nearest-2x + 3 x 3 as four 2 x 2 sub-pixel convs (the reference's mode 2, vae.mm:137-150): folded
      // weights W2 [4 Cin (-> 64), 4 Np] and a bias per phase in the workspace, then one implicit GEMM
      const int K2 = (int)ru(4 * x.C, 64);
      uint16_t* wp = (uint16_t*)(ws_ + pl_.off_wpad);
      float* bp = (float*)(ws_ + pl_.off_bpad);
      if ((size_t)K2 * 4 * Np * 2 > pl_.wpad || (size_t)4 * Np * 4 > pl_.bpad)
        return e_.fail("vae: sub-pixel weight too large");
      if ((rc = vae_subpix_weights(st_, w, KH_BF16, x.C, cout, wp, K2, Np, bias, bp, e_))) return rc;
      if (res) return e_.fail("vae: no residual on an upsampling conv");
      if ((rc = acquire(2 * x.H, 2 * x.W, cout, Np, y))) return rc;
      const kh_weight w2{wp, nullptr, KH_BF16, KH_F32, 0};
      return conv_up2_subpix(st_, x.p, x.ld, x.C, x.H, x.W, KH_BF16, w2, K2, Np, bp, y.p, Np, e_, &gws_);
    }
    if (Kp != K || Np != cout) {  // the GEMM's K and N multiples of 64: zero rows / columns
      uint16_t* wp = (uint16_t*)(ws_ + pl_.off_wpad);
      float* bp = (float*)(ws_ + pl_.off_bpad);
      if ((size_t)Kp * Np * 2 > pl_.wpad || (size_t)Np * 4 > pl_.bpad) return e_.fail("vae: padded weight too large");
      if ((rc = vae_pad_weight(st_, w, K, cout, wp, Kp, Np, bias, bp, e_))) return rc;
      W = wp;
      bias = bp;
    }
    const int H = up ? 2 * x.H : x.H, Wd = up ? 2 * x.W : x.W;
    if ((rc = acquire(H, Wd, cout, Np, y))) return rc;
    const kh_weight wt{W, nullptr, KH_BF16, KH_F32, 0};
    if (res && (res->ld != y.ld || res->P() != y.P())) return e_.fail("vae: residual shape mismatch");
    // the residual add is fused into the GEMM epilogue (the reference's vconv res input, vae.mm:112-125)
    return kh::conv3x3(st_, x.p, x.ld, x.C, H, Wd, up, KH_BF16, wt, Kp, Np, bias, res ? res->p : nullptr, y.p, Np, e_, &gws_);
  }

  // 1 x 1 conv x.C -> cout (+ residual): a plain GEMM on the activation rows
  int conv1x1(const Act& x, const std::string& name, int cout, const Act* res, Act& y) {
    int rc;
    const void *w, *b;
    if (x.C % 64 || cout % 64) return e_.fail("vae: 1x1 conv %s needs channels %% 64", name.c_str());
    if ((rc = tensor(name + ".weight", KH_BF16, x.C, cout, w)) || (rc = tensor(name + ".bias", KH_F32, cout, -1, b)))
      return rc;
    if ((rc = acquire(x.H, x.W, cout, cout, y))) return rc;
    const kh_weight wt{w, nullptr, KH_BF16, KH_F32, 0};
    if ((rc = gemm(st_, KH_EPI_BIAS16, x.p, KH_BF16, wt, y.p, (int)x.P(), cout, x.C, x.ld, cout, cout, (const float*)b,
                   e_, &gws_)))
      return rc;
    if (res) {
      if (res->ld != y.ld || res->P() != y.P()) return e_.fail("vae: residual shape mismatch");
      if ((rc = vae_add(st_, y.p, res->p, y.P() * y.ld, e_))) return rc;
    }
    return KH_OK;
  }

  int norm(const Act& x, const std::string& gamma, int silu, Act& y) {
    int rc;
    const void* g;
    if ((rc = tensor(gamma, KH_F32, x.C, -1, g))) return rc;
    if ((rc = acquire(x.H, x.W, x.C, x.ld, y))) return rc;
    return vae_norm_silu(st_, x.p, x.ld, (const float*)g, y.p, y.ld, (int)x.P(), x.C, silu, e_);
  }

  // vae.mm:171-186 (resblock); consumes x
  int resblock(Act& x, const std::string& p, int cout) {
    int rc;
    Act h = x, t1, t2, t3, y;
    if (x.C != cout && (rc = conv1x1(x, p + "conv_shortcut", cout, nullptr, h))) return rc;
    if ((rc = norm(x, p + "norm1.gamma", 1, t1))) return rc;
    if ((rc = conv3x3(t1, p + "conv1", cout, 0, nullptr, t2))) return rc;
    release(t1);
    if ((rc = norm(t2, p + "norm2.gamma", 1, t3))) return rc;
    release(t2);
    if ((rc = conv3x3(t3, p + "conv2", cout, 0, &h, y))) return rc;
    release(t3);
    if (h.slot != x.slot) release(h);
    release(x);
    x = y;
    return KH_OK;
  }

  // vae.mm:245-270: single-head self-attention over all pixels (C = 384), S = Q K^T in f32 chunks of query
  // rows, row softmax, P V; then proj + residual. Consumes x.
  int attention(Act& x, const std::string& p) {
    int rc;
    const int C = x.C;
    const long long P = x.P(), Pp = pl_.Pp0;
    if (C != MID_C || P > pl_.P0) return e_.fail("vae: attention shape");
    const void *wq, *bq;
    if ((rc = tensor(p + "to_qkv.weight", KH_BF16, C, 3 * C, wq)) || (rc = tensor(p + "to_qkv.bias", KH_F32, 3 * C, -1, bq)))
      return rc;
    Act n, o, y;
    if ((rc = norm(x, p + "norm.gamma", 0, n))) return rc;
    uint16_t* qkv = (uint16_t*)(ws_ + pl_.off_qkv);
    uint16_t* kt = (uint16_t*)(ws_ + pl_.off_kt);
    float* S = (float*)(ws_ + pl_.off_S);
    uint16_t* Pm = (uint16_t*)(ws_ + pl_.off_Pm);
    // padded keys must be zero: V rows [P, Pp) of qkv, K^T columns [P, Pp), P columns [P, Pp)
    if (Pp != P && ((rc = vae_zero(st_, qkv, pl_.qkv, e_)) || (rc = vae_zero(st_, kt, pl_.kt, e_)) ||
                    (rc = vae_zero(st_, Pm, pl_.Pm, e_))))
      return rc;
    const kh_weight wqkv{wq, nullptr, KH_BF16, KH_F32, 0};
    if ((rc = gemm(st_, KH_EPI_BIAS16, n.p, KH_BF16, wqkv, qkv, (int)P, 3 * C, C, n.ld, 3 * C, 3 * C, (const float*)bq, e_, &gws_)))
      return rc;
    release(n);
    if ((rc = vae_transpose(st_, qkv, 3 * C, C, (int)P, C, kt, (int)Pp, e_))) return rc;
    if ((rc = acquire(x.H, x.W, C, C, o))) return rc;
    const kh_weight wk{kt, nullptr, KH_BF16, KH_F32, 0};
    const kh_weight wv{qkv + 2 * C, nullptr, KH_BF16, KH_F32, 0};
    const float scale = (float)(1.0 / std::sqrt((double)C));
    for (long long q0 = 0; q0 < P; q0 += pl_.qc) {
      const int rows = (int)std::min<long long>(pl_.qc, P - q0);
      if ((rc = gemm(st_, KH_EPI_F32, qkv + (size_t)q0 * 3 * C, KH_BF16, wk, S, rows, (int)Pp, C, 3 * C, (int)Pp, (int)Pp,
                     nullptr, e_, &gws_)))
        return rc;
      if ((rc = vae_softmax(st_, S, (int)Pp, rows, (int)P, scale, Pm, e_))) return rc;
      if ((rc = gemm(st_, KH_EPI_STORE16, Pm, KH_BF16, wv, o.p + (size_t)q0 * C, rows, C, (int)Pp, (int)Pp, 3 * C, C,
                     nullptr, e_, &gws_)))
        return rc;
    }
    if ((rc = conv1x1(o, p + "proj", C, &x, y))) return rc;
    release(o);
    release(x);
    x = y;
    return KH_OK;
  }
};

int Decoder::run(const float* z, int H16, int W16, void* rgba) {
  int rc;
  if (gws_.bytes && (rc = gemm_workspace_init(st_, gws_.p, gws_.bytes, e_))) return rc;
  const void *mean, *stdv, *pw, *pb;
  if ((rc = tensor("latents_mean", KH_F32, 16, -1, mean)) || (rc = tensor("latents_std", KH_F32, 16, -1, stdv)) ||
      (rc = tensor("post_quant_conv.weight", KH_F32, 16, 16, pw)) || (rc = tensor("post_quant_conv.bias", KH_F32, 16, -1, pb)))
    return rc;
  Act x;
  if ((rc = acquire(2 * H16, 2 * W16, 16, 16, x))) return rc;
  if ((rc = vae_unpack(st_, z, (const float*)mean, (const float*)stdv, (const float*)pw, (const float*)pb, x.p, H16, W16,
                       e_)))
    return rc;
  Act y;
  if ((rc = conv3x3(x, "decoder.conv_in", MID_C, 0, nullptr, y))) return rc;
  release(x);
  x = y;
  if ((rc = resblock(x, "decoder.mid_block.resnets.0.", MID_C))) return rc;
  if ((rc = attention(x, "decoder.mid_block.attentions.0."))) return rc;
  if ((rc = resblock(x, "decoder.mid_block.resnets.1.", MID_C))) return rc;
  for (int b = 0; b < 4; b++) {
    const std::string p = "decoder.up_blocks." + std::to_string(b) + ".";
    for (int r = 0; r < 3; r++)
      if ((rc = resblock(x, p + "resnets." + std::to_string(r) + ".", OUTS[b]))) return rc;
    if (b < 3) {
      if ((rc = conv3x3(x, p + "upsamplers.0.resample.1", OUTS[b] / 2, 1, nullptr, y))) return rc;
      release(x);
      x = y;
    }
  }
  Act n;
  if ((rc = norm(x, "decoder.norm_out.gamma", 1, n))) return rc;
  release(x);
  const void *wo, *bo;
  if ((rc = tensor("decoder.conv_out.weight", KH_BF16, 9LL * n.C, 4, wo)) ||
      (rc = tensor("decoder.conv_out.bias", KH_F32, 4, -1, bo)))
    return rc;
  rc = vae_conv_out(st_, n.p, n.ld, n.C, wo, (const float*)bo, rgba, n.H, n.W, e_);
  release(n);
  return rc;
}

}  // namespace

size_t vae_workspace_bytes(int H16, int W16) {
  if (H16 <= 0 || W16 <= 0) return 0;
  return plan(H16, W16).total;
}

int vae_decode(hipStream_t st, const kh_qw* f, const float* z, int H16, int W16, void* ws, size_t ws_bytes, void* rgba,
               Err& e) {
  if (!f || !z || !ws || !rgba) return e.fail("vae_decode: null argument");
  if (H16 <= 0 || W16 <= 0 || H16 > 512 || W16 > 512) return e.fail("vae_decode: latent %d x %d out of range", H16, W16);
  const Plan pl = plan(H16, W16);
  if (ws_bytes < pl.total) return e.fail("vae_decode: workspace %zu bytes < %zu needed", ws_bytes, pl.total);
  if ((uintptr_t)ws & 255) return e.fail("vae_decode: workspace must be 256-byte aligned");
  Decoder d(st, f, pl, (char*)ws, e);
  return d.run(z, H16, W16, rgba);
}

}  // namespace kh
