"""The oracle's composition of VAEDecoder::run (engine/src/vae.mm:289-337) over a vae.qw file read on the host:
the decoder graph of krea_image_amd/vae.py built from oracle/oracle.c's per-op restatements (or_vae_*), with the
mid-block attention (vae.mm:245-270) as numpy f32 Q K^T + the oracle's row softmax + P V rounded to bf16, and
the upsamplers as the reference's sub-pixel convs (vae.mm:137-150).
Test infrastructure only."""
import numpy as np

from oracle import oracle as O

OUTS = (384, 384, 192, 96)


def _bf(a):
    return O.from_f32(a, O.BF16)


def _resblock(f, x, H, W, p, cout):
    h = x if x.shape[1] == cout else O.vae_conv(x, H, W, f.array(p + "conv_shortcut.weight"),
                                                f.array(p + "conv_shortcut.bias"), cout, ks=1)
    t = O.vae_norm_silu(x, f.array(p + "norm1.gamma"), 1)
    t = O.vae_conv(t, H, W, f.array(p + "conv1.weight"), f.array(p + "conv1.bias"), cout)
    t = O.vae_norm_silu(t, f.array(p + "norm2.gamma"), 1)
    return O.vae_conv(t, H, W, f.array(p + "conv2.weight"), f.array(p + "conv2.bias"), cout, res=h)


def _attention(f, x, H, W, p):
    C = x.shape[1]
    n = O.vae_norm_silu(x, f.array(p + "norm.gamma"), 0)
    qkv = O.to_f32(O.vae_conv(n, H, W, f.array(p + "to_qkv.weight"), f.array(p + "to_qkv.bias"), 3 * C, ks=1), O.BF16)
    q, k, v = qkv[:, :C], qkv[:, C:2 * C], qkv[:, 2 * C:]
    S = (q.astype(np.float64) @ k.T.astype(np.float64)).astype(np.float32)
    P = O.to_f32(O.vae_softmax(S, S.shape[1], 1.0 / np.sqrt(C)), O.BF16)
    o = _bf((P.astype(np.float64) @ v.astype(np.float64)).astype(np.float32))
    return O.vae_conv(o, H, W, f.array(p + "proj.weight"), f.array(p + "proj.bias"), C, ks=1, res=x)


def decode(f, z, H16, W16):
    """z f32 [H16 W16, 64] -> uint8 [16 H16, 16 W16, 4]."""
    H, W = 2 * H16, 2 * W16
    x = O.vae_unpack(z, f.array("latents_mean"), f.array("latents_std"), f.array("post_quant_conv.weight"),
                     f.array("post_quant_conv.bias"), H16, W16)
    d = "decoder."
    x = O.vae_conv(x, H, W, f.array(d + "conv_in.weight"), f.array(d + "conv_in.bias"), 384)
    x = _resblock(f, x, H, W, d + "mid_block.resnets.0.", 384)
    x = _attention(f, x, H, W, d + "mid_block.attentions.0.")
    x = _resblock(f, x, H, W, d + "mid_block.resnets.1.", 384)
    for b, cout in enumerate(OUTS):
        for r in range(3):
            x = _resblock(f, x, H, W, f"{d}up_blocks.{b}.resnets.{r}.", cout)
        if b < 3:
            u = f"{d}up_blocks.{b}.upsamplers.0.resample.1."
            w2 = O.vae_subpix_weights(f.array(u + "weight"), cout, cout // 2)
            x = O.vae_conv_up2(x, H, W, w2, f.array(u + "bias"), cout // 2)  # the reference's mode 2
            H, W = 2 * H, 2 * W
    x = O.vae_norm_silu(x, f.array(d + "norm_out.gamma"), 1)
    return O.vae_conv_out(x, f.array(d + "conv_out.weight"), f.array(d + "conv_out.bias"), H, W).reshape(H, W, 4)
