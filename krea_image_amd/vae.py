"""VAE decoder on libkh: the Qwen-Image (Wan 2.1) decoder of the Krea 2 engine (engine/src/vae.mm:289-337,
VAEDecoder::run), single frame, over the C ABI (kh_vae_decode and the kh_vae_* ops).

Weights are the converter's vae.qw tensors (tools/convert.py:338-390): 3x3 / 1x1 conv weights bf16 in the
implicit-GEMM layout Wt[(ky*3 + kx)*Cin + ci, co], biases / norm gammas / post_quant_conv / latent statistics f32,
conv_out padded to 4 outputs (alpha: zero weights, bias 1). No checkpoint is available offline, so
write_random_vae() writes a random-init file with exactly those names and shapes.
"""
import ctypes
from typing import List, Tuple

import numpy as np
import torch

from . import kh
from .qw import QwFile, QwWriter, bf16_bits

OUTS = (384, 384, 192, 96)  # up-block output channels (vae.mm:319)
MID = 384


def _resblock_specs(p: str, cin: int, cout: int) -> List[Tuple[str, str, tuple]]:
    s = []
    if cin != cout:
        s += [(p + "conv_shortcut.weight", "bf16", (cin, cout)), (p + "conv_shortcut.bias", "f32", (cout,))]
    s += [(p + "norm1.gamma", "f32", (cin,)), (p + "conv1.weight", "bf16", (9 * cin, cout)), (p + "conv1.bias", "f32", (cout,)),
          (p + "norm2.gamma", "f32", (cout,)), (p + "conv2.weight", "bf16", (9 * cout, cout)), (p + "conv2.bias", "f32", (cout,))]
    return s


def decoder_specs() -> List[Tuple[str, str, tuple]]:
    """(name, dtype, shape) of every tensor kh_vae_decode reads, in the converter's layout."""
    d = "decoder."
    s = [("latents_mean", "f32", (16,)), ("latents_std", "f32", (16,)),
         ("post_quant_conv.weight", "f32", (16, 16)), ("post_quant_conv.bias", "f32", (16,)),
         (d + "conv_in.weight", "bf16", (9 * 16, MID)), (d + "conv_in.bias", "f32", (MID,))]
    s += _resblock_specs(d + "mid_block.resnets.0.", MID, MID)
    a = d + "mid_block.attentions.0."
    s += [(a + "norm.gamma", "f32", (MID,)), (a + "to_qkv.weight", "bf16", (MID, 3 * MID)),
          (a + "to_qkv.bias", "f32", (3 * MID,)), (a + "proj.weight", "bf16", (MID, MID)), (a + "proj.bias", "f32", (MID,))]
    s += _resblock_specs(d + "mid_block.resnets.1.", MID, MID)
    cin = MID
    for b, cout in enumerate(OUTS):
        p = f"{d}up_blocks.{b}."
        for r in range(3):
            s += _resblock_specs(f"{p}resnets.{r}.", cin if r == 0 else cout, cout)
        cin = cout
        if b < 3:
            u = p + "upsamplers.0.resample.1."
            s += [(u + "weight", "bf16", (9 * cout, cout // 2)), (u + "bias", "f32", (cout // 2,))]
            cin = cout // 2
    s += [(d + "norm_out.gamma", "f32", (96,)), (d + "conv_out.weight", "bf16", (9 * 96, 4)),
          (d + "conv_out.bias", "f32", (4,))]
    return s


def write_random_vae(path: str, seed: int = 0):
    """Random-init decoder weights with He-like scales (conv outputs keep unit-order activations), gammas near
    1, latent statistics like the real model's order of magnitude; conv_out's alpha row zero, bias 1."""
    rng = np.random.default_rng(seed)
    specs = decoder_specs()
    w = QwWriter(path, specs, {"model": "qwen-image-vae decoder (random init)", "seed": seed})
    for name, dt, shape in specs:
        if name.endswith("gamma"):
            a = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
        elif name == "latents_std":
            a = (1.0 + 0.5 * rng.random(shape)).astype(np.float32)
        elif name == "decoder.conv_out.weight":
            a = (rng.standard_normal(shape) / np.sqrt(shape[0])).astype(np.float32)
            a[:, 3] = 0.0
        elif name == "decoder.conv_out.bias":
            a = np.array([0.0, 0.0, 0.0, 1.0], np.float32)
        elif name.endswith(".bias") or name == "latents_mean":
            a = (0.05 * rng.standard_normal(shape)).astype(np.float32)
        else:  # weights [fan_in, fan_out]
            a = (rng.standard_normal(shape) / np.sqrt(shape[0])).astype(np.float32)
        w.write(name, bf16_bits(a) if dt == "bf16" else a)
    w.close()


def decode_flops(H16: int, W16: int) -> float:
    """Algorithmic FLOPs of one decode (2 per multiply-add, unpadded channel counts): the convolutions (3 x 3,
    1 x 1, and the upsamplers in the reference's sub-pixel form: 2 x 2 taps per output pixel), the mid-block
    attention's Q K^T and P V, and the output conv."""
    P = 4 * H16 * W16
    f = 2.0 * P * 144 * MID  # conv_in

    def res(P, cin, cout):
        return 2.0 * P * (9 * cin * cout + 9 * cout * cout + (cin * cout if cin != cout else 0))

    f += res(P, MID, MID) * 2
    f += 2.0 * P * MID * 4 * MID + 4.0 * P * P * MID  # to_qkv + proj, Q K^T + P V
    cin = MID
    for b, cout in enumerate(OUTS):
        for r in range(3):
            f += res(P, cin if r == 0 else cout, cout)
        cin = cout
        if b < 3:
            P *= 4
            f += 2.0 * P * 4 * cout * (cout // 2)  # sub-pixel form: 2 x 2 taps per output pixel
            cin = cout // 2
    return f + 2.0 * P * 9 * 96 * 4


def _bind(lib):
    if getattr(lib, "_vae_bound", False):
        return lib
    vp, i, cp, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t
    lib.kh_vae_workspace_bytes.argtypes, lib.kh_vae_workspace_bytes.restype = [i, i], sz
    lib.kh_vae_decode.argtypes = [vp, vp, vp, i, i, vp, sz, vp, cp, i]
    lib.kh_vae_decode.restype = i
    lib.kh_vae_im2col.argtypes = [vp, vp, i, i, i, i, i, i, i, vp, i, cp, i]
    lib.kh_vae_conv3x3.argtypes = [vp, vp, i, i, i, i, i, i, vp, i, i, vp, vp, vp, i, vp, ctypes.c_size_t, cp, i]
    lib.kh_vae_subpix_weights.argtypes = [vp, vp, i, i, i, vp, i, i, vp, vp, cp, i]
    lib.kh_vae_conv_up2.argtypes = [vp, vp, i, i, i, i, i, vp, i, i, vp, vp, i, vp, ctypes.c_size_t, cp, i]
    lib.kh_vae_norm_silu.argtypes = [vp, vp, i, vp, vp, i, i, i, i, cp, i]
    lib.kh_vae_unpack.argtypes = [vp] * 7 + [i, i, cp, i]
    lib.kh_vae_softmax.argtypes = [vp, vp, i, i, i, ctypes.c_float, vp, cp, i]
    lib.kh_vae_conv_out.argtypes = [vp, vp, i, i, vp, vp, vp, i, i, cp, i]
    for n in ("kh_vae_conv3x3", "kh_vae_subpix_weights", "kh_vae_conv_up2", "kh_vae_im2col", "kh_vae_norm_silu", "kh_vae_unpack", "kh_vae_softmax", "kh_vae_conv_out"):
        getattr(lib, n).restype = i
    lib._vae_bound = True
    return lib


def _call(fn, *args):
    err = ctypes.create_string_buffer(512)
    kh._check(fn(*args, err, 512), err)


def _dp(t):
    return ctypes.c_void_p(t.data_ptr() if hasattr(t, "data_ptr") else int(t))


def _ws(ws):
    return None if ws is None else _dp(ws)


def _ws_bytes(ws) -> int:
    return 0 if ws is None else ws.numel() * ws.element_size()


def conv3x3(x, ldx, C, H, W, up, w, K, N, bias, y, ldy, res=None, ws=None):
    """VAEDecoder::conv mode 3 (engine/src/vae.mm:112-125): implicit-GEMM 3x3 conv, y = conv(x) + bias
    (+ res, added after the 16-bit rounding of the biased output). w: 16-bit Wt [K, N] (K >= 9 C, a multiple
    of 64); H x W output pixels (up: x is H/2 x W/2); res like y."""
    P, Pin = H * W, (H // 2) * (W // 2) if up else H * W
    kh._need(x, "x", Pin, C, ldx, x.element_size())
    kh._need(w, "W", K, N, N, 2)
    kh._need(bias, "bias", 1, N, N, 4)
    kh._need(y, "y", P, N, ldy, y.element_size())
    if res is not None:
        kh._need(res, "res", P, N, ldy, res.element_size())
        if res.dtype != x.dtype:
            raise kh.KhError("conv3x3: res must have the activation type")
    if w.dtype != x.dtype or y.dtype != x.dtype or bias.dtype != torch.float32:
        raise kh.KhError("conv3x3: x, w and y share one 16-bit type; bias is f32")
    wc = kh.Weight(w).c()
    _call(_bind(kh.load()).kh_vae_conv3x3, kh._stream(), _dp(x), ldx, C, H, W, up, kh.dtype_code(x.dtype),
          ctypes.byref(wc), K, N, _dp(bias), None if res is None else _dp(res), _dp(y), ldy, _ws(ws), _ws_bytes(ws))


def subpix_weights(w, Cin, Cout, w2, K, Np, bias=None, bias4=None):
    """vae_subpix_weights (engine/kernels/vae.metal:134-160): w [9 Cin, Cout] 16-bit -> w2 [K, 4 Np]."""
    kh._need(w, "w", 9 * Cin, Cout, Cout, 2)
    kh._need(w2, "w2", K, 4 * Np, 4 * Np, 2)
    if bias4 is not None:
        kh._need(bias4, "bias4", 1, 4 * Np, 4 * Np, 4)
    _call(_bind(kh.load()).kh_vae_subpix_weights, kh._stream(), _dp(w), kh.dtype_code(w.dtype), Cin, Cout, _dp(w2), K,
          Np, None if bias is None else _dp(bias), None if bias4 is None else _dp(bias4))


def conv_up2(x, ldx, C, H, W, w2, K, Np, bias4, y, ldy, ws=None):
    """VAEDecoder::conv mode 2 (engine/src/vae.mm:137-150): y [(2H)(2W), ldy] = conv3x3(nearest2x(x)) + bias
    as four sub-pixel 2 x 2 convs; x [H W, ldx] low-res, w2 / bias4 from subpix_weights."""
    kh._need(x, "x", H * W, C, ldx, x.element_size())
    kh._need(w2, "w2", K, 4 * Np, 4 * Np, 2)
    kh._need(bias4, "bias4", 1, 4 * Np, 4 * Np, 4)
    kh._need(y, "y", 4 * H * W, Np, ldy, y.element_size())
    if w2.dtype != x.dtype or y.dtype != x.dtype:
        raise kh.KhError("conv_up2: x, w2 and y share one 16-bit type")
    wc = kh.Weight(w2).c()
    _call(_bind(kh.load()).kh_vae_conv_up2, kh._stream(), _dp(x), ldx, C, H, W, kh.dtype_code(x.dtype),
          ctypes.byref(wc), K, Np, _dp(bias4), _dp(y), ldy, _ws(ws), _ws_bytes(ws))


def im2col(x, ldx, C, H, W, up, m0, rows, col, Kpad):
    _call(_bind(kh.load()).kh_vae_im2col, kh._stream(), _dp(x), ldx, C, H, W, up, m0, rows, _dp(col), Kpad)


def norm_silu(x, ldx, gamma, y, ldy, P, C, silu):
    _call(_bind(kh.load()).kh_vae_norm_silu, kh._stream(), _dp(x), ldx, _dp(gamma), _dp(y), ldy, P, C, silu)


def unpack(z, mean, stdv, w, b, y, H16, W16):
    _call(_bind(kh.load()).kh_vae_unpack, kh._stream(), _dp(z), _dp(mean), _dp(stdv), _dp(w), _dp(b), _dp(y), H16, W16)


def softmax(S, ld, rows, n, scale, P):
    _call(_bind(kh.load()).kh_vae_softmax, kh._stream(), _dp(S), ld, rows, n, scale, _dp(P))


def conv_out(x, ldx, C, w, bias, rgba, H, W):
    _call(_bind(kh.load()).kh_vae_conv_out, kh._stream(), _dp(x), ldx, C, _dp(w), _dp(bias), _dp(rgba), H, W)


def workspace_bytes(H16: int, W16: int) -> int:
    return int(_bind(kh.load()).kh_vae_workspace_bytes(H16, W16))


class VaeDecoder:
    """VAEDecoder (engine/src/vae.mm) over an uploaded vae.qw; the workspace is allocated once per latent size."""

    def __init__(self, f: QwFile, dev):
        self.f, self.dev = f, dev
        self._ws = None
        self._ws_key = None

    def decode(self, z: torch.Tensor, H16: int, W16: int, rgba: torch.Tensor = None) -> torch.Tensor:
        """z: f32 [H16 * W16, 64] DiT latent tokens on the device -> uint8 [16 H16, 16 W16, 4] RGBA."""
        if rgba is None:
            rgba = torch.empty(16 * H16, 16 * W16, 4, dtype=torch.uint8, device=self.dev)
        need = workspace_bytes(H16, W16)
        if self._ws_key != (H16, W16):
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.dev)
            self._ws_key = (H16, W16)
        lib = _bind(kh.load())
        err = ctypes.create_string_buffer(512)
        rc = lib.kh_vae_decode(kh._stream(), ctypes.c_void_p(self.f.h), _dp(z), H16, W16, _dp(self._ws), need,
                               _dp(rgba), err, 512)
        kh._check(rc, err)
        return rgba
