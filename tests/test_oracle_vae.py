"""Pins the oracle's VAE functions (oracle/oracle.c, or_vae_*) against numpy float64 restatements written
here from the reference kernels' definitions (engine/kernels/vae.metal), plus invariants: nearest-upsample
conv == conv of the explicitly upsampled input; 1x1 conv == matmul; unpack round trip of the latent patch
layout; softmax rows sum to 1; the RGBA quantization's fixed points. CPU only."""
import numpy as np
import pytest

from oracle import oracle as O

rng = np.random.default_rng(42)


def bf(a):
    return O.from_f32(np.asarray(a, np.float32), O.BF16)


def f32(b):
    return O.to_f32(b, O.BF16).astype(np.float64)


def conv_ref(x, H, W, w, bias, ks=3, up=0, res=None):
    """float64 conv on the bf16 values: zero padding ks // 2, NHWC."""
    C = x.shape[1]
    Hin, Win = (H // 2, W // 2) if up else (H, W)
    img = f32(x).reshape(Hin, Win, C)
    if up:
        img = img.repeat(2, axis=0).repeat(2, axis=1)
    pad = ks // 2
    imgp = np.pad(img, ((pad, pad), (pad, pad), (0, 0)))
    wt = f32(w).reshape(ks * ks, C, -1)
    out = np.zeros((H, W, wt.shape[2]))
    for t in range(ks * ks):
        dy, dx = t // ks, t % ks
        out += imgp[dy:dy + H, dx:dx + W, :] @ wt[t]
    out = out.reshape(H * W, -1) + bias
    if res is not None:
        out += f32(res)
    return out


@pytest.mark.parametrize("up,ks,res", [(0, 3, False), (1, 3, False), (0, 3, True), (0, 1, False), (0, 1, True)])
def test_vae_conv_matches_float64(up, ks, res):
    H, W, C, N = 6, 10, 16, 24
    Hin, Win = (H // 2, W // 2) if up else (H, W)
    x = bf(rng.standard_normal((Hin * Win, C)))
    w = bf(rng.standard_normal((ks * ks * C, N)) * 0.2)
    b = rng.standard_normal(N).astype(np.float32) * 0.1
    r = bf(rng.standard_normal((H * W, N))) if res else None
    got = f32(O.vae_conv(x, H, W, w, b, N, ks=ks, up=up, res=r))
    ref = conv_ref(x, H, W, w, b, ks=ks, up=up, res=r)
    # one bf16 rounding of the result (2^-9 relative) and fp32 summation differences
    assert np.abs(got - ref).max() <= 2 ** -8 * np.abs(ref).max() + 1e-6


def test_vae_conv_upsample_equals_conv_of_repeated_input():
    H, W, C, N = 8, 6, 8, 16
    x = bf(rng.standard_normal((H // 2 * W // 2, C)))
    w = bf(rng.standard_normal((9 * C, N)) * 0.2)
    b = np.zeros(N, np.float32)
    xu = x.reshape(H // 2, W // 2, C).repeat(2, axis=0).repeat(2, axis=1).reshape(H * W, C)
    np.testing.assert_array_equal(O.vae_conv(x, H, W, w, b, N, up=1), O.vae_conv(xu, H, W, w, b, N, up=0))


def test_vae_norm_silu_matches_float64():
    P, C = 37, 96
    x = bf(rng.standard_normal((P, C)) * 3)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    for silu in (0, 1):
        got = f32(O.vae_norm_silu(x, g, silu))
        xf = f32(x)
        t = xf / np.maximum(np.linalg.norm(xf, axis=1, keepdims=True), 1e-12) * np.sqrt(C) * g
        if silu:
            t = t / (1 + np.exp(-t))
        assert np.abs(got - t).max() <= 2 ** -8 * np.abs(t).max()
    z = O.vae_norm_silu(np.zeros((2, 8), np.uint16), np.ones(8, np.float32), 1)
    assert (f32(z) == 0).all()  # ||x|| = 0: the 1e-12 floor, no NaN


def test_vae_unpack_layout_and_affine():
    H16, W16 = 3, 5
    z = rng.standard_normal((H16 * W16, 64)).astype(np.float32)
    mean = rng.standard_normal(16).astype(np.float32)
    std = (1 + rng.random(16)).astype(np.float32)
    w = rng.standard_normal((16, 16)).astype(np.float32) * 0.3
    b = rng.standard_normal(16).astype(np.float32)
    got = f32(O.vae_unpack(z, mean, std, w, b, H16, W16))
    # token (i, j) feature c * 4 + py * 2 + px -> latent pixel (2 i + py, 2 j + px), channel c
    lat = z.reshape(H16, W16, 16, 2, 2).transpose(0, 3, 1, 4, 2).reshape(2 * H16 * 2 * W16, 16).astype(np.float64)
    ref = (lat * std + mean) @ w + b
    assert np.abs(got - ref).max() <= 2 ** -8 * np.abs(ref).max() + 1e-6


def test_vae_softmax_rows():
    S = rng.standard_normal((5, 40)).astype(np.float32) * 4
    P = f32(O.vae_softmax(S, 33, 0.5))
    e = np.exp(S[:, :33] * 0.5 - (S[:, :33] * 0.5).max(axis=1, keepdims=True))
    ref = e / e.sum(axis=1, keepdims=True)
    assert np.abs(P[:, :33] - ref).max() <= 2 ** -8
    assert (P[:, 33:] == 0).all()
    assert np.allclose(P[:, :33].sum(axis=1), 1, atol=0.02)


def test_vae_conv_out_quantization():
    H, W, C = 5, 7, 16
    x = bf(rng.standard_normal((H * W, C)))
    w = bf(rng.standard_normal((9 * C, 4)) * 0.3)
    b = np.array([0.1, -0.2, 0.0, 1.0], np.float32)
    got = O.vae_conv_out(x, w, b, H, W)
    acc = conv_ref(x, H, W, w, b)
    ref = np.rint(np.clip(np.clip(acc, -1, 1) * 0.5 + 0.5, 0, 1) * 255)
    assert np.abs(got.astype(np.int32) - ref).max() <= 1  # a rounding tie may land either way
    # fixed points: bias -1 / 0 / +1 with zero weights -> 0 / 128 (rint(127.5) = 128) / 255
    z = O.vae_conv_out(x, np.zeros((9 * C, 4), np.uint16), np.array([-1, 0, 1, 1], np.float32), H, W)
    assert (z[:, 0] == 0).all() and (z[:, 1] == 128).all() and (z[:, 2] == 255).all()


def test_decoder_spec_names():
    from krea_image_amd import vae
    specs = vae.decoder_specs()
    names = [n for n, _, _ in specs]
    assert len(names) == len(set(names))
    assert "decoder.up_blocks.1.resnets.0.conv_shortcut.weight" in names   # 192 -> 384
    assert "decoder.up_blocks.0.resnets.0.conv_shortcut.weight" not in names
    assert dict((n, s) for n, _, s in specs)["decoder.up_blocks.2.upsamplers.0.resample.1.weight"] == (9 * 192, 96)


def test_vae_conv_more_than_1024_outputs():
    """The oracle accumulates output channels in blocks of 1024: to_qkv has 1152."""
    P, C, N = 3, 16, 1152
    x = bf(rng.standard_normal((P, C)))
    w = bf(rng.standard_normal((C, N)) * 0.2)
    b = rng.standard_normal(N).astype(np.float32)
    got = f32(O.vae_conv(x, 1, P, w, b, N, ks=1))
    ref = f32(x) @ f32(w) + b
    assert np.abs(got - ref).max() <= 2 ** -8 * np.abs(ref).max()


def test_vae_subpix_weights_closed_form():
    """Each folded tap is the sum of the 3x3 taps that the nearest upsample maps onto it: every 3x3 tap is used
    exactly once per phase, so the four 2x2 taps of a phase add up to the sum of all nine (up to rounding)."""
    rng = np.random.default_rng(4)
    Cin, Cout = 8, 16
    w = O.from_f32(rng.standard_normal((9 * Cin, Cout)).astype(np.float32), O.BF16)
    w2 = O.to_f32(O.vae_subpix_weights(w, Cin, Cout), O.BF16)
    wf = O.to_f32(w, O.BF16).reshape(3, 3, Cin, Cout)
    # phase (0, 0), tap (0, 0) is the single corner tap W[0, 0]; tap (1, 1) sums W[1:, 1:]
    np.testing.assert_array_equal(w2[:Cin, :Cout], wf[0, 0])
    np.testing.assert_allclose(w2[3 * Cin:4 * Cin, :Cout], wf[1:, 1:].sum((0, 1)), rtol=1e-2, atol=1e-2)
    for ph in range(4):
        tot = w2[:, ph * Cout:(ph + 1) * Cout].reshape(4, Cin, Cout).sum(0)
        np.testing.assert_allclose(tot, wf.sum((0, 1)), rtol=3e-2, atol=3e-2)


def test_vae_conv_up2_matches_direct_upsampled_conv():
    """conv3x3(nearest2x(x)) == the sub-pixel form exactly in real arithmetic; here the folded weights are
    rounded to bf16 once, so the two agree to a few bf16 ulps."""
    rng = np.random.default_rng(5)
    H, W, Cin, Cout = 5, 6, 16, 8
    x = O.from_f32(rng.standard_normal((H * W, Cin)).astype(np.float32), O.BF16)
    w = O.from_f32((rng.standard_normal((9 * Cin, Cout)) / 12).astype(np.float32), O.BF16)
    b = rng.standard_normal(Cout).astype(np.float32)
    direct = O.to_f32(O.vae_conv(x, 2 * H, 2 * W, w, b, Cout, ks=3, up=1), O.BF16)
    sub = O.to_f32(O.vae_conv_up2(x, H, W, O.vae_subpix_weights(w, Cin, Cout), b, Cout), O.BF16)
    assert np.linalg.norm(sub - direct) / np.linalg.norm(direct) < 1e-2
