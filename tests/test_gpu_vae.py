"""VAE decoder on the GPU (kh_vae_* through libkh) against the oracle: the per-op kernels (im2col bit-exact; norm,
unpack, softmax within one bf16 rounding; conv_out within one level), and the full kh_vae_decode
(engine/src/vae.mm:289-337) on a random-init vae.qw against the oracle's composition of the same graph.

Decode tolerance: the decoder runs ~30 bf16 convolutions whose GPU and oracle summation orders differ, and the
GPU rounds a conv's output before the residual add (two roundings where the oracle has one), so the RGBA
channels may differ by a few levels: mean |diff| <= 1 level, >= 99 % of channels within 4 levels, alpha exact."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import vae_oracle

pytestmark = pytest.mark.gpu


def _bf(a):
    return O.from_f32(np.asarray(a, np.float32), O.BF16)


def _dev16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev)


def _host16(t):
    return t.cpu().numpy().view(np.uint16)


def _sync():
    torch.cuda.synchronize()


@pytest.mark.parametrize("up", [0, 1])
def test_im2col_exact(dev, up):
    from krea_image_amd import vae
    rng = np.random.default_rng(1)
    H, W, C, ldx, Kpad = 6, 10, 24, 32, 256
    Hin, Win = (H // 2, W // 2) if up else (H, W)
    x = _bf(rng.standard_normal((Hin * Win, ldx)))
    m0, rows = 7, 41
    col = torch.full((rows, Kpad), -1, dtype=torch.int16, device=dev)
    print(f"[vae im2col] up={up} H={H} W={W} C={C} rows [{m0}, {m0 + rows})", flush=True)
    vae.im2col(_dev16(x, dev), ldx, C, H, W, up, m0, rows, col, Kpad)
    _sync()
    img = x[:, :C].reshape(Hin, Win, C)
    if up:
        img = img.repeat(2, axis=0).repeat(2, axis=1)
    imgp = np.pad(img, ((1, 1), (1, 1), (0, 0)))
    ref = np.zeros((rows, Kpad), np.uint16)
    for r in range(rows):
        py, px = divmod(m0 + r, W)
        ref[r, :9 * C] = np.concatenate([imgp[py + t // 3, px + t % 3] for t in range(9)])
    np.testing.assert_array_equal(_host16(col), ref)


# 96 / 192 / 384: the register kernel (4, 8, 16 lanes per pixel); 8 and 104: the generic one
@pytest.mark.parametrize("C,silu", [(96, 1), (96, 0), (192, 1), (384, 0), (384, 1), (8, 1), (104, 1)])
def test_norm_silu(dev, C, silu):
    from krea_image_amd import vae
    rng = np.random.default_rng(C)
    P, ld = 301, C + 64
    x = _bf(rng.standard_normal((P, ld)) * 2)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    y = torch.zeros((P, ld), dtype=torch.int16, device=dev)
    print(f"[vae norm] P={P} C={C} silu={silu}", flush=True)
    vae.norm_silu(_dev16(x, dev), ld, torch.from_numpy(g).to(dev), y, ld, P, C, silu)
    _sync()
    got = O.to_f32(_host16(y)[:, :C], O.BF16)
    ref = O.to_f32(O.vae_norm_silu(x[:, :C].copy(), g, silu), O.BF16)
    assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max()
    assert (_host16(y)[:, C:] == 0).all()  # columns past C untouched


def test_unpack(dev):
    from krea_image_amd import vae
    rng = np.random.default_rng(3)
    H16, W16 = 5, 7
    z = rng.standard_normal((H16 * W16, 64)).astype(np.float32)
    mean, std = rng.standard_normal(16).astype(np.float32), (1 + rng.random(16)).astype(np.float32)
    w, b = (rng.standard_normal((16, 16)) * 0.3).astype(np.float32), rng.standard_normal(16).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    y = torch.empty((4 * H16 * W16, 16), dtype=torch.int16, device=dev)
    print(f"[vae unpack] {H16}x{W16}", flush=True)
    vae.unpack(t(z), t(mean), t(std), t(w), t(b), y, H16, W16)
    _sync()
    got = O.to_f32(_host16(y), O.BF16)
    ref = O.to_f32(O.vae_unpack(z, mean, std, w, b, H16, W16), O.BF16)
    assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max()


# ld % 4 != 0: the three-pass kernel; ld % 4 == 0 and n <= 16384: the one-read kernel (ragged tail, full rows)
@pytest.mark.parametrize("n,ld", [(1, 62), (100, 161), (4099, 4160), (16384, 16384), (13, 16), (16385, 16448)])
def test_softmax(dev, n, ld):
    from krea_image_amd import vae
    rng = np.random.default_rng(n)
    rows = 9
    S = (rng.standard_normal((rows, ld)) * 6).astype(np.float32)
    Pm = torch.zeros((rows, ld), dtype=torch.int16, device=dev)
    print(f"[vae softmax] rows={rows} n={n} ld={ld}", flush=True)
    vae.softmax(torch.from_numpy(S).to(dev), ld, rows, n, 0.05, Pm)
    _sync()
    got = O.to_f32(_host16(Pm), O.BF16)
    ref = O.to_f32(O.vae_softmax(S, n, 0.05), O.BF16)
    assert np.abs(got - ref).max() <= 2 ** -8
    assert (got[:, n:] == 0).all()


def test_conv_out(dev):
    from krea_image_amd import vae
    rng = np.random.default_rng(4)
    H, W, C, ld = 9, 13, 96, 128
    x = _bf(rng.standard_normal((H * W, ld)))
    w = _bf(rng.standard_normal((9 * C, 4)) / np.sqrt(9 * C) * 2)
    b = np.array([0.1, -0.1, 0.0, 1.0], np.float32)
    rgba = torch.empty((H * W, 4), dtype=torch.uint8, device=dev)
    print(f"[vae conv_out] {H}x{W} C={C}", flush=True)
    vae.conv_out(_dev16(x, dev), ld, C, _dev16(w, dev), torch.from_numpy(b).to(dev), rgba, H, W)
    _sync()
    ref = O.vae_conv_out(x[:, :C].copy(), w, b, H, W)
    assert np.abs(rgba.cpu().numpy().astype(np.int32) - ref).max() <= 1


@pytest.fixture(scope="module")
def vae_file(tmp_path_factory, dev):
    from krea_image_amd import qw, vae
    path = str(tmp_path_factory.mktemp("vae") / "vae.qw")
    vae.write_random_vae(path, seed=1)
    f = qw.QwFile(path)
    f.upload()
    yield f
    f.close()


# 2 x 2: 16 mid pixels, keys padded to 64; 4 x 4: 64 pixels, no padding; 24 x 24: 2304 pixels, one query chunk
# by default, three of 768 rows with KH_VAE_QCHUNK (the multi-chunk path of larger images)
@pytest.mark.parametrize("H16,W16,qchunk", [(2, 2, None), (4, 4, None), (3, 5, None), (24, 24, None), (24, 24, 768)])
def test_decode_matches_oracle(dev, vae_file, H16, W16, qchunk, monkeypatch):
    from krea_image_amd import vae
    if qchunk:
        monkeypatch.setenv("KH_VAE_QCHUNK", str(qchunk))
    rng = np.random.default_rng(H16 * 100 + W16)
    z = rng.standard_normal((H16 * W16, 64)).astype(np.float32)
    print(f"[vae decode] latent {H16}x{W16} -> {16 * H16}x{16 * W16} qchunk={qchunk}", flush=True)
    dec = vae.VaeDecoder(vae_file, dev)
    zt = torch.from_numpy(z).to(dev)
    got = dec.decode(zt, H16, W16)
    again = dec.decode(zt, H16, W16)  # the workspace is reused: deterministic, no state carried over
    _sync()
    got, again = got.cpu().numpy(), again.cpu().numpy()
    np.testing.assert_array_equal(got, again)
    ref = vae_oracle.decode(vae_file, z, H16, W16)
    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    print(f"[vae decode] mean |diff| {d[..., :3].mean():.3f}  max {d.max()}  >4: {(d[..., :3] > 4).mean():.4%}")
    assert (got[..., 3] == 255).all()
    assert d[..., :3].mean() <= 1.0
    assert (d[..., :3] <= 4).mean() >= 0.99


def test_decode_rejects_bad_arguments(dev, vae_file):
    from krea_image_amd import kh, vae
    dec = vae.VaeDecoder(vae_file, dev)
    z = torch.zeros((4, 64), device=dev)
    with pytest.raises(kh.KhError):
        dec.decode(z, 0, 4)
    small = torch.empty(1024, dtype=torch.uint8, device=dev)
    lib = vae._bind(kh.load())
    import ctypes
    err = ctypes.create_string_buffer(256)
    rc = lib.kh_vae_decode(kh._stream(), ctypes.c_void_p(vae_file.h), ctypes.c_void_p(z.data_ptr()), 2, 2,
                           ctypes.c_void_p(small.data_ptr()), 1024, ctypes.c_void_p(small.data_ptr()), err, 256)
    assert rc != 0 and b"workspace" in err.value
