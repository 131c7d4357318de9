"""kh_vae_conv3x3: the 3 x 3 convolution as an implicit GEMM (the GEMM's activation DMA gathers each
(tap, channel) chunk from the image, or a zero chunk for padding) against (a) the oracle's direct
convolution (engine/kernels/vae.metal:5-128 semantics) and (b) bitwise, the explicit im2col panel
(kh_vae_im2col) fed to kh_gemm with the same weights: both multiply the same values in the same K order.
Shapes cover C = 8 .. 384, nearest-2x upsampling, ragged pixel counts, a stream-K launch and a 192-wide
tile launch."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gemm_ws

pytestmark = pytest.mark.gpu

CASES = [  # H, W (output), C, N, up
    (6, 10, 16, 64, 0),      # conv_in-like: 9 C = 144 -> K 192 (zero K padding)
    (12, 20, 96, 128, 1),    # C = 96: K steps straddle taps; upsampled input 6 x 10
    (30, 34, 192, 192, 0),   # ragged: 1020 pixels
    (64, 80, 384, 256, 0),   # 20 tiles x 54 K steps: stream-K
    (128, 120, 16, 768, 0),  # 60 x 3 tiles of 256 -> 60 x 4 tiles of 192
]


def _bf(a):
    return O.from_f32(np.asarray(a, np.float32), O.BF16)


def _dev16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


@pytest.mark.parametrize("H,W,C,N,up", CASES)
def test_conv3x3_implicit(dev, H, W, C, N, up):
    from krea_image_amd import kh, vae
    print(f"[vae conv3x3] H={H} W={W} C={C} N={N} up={up}", flush=True)
    rng = np.random.default_rng(H * 1000 + C)
    Hin, Win = (H // 2, W // 2) if up else (H, W)
    ldx = C + 8 if C % 64 else C  # a row stride wider than C on some cases
    x = _bf(rng.standard_normal((Hin * Win, ldx)))
    K = (9 * C + 63) // 64 * 64
    w = np.zeros((K, N), np.uint16)
    w[:9 * C] = _bf(rng.standard_normal((9 * C, N)) / np.sqrt(9 * C))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    xd, wd, bd = _dev16(x, dev), _dev16(w, dev), torch.from_numpy(bias).to(dev)
    P = H * W
    y = torch.empty(P, N, dtype=torch.bfloat16, device=dev)
    vae.conv3x3(xd, ldx, C, H, W, up, wd, K, N, bd, y, N, ws=gemm_ws(dev))
    col = torch.empty(P, K, dtype=torch.bfloat16, device=dev)
    vae.im2col(xd, ldx, C, H, W, up, 0, P, col, K)
    y2 = torch.empty(P, N, dtype=torch.bfloat16, device=dev)
    kh.gemm("bias16", col, kh.Weight(wd), y2, P, N, K, K, N, N, bd, gemm_ws(dev))
    torch.cuda.synchronize()
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got, y2.view(torch.int16).cpu().numpy().view(np.uint16))
    # fused residual: round16(round16(conv + bias) + res), bit for bit
    R = _bf(rng.standard_normal((P, N)))
    y3 = torch.empty(P, N, dtype=torch.bfloat16, device=dev)
    vae.conv3x3(xd, ldx, C, H, W, up, wd, K, N, bd, y3, N, res=_dev16(R, dev), ws=gemm_ws(dev))
    torch.cuda.synchronize()
    want = O.from_f32(O.to_f32(got, O.BF16) + O.to_f32(R, O.BF16), O.BF16)
    np.testing.assert_array_equal(y3.view(torch.int16).cpu().numpy().view(np.uint16), want)
    ref = O.vae_conv(x[:, :C], H, W, w[:9 * C], bias, N, ks=3, up=up)
    g, r = O.to_f32(got, O.BF16), O.to_f32(ref, O.BF16)
    rel = float(np.linalg.norm(g - r) / np.linalg.norm(r))
    assert rel < 5e-3, rel


def test_conv3x3_rejects_bad_arguments(dev):
    from krea_image_amd import kh, vae
    x = torch.zeros(64, 24, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(256, 64, dtype=torch.bfloat16, device=dev)
    b = torch.zeros(64, device=dev)
    y = torch.empty(64, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(kh.KhError, match="K=192"):
        vae.conv3x3(x, 24, 24, 8, 8, 0, w, 192, 64, b, y, 64)   # K < 9 C = 216
    with pytest.raises(kh.KhError, match="multiple of 8"):
        vae.conv3x3(x, 24, 20, 8, 8, 0, w, 256, 64, b, y, 64)   # C % 8
    with pytest.raises(kh.KhError, match="even"):
        vae.conv3x3(x, 24, 24, 7, 8, 1, w, 256, 64, b, y, 64)   # odd upsampled size


@pytest.mark.parametrize("H,W,C,Cout", [(5, 7, 16, 96), (12, 20, 384, 192), (30, 34, 192, 96), (16, 24, 96, 384)])
def test_conv_up2_subpixel(dev, H, W, C, Cout):
    """The upsampling conv as four sub-pixel 2x2 convs (the reference's mode 2): folded weights bit-exact
    against the oracle's restatement, the conv against the oracle's sub-pixel conv and, to the folding's
    bf16 rounding, against the direct 3x3 conv of the upsampled image."""
    from krea_image_amd import vae
    print(f"[vae conv_up2] H={H} W={W} C={C} Cout={Cout}", flush=True)
    rng = np.random.default_rng(7 * H + C)
    Np = (Cout + 63) // 64 * 64
    x = _bf(rng.standard_normal((H * W, C)))
    w = _bf(rng.standard_normal((9 * C, Cout)) / np.sqrt(9 * C))
    bias = (rng.standard_normal(Cout) * 0.1).astype(np.float32)
    K = (4 * C + 63) // 64 * 64
    wd, bd, xd = _dev16(w, dev), torch.from_numpy(bias).to(dev), _dev16(x, dev)
    w2 = torch.empty(K, 4 * Np, dtype=torch.bfloat16, device=dev)
    b4 = torch.empty(4 * Np, device=dev)
    vae.subpix_weights(wd, C, Cout, w2, K, Np, bd, b4)
    y = torch.empty(4 * H * W, Np, dtype=torch.bfloat16, device=dev)
    vae.conv_up2(xd, C, C, H, W, w2, K, Np, b4, y, Np, ws=gemm_ws(dev))
    torch.cuda.synchronize()
    ref_w2 = O.vae_subpix_weights(w, C, Cout)
    got_w2 = w2.view(torch.int16).cpu().numpy().view(np.uint16)
    for ph in range(4):
        np.testing.assert_array_equal(got_w2[:4 * C, ph * Np:ph * Np + Cout], ref_w2[:, ph * Cout:(ph + 1) * Cout])
        assert not got_w2[:, ph * Np + Cout:(ph + 1) * Np].any() and not got_w2[4 * C:].any()
    np.testing.assert_array_equal(b4.cpu().numpy().reshape(4, Np)[:, :Cout], np.tile(bias, (4, 1)))
    g = O.to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)[:, :Cout], O.BF16)
    ref = O.to_f32(O.vae_conv_up2(x, H, W, ref_w2, bias, Cout), O.BF16)
    assert np.linalg.norm(g - ref) / np.linalg.norm(ref) < 5e-3
    direct = O.to_f32(O.vae_conv(x, 2 * H, 2 * W, w, bias, Cout, ks=3, up=1), O.BF16)
    assert np.linalg.norm(g - direct) / np.linalg.norm(direct) < 2e-2
