"""kh_euler_step / kh_cfg_combine (HIP, through the C ABI) bitwise against the oracle, on ragged sizes and on
unaligned views (the scalar kernel), and the DiT runner's denoising loop (forward + Euler step per noise
level) against the same loop with the oracle's update applied on the host, bit for bit (every op of the
forward sums in a fixed order)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import rel_l2
from tests.test_gpu_dit import small_shapes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,off", [(1, 0), (5, 0), (4096, 0), (1000003, 0), (1003, 1)])
def test_euler_step_bitwise(dev, n, off):
    from krea_image_amd import kh
    rng = np.random.default_rng(n + off)
    z = rng.standard_normal(n + off).astype(np.float32)
    v = rng.standard_normal(n + off).astype(np.float32)
    dt = np.float32(-0.0371)
    print(f"[euler] n={n} off={off}", flush=True)
    zd = torch.from_numpy(z).to(dev)
    kh.euler_step(zd[off:], torch.from_numpy(v).to(dev)[off:], float(dt))
    torch.cuda.synchronize()
    got = zd.cpu().numpy()
    np.testing.assert_array_equal(got[off:], O.euler_step(z[off:], v[off:], dt))
    np.testing.assert_array_equal(got[:off], z[:off])


@pytest.mark.parametrize("n,off", [(7, 0), (65536, 0), (70001, 3)])
def test_cfg_combine_bitwise(dev, n, off):
    from krea_image_amd import kh
    rng = np.random.default_rng(7 * n + off)
    vc = rng.standard_normal(n + off).astype(np.float32)
    vn = rng.standard_normal(n + off).astype(np.float32)
    print(f"[cfg] n={n} off={off}", flush=True)
    vcd = torch.from_numpy(vc).to(dev)
    kh.cfg_combine(vcd[off:], torch.from_numpy(vn).to(dev)[off:], 4.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(vcd.cpu().numpy()[off:], O.cfg_combine(vc[off:], vn[off:], np.float32(4.0)))


def test_sampler_rejects(dev):
    from krea_image_amd import kh
    z = torch.zeros(8, device=dev)
    with pytest.raises(kh.KhError, match="differ"):
        kh.euler_step(z, torch.zeros(9, device=dev), 0.1)
    with pytest.raises(kh.KhError, match="float32"):
        kh.cfg_combine(z.half(), z.half(), 1.0)


def test_denoise_loop_matches_host_updates(dev):
    from krea_image_amd import dit, kh
    shape = small_shapes()["baseline"]
    shape.layers = 2
    run = dit.DitRunner(shape, 16, 8, 10, dev, seed=6)
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    txt = torch.randn(16, shape.dim, generator=g, device=dev)
    z0 = torch.randn(80, 64, generator=g, device=dev)
    sig = kh.sigmas(3)
    print("[denoise] 3 steps, 2 layers", flush=True)
    z = run.denoise(txt, z0.clone(), sig)
    # the same loop, the update done by the oracle on the host
    zr = z0.clone()
    vel = torch.empty_like(zr)
    for i in range(3):
        run.forward(txt, zr, vel)
        torch.cuda.synchronize()
        upd = O.euler_step(zr.cpu().numpy(), vel.cpu().numpy(), np.float32(float(sig[i + 1]) - float(sig[i])))
        zr = torch.from_numpy(upd).to(dev)
    torch.cuda.synchronize()
    assert torch.isfinite(z).all()
    # bitwise: every op of the forward sums in a fixed order, so two forwards of the same input agree exactly,
    # and the update is the oracle's
    assert torch.equal(z.cpu(), zr.cpu())
    assert not torch.equal(z.cpu(), z0.cpu())


def test_denoise_loop_with_guidance(dev):
    """pipeline.mm:300-316 with classifier-free guidance: the negative prompt's forward (a sibling runner at
    another text length over the same weights), kh_cfg_combine, then the Euler step; against the same loop
    with both updates done by the oracle on the host (bitwise: the forward is deterministic)."""
    from krea_image_amd import dit, kh
    shape = small_shapes()["baseline"]
    shape.layers = 2
    run = dit.DitRunner(shape, 16, 8, 10, dev, seed=9)
    neg = run.sibling(8)
    g = torch.Generator(device=dev)
    g.manual_seed(10)
    txt = torch.randn(16, shape.dim, generator=g, device=dev)
    ntxt = torch.randn(8, shape.dim, generator=g, device=dev)
    z0 = torch.randn(80, 64, generator=g, device=dev)
    sig = kh.sigmas(2)
    print("[denoise cfg] 2 steps, scale 3.5", flush=True)
    z = run.denoise(txt, z0.clone(), sig, neg=neg, ntxt=ntxt, cfg_scale=3.5)
    zr = z0.clone()
    v, v2 = torch.empty_like(zr), torch.empty_like(zr)
    for i in range(2):
        neg.forward(ntxt, zr, v2)
        run.forward(txt, zr, v)
        torch.cuda.synchronize()
        vc = O.cfg_combine(v.cpu().numpy(), v2.cpu().numpy(), np.float32(3.5))
        upd = O.euler_step(zr.cpu().numpy(), vc, np.float32(float(sig[i + 1]) - float(sig[i])))
        zr = torch.from_numpy(upd).to(dev)
    torch.cuda.synchronize()
    assert torch.isfinite(z).all()
    assert torch.equal(z.cpu(), zr.cpu())
    # guidance changes the result
    zn = run.denoise(txt, z0.clone(), sig)
    assert rel_l2((zn - z0).cpu().numpy(), (z - z0).cpu().numpy()) > 1e-3
