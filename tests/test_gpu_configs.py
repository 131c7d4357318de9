"""BASELINE configs[2..4] at their real workloads, on the GPU, checked against the oracle on row / head subsets
and by size-independent properties:
  configs[2]  joint attention, 4096 image + 512 text tokens = 4608, 24 heads x 128 (the launch with 432
              workgroups, whose XCD remap runs), three heads (first, middle, last) on 96 query rows;
  configs[3]  one DiT block at D = 3072, R = 4608 (adaLN, LayerNorm, QKV, RMS q/k norm + 2-D RoPE, joint
              attention, O + gated residual, GELU MLP + gated residual): the oracle runs the QKV projection on
              every row (keys and values) and the rest on 96 rows; residual increment <= 1.6 % relative L2;
  configs[4]  the full 71-block step at 1536 / 4608 / 8704 rows: bitwise repeatable, bitwise equal to a chain of
              single-layer kh_dit_layer_forward calls, finite; at 4608 rows the first and the last block against
              the oracle as in configs[3].
engine/src/model.mm:369-385 (DiT::layer), 519-538 (run_layers / forward); engine/kernels/attention.metal."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, host_int8, rel_l2

pytestmark = pytest.mark.gpu
TOL_BLOCK = 1.6e-2
TOL_ATTN = 5e-3


def _rows(R, T, n=96, seed=0):
    """Query rows to check: the first and last text and image rows plus a seeded spread."""
    rng = np.random.default_rng(seed)
    fixed = [0, T - 1, T, R - 1]
    rest = rng.choice(np.setdiff1d(np.arange(R), fixed), n - len(fixed), replace=False)
    return np.sort(np.concatenate([fixed, rest]))


def test_config2_joint_attention_4608_24_heads(dev):
    from krea_image_amd import kh
    T, Hh, Ww, heads = 512, 64, 64, 24
    R, D = T + Hh * Ww, heads * 128
    print(f"[configs[2]] attention R={R} heads={heads} (fp16, RMS q/k norm + 2-D RoPE theta 1e4)", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(20)
    qkv = torch.randn(R, 3 * D, generator=g, device=dev).to(torch.float16)
    c, s = kh.rope_tables(T, Hh, Ww, 1)
    ones = torch.ones(128, device=dev)
    kh.qk_norm_rope(qkv, ones, ones, c.to(dev), s.to(dev), R, 3 * D, 0, heads, D, heads, 1e-6, 0)
    out = torch.empty(R, D, dtype=torch.float16, device=dev)
    kh.attention(qkv, qkv[:, D:], qkv[:, 2 * D:], out, R, R, heads, 3 * D, 3 * D, 3 * D, D)
    torch.cuda.synchronize()
    host = from_dev16(qkv)
    got = from_dev16(out)
    rows = _rows(R, T, seed=21)
    for h in (0, heads // 2, heads - 1):
        Q = np.ascontiguousarray(host[rows, 128 * h:128 * h + 128])
        K = np.ascontiguousarray(host[:, D + 128 * h:D + 128 * h + 128])
        V = np.ascontiguousarray(host[:, 2 * D + 128 * h:2 * D + 128 * h + 128])
        ref = O.to_f32(O.attention(Q, K, V, O.F16, 1), O.F16)
        err = rel_l2(O.to_f32(got[rows, 128 * h:128 * h + 128], O.F16), ref)
        print(f"    head {h}: rel_l2={err:.3e}", flush=True)
        assert err <= TOL_ATTN


def oracle_block_rows(shape, L, x, cond, cos, sin, rows):
    """DiT::layer (model.mm:369-385) as the oracle composes it, with the QKV projection, q / k norm and RoPE on
    every row (the keys and values) and the rest on `rows` only (rows are independent there). Returns the
    residual stream at `rows` after the block."""
    dt = O.F16 if shape.dtype == torch.float16 else O.BF16
    D, kvD = shape.dim, shape.kv_heads * 128

    def w(W):
        return host_int8(W), O.I8, from_dev16(W.s), O.F16, W.w.shape[0]

    tvec = O.gemv(cond[None].astype(np.float32), *w(L.ada), act=1, bias=L.ada_bias.cpu().numpy())[0]
    mods = O.make_cond(tvec, None, L.n1.cpu().numpy(), L.n2.cpu().numpy())
    h = O.rms_norm(x, mods[0], mods[1], dt, shape.eps, shape.norm_center)
    qkv = O.gemm(0, h, dt, *w(L.qkv))
    qkv, _, _ = O.qk_norm_rope(qkv, dt, L.qn.cpu().numpy(), L.kn.cpu().numpy(), cos, sin, 0, shape.heads, D,
                               shape.kv_heads, shape.eps, 0)
    Q = np.ascontiguousarray(qkv[rows, :D])
    K = np.ascontiguousarray(qkv[:, D:D + kvD])
    V = np.ascontiguousarray(qkv[:, D + kvD:D + 2 * kvD])
    ao = O.attention(Q, K, V, dt, shape.heads, shape.heads // shape.kv_heads)
    x1 = np.ascontiguousarray(x[rows])
    O.gemm(O.EPI["resid_gate"], ao, dt, *w(L.o), C=x1, vec=mods[2])
    h = O.rms_norm(x1, mods[3], mods[4], dt, shape.eps, shape.norm_center)
    mid = O.gemm(O.EPI["gelu"], h, dt, *w(L.up))
    O.gemm(O.EPI["resid_gate"], mid, dt, *w(L.down), C=x1, vec=mods[5])
    return x1


def test_config3_one_block_3072_4608(dev):
    from krea_image_amd import dit
    shape = dit.baseline_shape(layers=1)
    T, Hh, Ww = 512, 64, 64
    print(f"[configs[3]] one block D={shape.dim} R={T + Hh * Ww}", flush=True)
    run = dit.DitRunner(shape, T, Hh, Ww, dev, seed=30)
    g = torch.Generator(device=dev)
    g.manual_seed(31)
    run.x.copy_(torch.randn(run.R, shape.dim, generator=g, device=dev))
    x0 = run.x.cpu().numpy()
    run.run_layers()
    torch.cuda.synchronize()
    got = run.x.cpu().numpy()
    rows = _rows(run.R, T, seed=32)
    ref = oracle_block_rows(shape, run.layers[0], x0, run.cond.cpu().numpy(), run.cos.cpu().numpy(),
                            run.sin.cpu().numpy(), rows)
    err = rel_l2(got[rows] - x0[rows], ref - x0[rows])
    print(f"    block increment rel_l2={err:.3e} ({len(rows)} rows)", flush=True)
    assert np.isfinite(got).all() and err <= TOL_BLOCK


@pytest.fixture(scope="module")
def step_layers(dev):
    """71 random-init blocks of the configs' 12B-class DiT (12.06 B int8 parameters, ~12.1 GB resident)."""
    from krea_image_amd import dit
    shape = dit.baseline_shape(layers=71)
    gen = torch.Generator(device=dev)
    gen.manual_seed(40)
    layers = [dit.random_layer(shape, gen, dev) for _ in range(shape.layers)]
    yield shape, layers
    del layers
    torch.cuda.empty_cache()


def _layer_chain(run):
    """The blocks as single kh_dit_layer_forward calls (the C ABI's one-layer entry point), in order."""
    from krea_image_amd import kh
    lib = kh.load()
    err = ctypes.create_string_buffer(512)
    size = ctypes.sizeof(kh.DitLayerC)
    for i in range(len(run.layers)):
        lp = ctypes.cast(ctypes.addressof(run._layers_c) + i * size, ctypes.POINTER(kh.DitLayerC))
        kh._check(lib.kh_dit_layer_forward(kh._stream(), ctypes.byref(run._cfg), lp, ctypes.byref(run._state), run.R,
                                           err, 512), err)


@pytest.mark.parametrize("grid", [(32, 32), (64, 64), (64, 128)], ids=["1024", "4096", "8192"])
def test_config4_full_step(dev, step_layers, grid):
    from krea_image_amd import dit
    shape, layers = step_layers
    T = 512
    run = dit.DitRunner(shape, T, grid[0], grid[1], dev, seed=41, layers=layers)
    print(f"[configs[4]] 71-block step R={run.R}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    txt = torch.randn(T, shape.dim, generator=g, device=dev)
    z = torch.randn(grid[0] * grid[1], 64, generator=g, device=dev)
    v1, v2 = torch.empty_like(z), torch.empty_like(z)
    run.forward(txt, z, v1)
    x1 = run.x.clone()
    run.forward(txt, z, v2)
    torch.cuda.synchronize()
    assert torch.isfinite(v1).all() and torch.isfinite(x1).all()
    assert torch.equal(v1, v2) and torch.equal(x1, run.x), "the step is not bitwise repeatable"
    # the same blocks as a chain of single-layer calls from the same embedded input
    run.x[:T].copy_(txt)
    from krea_image_amd import kh
    kh.gemm_f32(z, run.first_w, run.x[T:], z.shape[0], shape.dim, 64, 64, shape.dim, shape.dim, 1, run.first_b)
    _layer_chain(run)
    torch.cuda.synchronize()
    assert torch.equal(x1, run.x), "kh_dit_forward differs from the chain of kh_dit_layer_forward calls"
    if run.R != 4608:
        return
    # first and last block at full width against the oracle (96 rows)
    rows = _rows(run.R, T, seed=43)
    cond, cos, sin = run.cond.cpu().numpy(), run.cos.cpu().numpy(), run.sin.cpu().numpy()
    for li in (0, len(layers) - 1):
        run.x.normal_(generator=g)
        x0 = run.x.cpu().numpy()
        run.run_layers(li, li + 1)
        torch.cuda.synchronize()
        got = run.x.cpu().numpy()
        ref = oracle_block_rows(shape, layers[li], x0, cond, cos, sin, rows)
        err = rel_l2(got[rows] - x0[rows], ref - x0[rows])
        print(f"    block {li}: increment rel_l2={err:.3e}", flush=True)
        assert err <= TOL_BLOCK
