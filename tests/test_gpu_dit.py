"""DiT block / forward parity: kh_dit_forward (HIP, C++ layer loop over the C ABI) against the oracle's
restatement of DiT::layer (engine/src/model.mm:369-385) composed from the CPU oracle functions, on seeded
random weights. Tolerance: <= 1.6 % relative L2 per full DiT forward (the reference's accuracy budget,
README.md:121); per block the residual increment is held to the same bound."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, host_int8, rel_l2

pytestmark = pytest.mark.gpu
TOL = 1.6e-2


def small_shapes():
    from krea_image_amd import dit
    base = dit.DitShape(256, 2, 2, 1024, 0, 0, 1, 1, torch.float16, 1)          # baseline-like: GELU, LN, 2-D RoPE
    ref = dit.DitShape(512, 4, 2, 1024, 1, 1, 0, 0, torch.bfloat16, 1)          # reference-like: GQA, gate, SwiGLU
    return {"baseline": base, "reference": ref}


def np16(t):
    return from_dev16(t)


def oracle_layer(shape, L, x, cond, cos, sin):
    dt = O.F16 if shape.dtype == torch.float16 else O.BF16
    D, kvD = shape.dim, shape.kv_heads * 128
    w = lambda W: (host_int8(W), O.I8, np16(W.s), O.F16, W.w.shape[0])  # noqa: E731
    tvec = O.gemv(cond[None].astype(np.float32), *w(L.ada), act=1, bias=L.ada_bias.cpu().numpy())[0]
    mods = O.make_cond(tvec, None, L.n1.cpu().numpy(), L.n2.cpu().numpy())
    h = O.rms_norm(x, mods[0], mods[1], dt, shape.eps, shape.norm_center)
    qkv = O.gemm(0, h, dt, *w(L.qkv))
    qkv, _, _ = O.qk_norm_rope(qkv, dt, L.qn.cpu().numpy(), L.kn.cpu().numpy(), cos, sin, 0, shape.heads, D,
                               shape.kv_heads, shape.eps, 0)
    Q = np.ascontiguousarray(qkv[:, :D])
    K = np.ascontiguousarray(qkv[:, D:D + kvD])
    V = np.ascontiguousarray(qkv[:, D + kvD:D + 2 * kvD])
    G = np.ascontiguousarray(qkv[:, D + 2 * kvD:]) if shape.attn_gate else None
    ao = O.attention(Q, K, V, dt, shape.heads, shape.heads // shape.kv_heads, G=G)
    x1 = x.copy()
    O.gemm(O.EPI["resid_gate"], ao, dt, *w(L.o), C=x1, vec=mods[2])
    h = O.rms_norm(x1, mods[3], mods[4], dt, shape.eps, shape.norm_center)
    mid = O.gemm(O.EPI["swiglu" if shape.mlp == 1 else "gelu"], h, dt, *w(L.up))
    O.gemm(O.EPI["resid_gate"], mid, dt, *w(L.down), C=x1, vec=mods[5])
    return x1


@pytest.mark.parametrize("name", ["baseline", "reference"])
def test_dit_block_matches_oracle(dev, name):
    from krea_image_amd import dit
    shape = small_shapes()[name]
    print(f"[dit block] {name} D={shape.dim} heads={shape.heads}/{shape.kv_heads} ff={shape.ff}", flush=True)
    run = dit.DitRunner(shape, 20, 12, 14, dev, seed=3)
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    run.x.copy_(torch.randn(run.R, shape.dim, generator=g, device=dev))
    x0 = run.x.cpu().numpy()
    run.run_layers()
    torch.cuda.synchronize()
    got = run.x.cpu().numpy()
    ref = oracle_layer(shape, run.layers[0], x0, run.cond.cpu().numpy(), run.cos.cpu().numpy(), run.sin.cpu().numpy())
    err = rel_l2(got - x0, ref - x0)
    print(f"    block increment rel_l2={err:.3e}", flush=True)
    assert np.isfinite(got).all() and err <= TOL


def test_dit_forward_two_layers_matches_oracle(dev):
    from krea_image_amd import dit
    shape = small_shapes()["baseline"]
    shape.layers = 2
    run = dit.DitRunner(shape, 16, 8, 10, dev, seed=5)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    txt = torch.randn(16, shape.dim, generator=g, device=dev)
    z = torch.randn(80, 64, generator=g, device=dev)
    vel = torch.empty_like(z)
    run.forward(txt, z, vel)
    torch.cuda.synchronize()
    # oracle: embed (f32 GEMM in numpy), two layers, head
    x = np.concatenate([txt.cpu().numpy(), z.cpu().numpy() @ run.first_w.cpu().numpy() + run.first_b.cpu().numpy()])
    cond, cos, sin = run.cond.cpu().numpy(), run.cos.cpu().numpy(), run.sin.cpu().numpy()
    for L in run.layers:
        x = oracle_layer(shape, L, x.astype(np.float32), cond, cos, sin)
    hf = O.rms_norm(np.ascontiguousarray(x[16:]), run.fin_mul.cpu().numpy(), run.fin_add.cpu().numpy(), O.F32,
                    shape.eps, shape.norm_center)
    ref = hf.astype(np.float64) @ run.last_w.cpu().numpy() + run.last_b.cpu().numpy()
    err = rel_l2(vel.cpu().numpy(), ref)
    print(f"    forward velocity rel_l2={err:.3e}", flush=True)
    assert err <= TOL


def test_dit_layer_rejects_bad_config(dev):
    from krea_image_amd import dit, kh
    shape = small_shapes()["baseline"]
    shape.heads = 3          # 3 * 128 != 256
    run_shape = dit.DitShape(256, 2, 2, 1024, 0, 0, 1, 1, torch.float16, 1)
    run = dit.DitRunner(run_shape, 4, 4, 4, dev)
    run._cfg = shape.config()
    with pytest.raises(kh.KhError, match="heads"):
        run.run_layers()
