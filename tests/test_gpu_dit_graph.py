"""The DiT step replayed from a HIP graph (DitRunner.capture: torch.cuda.CUDAGraph around forward, i.e. the embed,
kh_dit_forward's per-layer launches and the head) against eager forward on the same inputs. The graph holds the
same kernel launches, so every replay must be bitwise equal to the eager step. Each replay follows eager work
and a synchronisation and sees new inputs written into the captured tensors, and every replay is checked, so a
graph node that only works on its first replay (or ignores new inputs) fails here. Two shapes: baseline-like
(GELU, LayerNorm, per-layer adaLN GEMV) and reference-like (GQA, gate, SwiGLU, group-128 int8, mod tables), at
row counts where the GEMMs run stream-K in the runner's workspace."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _shapes():
    from krea_image_amd import dit
    base = dit.DitShape(256, 2, 2, 1024, 0, 0, 1, 1, torch.float16, 2)
    ref = dit.DitShape(512, 4, 2, 1024, 1, 1, 0, 0, torch.bfloat16, 2, eps=1e-5, weight_group=128)
    return {"baseline": base, "reference": ref}


@pytest.mark.parametrize("name", ["baseline", "reference"])
def test_graph_replay_equals_eager(dev, name):
    from krea_image_amd import dit
    shape = _shapes()[name]
    T, Hh, Ww = 40, 12, 16
    print(f"[dit graph] {name} D={shape.dim} layers={shape.layers} R={T + Hh * Ww}", flush=True)
    run = dit.DitRunner(shape, T, Hh, Ww, dev, seed=60)
    g = torch.Generator(device=dev)
    g.manual_seed(61)
    txt = torch.randn(T, shape.dim, generator=g, device=dev)
    z = torch.randn(Hh * Ww, 64, generator=g, device=dev)
    vel = torch.empty_like(z)
    graph = run.capture(txt, z, vel)
    for i in range(3):
        txt.copy_(torch.randn(T, shape.dim, generator=g, device=dev))
        z.copy_(torch.randn(Hh * Ww, 64, generator=g, device=dev))
        ref = torch.empty_like(vel)
        run.forward(txt, z, ref)             # eager, on the same inputs
        torch.cuda.synchronize()
        vel.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(vel, ref), f"replay {i} differs from the eager step"
    del graph, run
    torch.cuda.empty_cache()
