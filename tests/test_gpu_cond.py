"""The step's timestep conditioning on the device (kh_conditioning: Conditioning::get / compute,
engine/src/model.mm:545-591) from a cond.qw in the converter's layout (tools/convert.py:287-308), the head's
final-norm vectors (kh_make_fin, model.mm:340-346), and a guided denoising loop whose conditioning changes every
step (both passes see the step's conditioning, engine/src/pipeline.mm:304-310).
Tolerances: table hits are bitwise copies; the computed MLP is f32 end to end, <= 1e-5 relative L2 against the
oracle's composition (oracle.conditioning)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import rel_l2

pytestmark = pytest.mark.gpu
BASE = [1.0, 0.9166, 0.8044, 0.6582, 0.4742, 0.2697, 0.1005, 0.0211]
FAST = [1.0, 0.8044, 0.4742, 0.1005]


@pytest.fixture(scope="module")
def cond_file(tmp_path_factory):
    from krea_image_amd import qw
    path = str(tmp_path_factory.mktemp("cond") / "cond.qw")
    qw.write_random_cond(path, 256, BASE, FAST, seed=21)
    f = qw.QwFile(path)
    f.upload()
    yield f
    f.close()


def _oracle_compute(f, sigma):
    a = f.array
    return O.conditioning(sigma, a("tmlp1.w"), a("tmlp1.b"), a("tmlp2.w"), a("tmlp2.b"), a("tproj.w"), a("tproj.b"))


@pytest.mark.parametrize("sigma", [0.55, 0.0, 1.0 - 1e-7, 0.9166 + 1e-4])
def test_conditioning_computed_matches_oracle(dev, cond_file, sigma):
    D = 256
    print(f"[conditioning compute] sigma={sigma}", flush=True)
    t, tvec, work = torch.empty(D, device=dev), torch.empty(6 * D, device=dev), torch.empty(256 + D, device=dev)
    outs = []
    for _ in range(2):
        hit = cond_file.conditioning(False, sigma, t, tvec, work)
        torch.cuda.synchronize()
        assert not hit
        outs.append((t.cpu().clone(), tvec.cpu().clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    rt, rtv = _oracle_compute(cond_file, sigma)
    assert rel_l2(outs[0][0].numpy(), rt) <= 1e-5
    assert rel_l2(outs[0][1].numpy(), rtv) <= 1e-5


@pytest.mark.parametrize("fast,idx", [(False, 0), (False, 5), (True, 2)])
def test_conditioning_table_hit_copies_row(dev, cond_file, fast, idx):
    D = 256
    tag = "fast." if fast else "base."
    sigma = float(cond_file.array(tag + "sigma")[idx])
    print(f"[conditioning table] {tag} sigma={sigma}", flush=True)
    t, tvec = torch.full((D,), 7.0, device=dev), torch.full((6 * D,), 7.0, device=dev)
    hit = cond_file.conditioning(fast, sigma, t, tvec, torch.empty(256 + D, device=dev))
    torch.cuda.synchronize()
    assert hit
    assert np.array_equal(t.cpu().numpy(), cond_file.array(tag + "t")[idx])
    assert np.array_equal(tvec.cpu().numpy(), cond_file.array(tag + "tvec")[idx])
    # the table holds values unrelated to the MLP: a hit is not what compute would give
    assert rel_l2(t.cpu().numpy(), _oracle_compute(cond_file, sigma)[0]) > 0.1


def test_conditioning_fast_without_match_fails(dev, cond_file):
    from krea_image_amd import kh
    D = 256
    t, tvec = torch.empty(D, device=dev), torch.empty(6 * D, device=dev)
    with pytest.raises(kh.KhError, match="not in the fast schedule"):
        cond_file.conditioning(True, 0.55, t, tvec, torch.empty(256 + D, device=dev))
    with pytest.raises(kh.KhError, match="256 \\+ D"):
        cond_file.conditioning(False, 0.55, t, tvec, torch.empty(16, device=dev))


def test_conditioning_tables_only_file(dev, tmp_path):
    """Conditioning::get reads only the schedule tables (model.mm:545-569): a cond file holding just the tables
    serves a listed sigma (bitwise row copy, D from the table's shape) and reports a missing MLP on a miss."""
    from krea_image_amd import kh, qw
    D = 128
    rng = np.random.default_rng(22)
    specs = [sp for sp in qw.cond_specs(D, len(BASE), len(FAST)) if sp[0].startswith(("base.", "fast."))]
    path = str(tmp_path / "tables.qw")
    w = qw.QwWriter(path, specs, {"model": "tables-only"})
    rows = {}
    for tag, sig in (("base", BASE), ("fast", FAST)):
        w.write(tag + ".sigma", np.asarray(sig, np.float32))
        rows[tag] = (rng.standard_normal((len(sig), D), dtype=np.float32),
                     rng.standard_normal((len(sig), 6 * D), dtype=np.float32))
        w.write(tag + ".t", rows[tag][0])
        w.write(tag + ".tvec", rows[tag][1])
    w.close()
    print("[conditioning tables-only]", flush=True)
    with qw.QwFile(path) as f:
        f.upload()
        t, tvec = torch.empty(D, device=dev), torch.empty(6 * D, device=dev)
        assert f.conditioning(True, float(np.float32(FAST[1])), t, tvec, None)
        torch.cuda.synchronize()
        assert np.array_equal(t.cpu().numpy(), rows["fast"][0][1])
        assert np.array_equal(tvec.cpu().numpy(), rows["fast"][1][1])
        with pytest.raises(kh.KhError, match="tmlp1.w"):
            f.conditioning(False, 0.55, t, tvec, torch.empty(256 + D, device=dev))


def test_make_fin(dev):
    from krea_image_amd import kh
    rng = np.random.default_rng(4)
    D = 6144
    t, nf = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    lin = rng.standard_normal((2, D)).astype(np.float32)
    fin = torch.empty(2, D, device=dev)
    td = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    kh.make_fin(td(t), td(lin), td(nf), D, fin)
    torch.cuda.synchronize()
    assert np.array_equal(fin.cpu().numpy(), O.make_fin(t, lin, nf))


def test_guided_denoise_with_per_step_conditioning(dev, tmp_path, cond_file):
    """A QwDit denoising loop with guidance, before_step = set_sigma(cond, sig[i]) (a different t / tvec every
    step). The negative pass's sibling shares the conditioning tensors, so its result is bitwise the loop run
    with an independent negative-prompt runner whose conditioning is copied from the positive one each step
    (what pipeline.mm:304-310 does by passing conds[i] to both passes)."""
    from krea_image_amd import dit, kh, qw
    path = str(tmp_path / "dit_q8.qw")
    qw.write_random_dit(path, D=256, kv_heads=1, FF=512, layers=2, quant=True, seed=17)
    print("[guided denoise, per-step conditioning] D=256 layers=2 steps=3", flush=True)
    sig = [1.0, 0.55, 0.2697, 0.0]  # step 0 and 2 from the base table, step 1 computed
    with qw.QwFile(path) as f:
        f.upload()
        run = dit.QwDit(f, 16, 8, 10, dev)
        neg = run.sibling(8)
        assert neg.tvec.data_ptr() == run.tvec.data_ptr() and neg.fin.data_ptr() == run.fin.data_ptr()
        g = torch.Generator(device=dev)
        g.manual_seed(3)
        txt = torch.randn(16, 256, generator=g, device=dev)
        ntxt = torch.randn(8, 256, generator=g, device=dev)
        z0 = torch.randn(80, 64, generator=g, device=dev)
        hits = []
        z = run.denoise(txt, z0.clone(), sig, before_step=lambda i: hits.append(run.set_sigma(cond_file, sig[i])),
                        neg=neg, ntxt=ntxt, cfg_scale=2.5)
        assert hits == [True, False, True]
        # the same loop with an independent negative runner, conditioned by explicit copies
        ind = dit.DitRunner(run.shape, 8, 8, 10, dev, layers=run.layers)
        for name in ("first_w", "first_b", "last_w", "last_b"):
            setattr(ind, name, getattr(run, name))
        zr = z0.clone()
        v, v2 = torch.empty_like(zr), torch.empty_like(zr)
        for i in range(3):
            run.set_sigma(cond_file, sig[i])
            ind.tvec.copy_(run.tvec)
            ind.fin.copy_(run.fin)
            ind.forward(ntxt, zr, v2)
            run.forward(txt, zr, v)
            kh.cfg_combine(v, v2, 2.5)
            kh.euler_step(zr, v, float(sig[i + 1]) - float(sig[i]))
        torch.cuda.synchronize()
        assert torch.isfinite(z).all()
        assert torch.equal(z.cpu(), zr.cpu())
        # the final-norm vectors are those of the last step's t
        t_last = torch.empty(256, device=dev)
        cond_file.conditioning(False, sig[2], t_last, torch.empty(6 * 256, device=dev), torch.empty(512, device=dev))
        torch.cuda.synchronize()
        fin = O.make_fin(t_last.cpu().numpy(), f.array("last.mod"), f.array("last.n"))
        assert np.array_equal(run.fin.cpu().numpy(), fin)
