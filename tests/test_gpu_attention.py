"""Parity of kh_attention (HIP, through the C ABI) against the CPU oracle's restatement of attention_d128 and
against the numpy golden fixture. Tolerance: <= 0.5 % relative L2 (P and O are rounded to the 16-bit type,
the oracle uses the exact running max and the kernel the lazy one, so the two differ by a few 16-bit ulps)."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, randn16, rel_l2, to_dev16

pytestmark = pytest.mark.gpu
TOL = 5e-3


def run(dev, dtype, Lq, Lk, heads, group=1, causal=0, q_pos0=0, gate=False, big=False, seed=0, scale=1.0,
        extra_cols=0):
    from krea_image_amd import kh
    print(f"[attn case] dtype={dtype} Lq={Lq} Lk={Lk} heads={heads} group={group} causal={causal} "
          f"q_pos0={q_pos0} gate={gate} big={big} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    kvh = heads // group
    ldq = heads * 128 + extra_cols
    Q = randn16(rng, (Lq, ldq), dtype, scale)
    K = randn16(rng, (Lk, kvh * 128), dtype, scale)
    V = randn16(rng, (Lk, kvh * 128), dtype)
    G = randn16(rng, (Lq, heads * 128), dtype) if gate else None
    QB = (rng.standard_normal((Lq, heads)) * 3).astype(np.float32) if big else None
    KB = (rng.standard_normal((Lk, kvh)) * 3).astype(np.float32) if big else None
    Od = torch.zeros(Lq, heads * 128, dtype=torch.float16 if dtype == O.F16 else torch.bfloat16, device=dev)
    kh.attention(to_dev16(Q, dtype, dev), to_dev16(K, dtype, dev), to_dev16(V, dtype, dev), Od, Lq, Lk, heads,
                 ldq, kvh * 128, kvh * 128, heads * 128, group, bool(causal), q_pos0,
                 None if G is None else to_dev16(G, dtype, dev), heads * 128 if gate else 0,
                 None if QB is None else torch.from_numpy(QB).to(dev), None if KB is None else torch.from_numpy(KB).to(dev))
    torch.cuda.synchronize()
    got = O.to_f32(from_dev16(Od), dtype)
    ref = O.to_f32(O.attention(np.ascontiguousarray(Q[:, :heads * 128]), K, V, dtype, heads, group, causal, q_pos0,
                               G, QB, KB), dtype)
    err = rel_l2(got, ref)
    print(f"    rel_l2={err:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL, f"rel L2 {err:.3e}"


@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
def test_attention_basic(dev, dtype):
    run(dev, dtype, 256, 256, 2)


@pytest.mark.parametrize("Lq,Lk", [(1, 1), (37, 100), (130, 64), (200, 517)])
def test_attention_ragged(dev, Lq, Lk):
    run(dev, O.F16, Lq, Lk, 2, seed=Lq + Lk)


@pytest.mark.parametrize("dtype,heads,group", [(O.F16, 4, 4), (O.BF16, 8, 8)])
def test_attention_mqa(dev, dtype, heads, group):
    """One K / V head shared by every query head (group = heads)."""
    run(dev, dtype, 150, 333, heads, group=group, gate=True, seed=11)


@pytest.mark.parametrize("Lq,Lk", [(1, 4608), (3, 4096), (64, 4097)])
def test_attention_few_queries_many_keys(dev, Lq, Lk):
    """A handful of queries over a long key range (one partly filled workgroup, 64 .. 73 key blocks, a ragged
    last block)."""
    run(dev, O.BF16, Lq, Lk, 2, seed=Lq + Lk)


def test_attention_gqa_gate(dev):
    run(dev, O.BF16, 192, 320, 8, group=4, gate=True, seed=3)


@pytest.mark.parametrize("q_pos0", [0, 77])
def test_attention_causal(dev, q_pos0):
    run(dev, O.F16, 300, 300 + q_pos0, 2, causal=1, q_pos0=q_pos0, seed=4)


def test_attention_big_term(dev):
    run(dev, O.BF16, 160, 200, 4, group=2, big=True, seed=5)


@pytest.mark.parametrize("dtype,causal,gate", [(O.F16, 0, True), (O.BF16, 1, False), (O.BF16, 0, True)])
def test_attention_big_term_many_blocks(dev, dtype, causal, gate):
    """The rank-1 fp32 term over many key blocks (its per-block kb prefetch), ragged tails, GQA, with the
    gate and the causal mask."""
    run(dev, dtype, 700, 700, 4, group=2, causal=causal, gate=gate, big=True, seed=8 + causal)


def test_attention_peaky_scores(dev):
    """Large logits (scale 4 inputs) exercise the lazy max update and the rescale path."""
    run(dev, O.F16, 256, 512, 2, seed=6, scale=4.0)


def test_attention_strided_q(dev):
    run(dev, O.F16, 128, 128, 2, extra_cols=64, seed=7)


def test_attention_golden_fixture(dev):
    from krea_image_amd import kh
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "attn.npz"), allow_pickle=False)
    H, grp = int(g["heads"]), int(g["group"])
    Lq, Lk = g["Q"].shape[0], g["K"].shape[0]
    for key, causal, gate in (("out", 0, None), ("out_causal", 1, None), ("out_gated", 0, g["G"])):
        Od = torch.zeros(Lq, H * 128, dtype=torch.float16, device=dev)
        kh.attention(to_dev16(g["Q"], O.F16, dev), to_dev16(g["K"], O.F16, dev), to_dev16(g["V"], O.F16, dev), Od,
                     Lq, Lk, H, H * 128, (H // grp) * 128, (H // grp) * 128, H * 128, grp, bool(causal),
                     int(g["q_pos0"]) if causal else 0, None if gate is None else to_dev16(gate, O.F16, dev),
                     H * 128 if gate is not None else 0)
        torch.cuda.synchronize()
        assert rel_l2(Od.cpu().float().numpy(), g[key]) < TOL, key


def test_attention_config3_rows(dev):
    """4608 tokens, 24 heads x 128, fp16; the oracle checks 3 heads' worth via a head subset."""
    run(dev, O.F16, 4608, 4608, 3, seed=8)


def test_attention_rows_past_lq_untouched(dev):
    """O rows >= Lq and the columns of other heads' slots past `heads` are never written: Lq = 300 ends inside
    a 256-query workgroup, O carries 20 extra sentinel rows and 128 extra sentinel columns (ldo > 128 heads)."""
    from krea_image_amd import kh
    rng = np.random.default_rng(71)
    Lq, Lk, H = 300, 200, 3
    q = to_dev16(randn16(rng, (Lq, H * 128), O.F16), O.F16, dev)
    k = to_dev16(randn16(rng, (Lk, H * 128), O.F16), O.F16, dev)
    v = to_dev16(randn16(rng, (Lk, H * 128), O.F16), O.F16, dev)
    ldo = (H + 1) * 128
    Od = torch.full((Lq + 20, ldo), 3.0, dtype=torch.float16, device=dev)
    print("[attention rows past Lq]", flush=True)
    kh.attention(q, k, v, Od, Lq, Lk, H, H * 128, H * 128, H * 128, ldo)
    torch.cuda.synchronize()
    o = Od.cpu()
    assert (o[Lq:] == 3.0).all(), "rows >= Lq were written"
    assert (o[:Lq, H * 128:] == 3.0).all(), "columns past the last head were written"
    assert torch.isfinite(o[:Lq, :H * 128].float()).all()
