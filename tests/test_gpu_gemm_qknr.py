"""kh_gemm_qk_norm_rope: the QKV projection with the per-head q / k RMSNorm + RoPE fused into the GEMM
epilogue (engine/src/model.mm:373-375 as one launch), against (a) the two-call path kh_gemm(STORE16) +
kh_qk_norm_rope, which the oracle pins (tests/test_gpu_ops.py), and (b) the oracle's qk_norm_rope applied to
the oracle GEMM. The fused epilogue norms the same 16-bit-rounded projection values; only the order of the
per-head sum of squares differs, so outputs agree to a 16-bit rounding (rel L2 < 2e-3, most bits equal) and
the v / gate columns are bitwise equal."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, gemm_ws, make_weight, randn16, rel_l2, to_dev16, weight_to_dev

pytestmark = pytest.mark.gpu


def _case(dev, dtype, kind, rope_mode, big_dim, nq, nk, gate, M, K, seed):
    from krea_image_amd import kh
    print(f"[gemm qknr] dtype={dtype} w={kind} rope={rope_mode} big={big_dim} nq={nq} nk={nk} gate={gate} M={M} "
          f"K={K}", flush=True)
    rng = np.random.default_rng(seed)
    N = (2 * nq + 2 * nk if gate else nq + 2 * nk) * 128
    A = randn16(rng, (M, K), dtype)
    wd = make_weight(rng, K, N, kind, dtype)
    Ad, W = to_dev16(A, dtype, dev), weight_to_dev(wd, dev)
    wq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    T = 7
    Hh = 8
    Ww = (M - T + Hh - 1) // Hh
    c, s = O.rope_tables(T, Hh, Ww, rope_mode % 2)
    c, s = np.ascontiguousarray(c[:M]), np.ascontiguousarray(s[:M])
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    wqd, wkd, cd, sd = t(wq), t(wk), t(c), t(s)
    big = big_dim >= 0
    qb1, kb1 = torch.zeros(M, nq, device=dev), torch.zeros(M, nk, device=dev)
    qb2, kb2 = torch.zeros(M, nq, device=dev), torch.zeros(M, nk, device=dev)
    tdt = torch.float16 if dtype == O.F16 else torch.bfloat16
    C1 = torch.empty(M, N, dtype=tdt, device=dev)
    kh.gemm_qk_norm_rope(Ad, W, C1, M, N, K, K, N, N, wqd, wkd, cd, sd, 0, nq, nq * 128, nk, 1e-5, rope_mode, big_dim,
                         qb1 if big else None, kb1 if big else None, ws=gemm_ws(dev))
    C2 = torch.empty(M, N, dtype=tdt, device=dev)
    kh.gemm("store16", Ad, W, C2, M, N, K, K, N, N, ws=gemm_ws(dev))
    kh.qk_norm_rope(C2, wqd, wkd, cd, sd, M, N, 0, nq, nq * 128, nk, 1e-5, rope_mode, big_dim,
                    qb2 if big else None, kb2 if big else None)
    torch.cuda.synchronize()
    g1, g2 = from_dev16(C1), from_dev16(C2)
    qk = (nq + nk) * 128
    assert np.array_equal(g1[:, qk:], g2[:, qk:]), "v / gate columns differ"
    f1, f2 = O.to_f32(g1[:, :qk], dtype), O.to_f32(g2[:, :qk], dtype)
    assert rel_l2(f1, f2) < 2e-3
    assert np.mean(g1[:, :qk] == g2[:, :qk]) > 0.9
    if big:
        assert rel_l2(qb1.cpu().numpy(), qb2.cpu().numpy()) < 1e-4
        assert rel_l2(kb1.cpu().numpy(), kb2.cpu().numpy()) < 1e-4
    # against the oracle: oracle GEMM (16-bit output) then the oracle's qk_norm_rope
    ref16 = O.gemm(O.EPI["store16"], A, dtype, wd["w"], wd["w_dtype"], wd["s"], wd["s_dtype"], wd["group"])
    ref, _, _ = O.qk_norm_rope(ref16, dtype, wq, wk, c, s, 0, nq, nq * 128, nk, 1e-5, rope_mode, big_dim)
    assert rel_l2(O.to_f32(g1, dtype), O.to_f32(ref, dtype)) < 5e-3


@pytest.mark.parametrize("rope_mode", [0, 1, 2])
@pytest.mark.parametrize("dtype,kind", [(O.F16, "ch"), (O.BF16, "g128")])
def test_qknr_modes(dev, rope_mode, dtype, kind):
    _case(dev, dtype, kind, rope_mode, -1, nq=4, nk=2, gate=False, M=333, K=256, seed=rope_mode + 10 * dtype)


@pytest.mark.parametrize("big_dim", [0, 37, 127])
def test_qknr_big_dim_gqa_gate(dev, big_dim):
    # reference layout: q | k | v | gate, GQA 4:1 (heads 8 / kv heads 2), a big dimension in f32
    _case(dev, O.BF16, "g128", 0, big_dim, nq=8, nk=2, gate=True, M=300, K=512, seed=20 + big_dim)


def test_qknr_16bit_weights_streamk(dev):
    # 4 x 6 = 24 tiles of 256 x 256 x 64 K steps over 256 CUs: a stream-K launch whose fix-up runs the fused
    # epilogue
    _case(dev, O.F16, "16", 1, -1, nq=8, nk=2, gate=False, M=1000, K=4096, seed=31)


def test_qknr_rejects_unaligned_heads(dev):
    from krea_image_amd import kh
    A = torch.zeros(64, 64, dtype=torch.bfloat16, device=dev)
    W = kh.Weight(torch.zeros(64, 512, dtype=torch.bfloat16, device=dev))
    C = torch.empty(64, 512, dtype=torch.bfloat16, device=dev)
    w = torch.ones(128, device=dev)
    tab = torch.zeros(64, 64, device=dev)
    with pytest.raises(kh.KhError, match="multiples of 128"):
        kh.gemm_qk_norm_rope(A, W, C, 64, 512, 64, 64, 512, 512, w, w, tab, tab, 64, 2, 320, 1, 1e-5, 0)
