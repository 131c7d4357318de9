"""Stream-K launches of kh_gemm_ws (caller workspace): tiles whose K steps are split over several workgroups (the
last to arrive adds the partials in K order). Checked against the oracle for every epilogue, for bitwise
run-to-run determinism, and against the data-parallel launch of the same GEMM (kh_gemm without a workspace, or
KH_GEMM_STREAMK=0), which sums the same products in a different grouping and so agrees to rounding."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, gemm_ws, make_weight, randn16, rel_l2, to_dev16, weight_to_dev
from tests.test_gpu_gemm import EPIS, F32_OUT, run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("epi", EPIS)
def test_streamk_many_way_split_all_epilogues(dev, epi):
    # 4 x 8 = 32 tiles x 64 K steps over one wave of workgroups: every tile is split ~8 ways
    run_case(dev, O.BF16, "g128", epi, M=1024, N=2048, K=4096, seed=31)


@pytest.mark.parametrize("kind", ["ch", "16"])
def test_streamk_few_way_split(dev, kind):
    # 5 x 12 = 60 tiles x 48 K steps: tiles split over 4-5 workgroups at uneven K offsets, ragged M
    run_case(dev, O.F16, kind, "resid_gate", M=1200, N=3072, K=3072, seed=32)


def _gemm_once(dev, epi, M, N, K, seed):
    from krea_image_amd import kh
    rng = np.random.default_rng(seed)
    A = to_dev16(randn16(rng, (M, K), O.F16), O.F16, dev)
    W = weight_to_dev(make_weight(rng, K, N, "ch", O.F16), dev)
    vec = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev)
    C0 = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(dev)

    def run(ws=True):
        C = C0.clone() if epi in F32_OUT else torch.zeros(M, N, dtype=torch.float16, device=dev)
        kh.gemm(epi, A, W, C, M, N, K, K, N, N, vec, gemm_ws(dev) if ws else None)
        torch.cuda.synchronize()
        return C.cpu()
    return run


@pytest.mark.parametrize("epi", ["resid", "gelu"])
def test_streamk_deterministic_and_matches_data_parallel(dev, epi):
    run = _gemm_once(dev, epi, 1536, 3072, 3072, seed=33)   # 72 tiles on 256 CUs: stream-K
    a, b = run(), run()
    assert torch.equal(a, b), "stream-K results differ between runs"
    os.environ["KH_GEMM_STREAMK"] = "0"
    try:
        c = run()
    finally:
        del os.environ["KH_GEMM_STREAMK"]
    assert torch.equal(c, run(ws=False)), "KH_GEMM_STREAMK=0 and no workspace both give the data-parallel launch"
    af, cf = a.float().numpy(), c.float().numpy()
    if epi in F32_OUT:
        assert rel_l2(af, cf) < 1e-6
    else:
        assert rel_l2(af, cf) < 2e-3  # one 16-bit rounding may flip


def test_streamk_workspace_shared_by_consecutive_launches(dev):
    """Consecutive stream-K launches on one workspace (the counters each launch leaves at zero) give the results
    of launches on fresh workspaces; a workspace of one byte too few runs data-parallel."""
    from krea_image_amd import kh
    run = _gemm_once(dev, "gelu", 1536, 3072, 3072, seed=34)
    first = [run(), run(), run()]
    assert all(torch.equal(first[0], x) for x in first[1:])
    fresh = kh.gemm_workspace(dev)
    rng = np.random.default_rng(34)
    A = to_dev16(randn16(rng, (1536, 3072), O.F16), O.F16, dev)
    W = weight_to_dev(make_weight(rng, 3072, 3072, "ch", O.F16), dev)
    vec = torch.from_numpy(rng.standard_normal(3072).astype(np.float32)).to(dev)
    C1 = torch.zeros(1536, 3072, device=dev)
    C2 = torch.zeros_like(C1)
    C3 = torch.zeros_like(C1)
    kh.gemm("f32", A, W, C1, 1536, 3072, 3072, 3072, 3072, 3072, vec, fresh)
    kh.gemm("f32", A, W, C2, 1536, 3072, 3072, 3072, 3072, 3072, vec, fresh[: fresh.numel() - 1])
    kh.gemm("f32", A, W, C3, 1536, 3072, 3072, 3072, 3072, 3072, vec)
    torch.cuda.synchronize()
    assert torch.equal(C2.cpu(), C3.cpu())
    assert not torch.equal(C1.cpu(), C3.cpu())  # stream-K splits the K sum: f32 results differ in rounding
    assert rel_l2(C1.cpu().numpy(), C3.cpu().numpy()) < 1e-6
