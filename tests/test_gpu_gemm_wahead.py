"""The three-step weight prefetch (gemm_kernel WA = 3, chosen per call by KH_GEMM_WAHEAD=3) against the two-step
kernel: the two differ only in when loads are issued and waited for, and sum the same products in the same
order, so every output must be bitwise equal. Covers the instantiations that have the form (packed int8 with
per-channel scales, data-parallel: 192-wide tiles for fp16 and bf16, 256-wide for fp16), every epilogue the DiT
and the configs use, K of 1, 2, 3, 4 and many steps (the loop's remainder paths after its three-step unroll),
ragged M and N, and one case against the oracle directly."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import make_weight, randn16, rel_l2, to_dev16, weight_to_dev
from tests.test_gpu_gemm import F32_OUT

pytestmark = pytest.mark.gpu


def _run(dev, a_dtype, epi, M, N, K, seed, wahead):
    from krea_image_amd import kh
    rng = np.random.default_rng(seed)
    A = to_dev16(randn16(rng, (M, K), a_dtype), a_dtype, dev)
    W = weight_to_dev(make_weight(rng, K, N, "ch", a_dtype), dev).pack()
    vec = torch.from_numpy(rng.standard_normal(N).astype(np.float32) * np.float32(0.1)).to(dev)
    C = (torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(dev) if epi in F32_OUT
         else torch.zeros(M, N, dtype=A.dtype, device=dev))
    old = os.environ.get("KH_GEMM_WAHEAD")
    os.environ["KH_GEMM_WAHEAD"] = str(wahead)
    try:
        kh.gemm(epi, A, W, C, M, N, K, K, N, N, vec)
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("KH_GEMM_WAHEAD", None)
        else:
            os.environ["KH_GEMM_WAHEAD"] = old
    return C.cpu(), A, W, vec


# (M, N, K): 4096 x 3072 runs 192-wide tiles (one wave on 256 CUs), 2048 x 8192 256-wide ones; K = 64 .. 256
# is 1 .. 4 K steps (no full three-step round, one round plus 0 or 1 remainder steps); 300 x 384 is ragged
SHAPES = [(4096, 3072, 1024), (2048, 8192, 1024), (4096, 3072, 64), (4096, 3072, 128), (4096, 3072, 192),
          (4096, 3072, 256), (2048, 8192, 320), (300, 384, 448)]
IDS = ["dp192", "dp256", "k1", "k2", "k3", "k4", "dp256k5", "ragged"]


@pytest.mark.parametrize("shape", SHAPES, ids=IDS)
@pytest.mark.parametrize("epi", ["store16", "resid", "resid_gate", "gelu", "bias16"])
def test_wahead3_bitwise_f16(dev, shape, epi):
    M, N, K = shape
    print(f"[wahead] f16 {epi} M={M} N={N} K={K}", flush=True)
    a = _run(dev, O.F16, epi, M, N, K, M + N + K, 2)[0]
    b = _run(dev, O.F16, epi, M, N, K, M + N + K, 3)[0]
    assert torch.equal(a, b), "three-step prefetch differs from the two-step kernel"


@pytest.mark.parametrize("shape", SHAPES[:1] + SHAPES[2:], ids=IDS[:1] + IDS[2:])
@pytest.mark.parametrize("epi", ["store16", "resid_gate"])
def test_wahead3_bitwise_bf16(dev, shape, epi):
    M, N, K = shape
    print(f"[wahead] bf16 {epi} M={M} N={N} K={K}", flush=True)
    a = _run(dev, O.BF16, epi, M, N, K, 3 * M + N + K, 2)[0]
    b = _run(dev, O.BF16, epi, M, N, K, 3 * M + N + K, 3)[0]
    assert torch.equal(a, b), "three-step prefetch differs from the two-step kernel"


def test_wahead3_against_oracle(dev):
    M, N, K = 512, 384, 704
    print(f"[wahead] f16 gelu vs oracle M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(77)
    Ab = randn16(rng, (M, K), O.F16)
    wd = make_weight(rng, K, N, "ch", O.F16)
    from krea_image_amd import kh
    A = to_dev16(Ab, O.F16, dev)
    W = weight_to_dev(wd, dev).pack()
    C = torch.zeros(M, N, dtype=torch.float16, device=dev)
    os.environ["KH_GEMM_WAHEAD"] = "3"
    try:
        kh.gemm("gelu", A, W, C, M, N, K, K, N, N)
        torch.cuda.synchronize()
    finally:
        os.environ.pop("KH_GEMM_WAHEAD", None)
    got = C.cpu().float().numpy()
    ref = O.to_f32(O.gemm(O.EPI["gelu"], Ab, O.F16, wd["w"], O.I8, wd["s"], O.F16, K), O.F16)
    assert rel_l2(got, ref) <= 5e-3
