"""kh_gemm launches on narrow tiles: 256 x 192 where 256-wide tiles fill only part of one wave of workgroups
and 192-wide ones still fit in one, or where N pads less to 192 (384, 320); 256 x 128 for 16-bit weights
where N pads less to 128 (64, 128). Checked against the oracle for every epilogue and weight format, with
ragged last row / column tiles, and bitwise against the 256-wide launch of the same GEMM
(KH_GEMM_TN192=0): every width sums the same products in the same order per output."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gemm_ws, make_weight, randn16, to_dev16, weight_to_dev
from tests.test_gpu_gemm import EPIS, F32_OUT, run_case

pytestmark = pytest.mark.gpu

# 16 x 12 = 192 tiles of 256 x 256 (stream-K needs < 60 % of 256 CUs, so these stay data-parallel) become
# 16 x 16 = 256 tiles of 256 x 192; M = 3900 leaves the last row tile ragged.
M, N = 3900, 3072


@pytest.mark.parametrize("epi", [e for e in EPIS if e != "swiglu"])
def test_tn192_all_epilogues(dev, epi):
    run_case(dev, O.F16, "ch", epi, M=M, N=N, K=256, seed=41)


@pytest.mark.parametrize("kind,a_dtype", [("g128", O.BF16), ("16", O.F16), ("16", O.BF16), ("ch", O.BF16)])
def test_tn192_weight_formats(dev, kind, a_dtype):
    run_case(dev, a_dtype, kind, "resid_gate", M=M, N=N, K=384, seed=42)


@pytest.mark.parametrize("epi", ["resid", "gelu", "bias16"])
def test_tn192_matches_256_wide_bitwise(dev, epi):
    from krea_image_amd import kh
    print(f"[tn192 bitwise] epi={epi} M={M} N={N}", flush=True)
    rng = np.random.default_rng(43)
    K = 512
    A = to_dev16(randn16(rng, (M, K), O.F16), O.F16, dev)
    W = weight_to_dev(make_weight(rng, K, N, "ch", O.F16), dev)
    vec = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev)
    C0 = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(dev)

    def run():
        C = C0.clone() if epi in F32_OUT else torch.zeros(M, N, dtype=torch.float16, device=dev)
        kh.gemm(epi, A, W, C, M, N, K, K, N, N, vec, gemm_ws(dev))
        torch.cuda.synchronize()
        return C.cpu()

    a = run()
    os.environ["KH_GEMM_TN192"] = "0"
    try:
        b = run()
    finally:
        del os.environ["KH_GEMM_TN192"]
    assert torch.equal(a, b), "192-wide and 256-wide launches differ"


@pytest.mark.parametrize("epi", ["store16", "bias16", "f32", "resid_gate", "gelu"])
@pytest.mark.parametrize("N", [64, 128])
def test_tn128_16bit_weights(dev, epi, N):
    # 129 row tiles: the narrow data-parallel launch needs less work per CU than 256-wide stream-K
    run_case(dev, O.BF16, "16", epi, M=32900, N=N, K=192, seed=44)


@pytest.mark.parametrize("kind,N", [("16", 320), ("ch", 384), ("g128", 384)])
def test_tn192_padding(dev, kind, N):
    # 320 -> two 192-wide tiles, the second ragged (128 of 192 columns); 384 -> exactly two
    run_case(dev, O.BF16, kind, "bias16", M=25500, N=N, K=256, seed=45)


@pytest.mark.parametrize("kind,N", [("16", 128), ("16", 320), ("ch", 384)])
def test_narrow_matches_256_wide_bitwise(dev, kind, N):
    from krea_image_amd import kh
    print(f"[narrow bitwise] w={kind} N={N}", flush=True)
    rng = np.random.default_rng(46)
    Mr, K = 40000, 256  # 157 row tiles: narrow data-parallel launches (>= 60 % of a wave)
    A = to_dev16(randn16(rng, (Mr, K), O.BF16), O.BF16, dev)
    W = weight_to_dev(make_weight(rng, K, N, kind, O.BF16), dev)
    vec = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev)

    def run():
        C = torch.zeros(Mr, N, dtype=torch.bfloat16, device=dev)
        kh.gemm("bias16", A, W, C, Mr, N, K, K, N, N, vec, gemm_ws(dev))
        torch.cuda.synchronize()
        return C.cpu()

    a = run()
    os.environ["KH_GEMM_TN192"] = "0"
    try:
        b = run()
    finally:
        del os.environ["KH_GEMM_TN192"]
    assert torch.equal(a, b), "narrow and 256-wide launches differ"
