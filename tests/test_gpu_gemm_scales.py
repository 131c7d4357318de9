"""kh_gemm with the int8 scale storage formats the other suites leave out, against the oracle: group scales
stored as fp16 (groups of 64 rows) and bf16 (groups of 256), and per-output-channel scales stored as f32 and
bf16 (kh_weight s_dtype KH_F32 / KH_F16 / KH_BF16 with group < K or = K). Group scales dequantize each weight
once, q s in f32 rounded to the activation type (engine/kernels/gemm.metal:190-196); per-channel scales multiply
the exact integer sum. Both activation types, the epilogues of every DiT projection, a data-parallel and a
stream-K launch (the latter through kh_gemm_ws), and the packed layout where the format allows it (per-channel
and f32 group scales: the others are rejected). Tolerance: <= 0.5 % relative L2, as every GEMM."""
import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import make_weight, randn16, to_dev16, weight_to_dev
from tests.test_gpu_gemm import run_case

pytestmark = pytest.mark.gpu
KINDS = ["g64h", "g256b", "chf32", "chbf"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("a_dtype", [O.F16, O.BF16])
@pytest.mark.parametrize("epi", ["store16", "resid_gate", "swiglu", "gelu", "bias_f32"])
def test_scale_formats_data_parallel(dev, kind, a_dtype, epi):
    run_case(dev, a_dtype, kind, epi, M=300, N=512, K=1024, seed=zlib.crc32(f"{kind}{a_dtype}{epi}".encode()) % 10000, ws=False)


@pytest.mark.parametrize("kind", KINDS)
def test_scale_formats_stream_k(dev, kind):
    # two 256 x 256 tiles over K = 32768 (512 K steps): the plan spreads them over one workgroup per CU, 4 K steps
    # each, so every tile's K range is split across many workgroups and summed in the fix-up
    run_case(dev, O.BF16, kind, "resid", M=256, N=512, K=32768, seed=7, ws=True)


def test_packed_rejects_16bit_group_scales(dev):
    from krea_image_amd import kh
    rng = np.random.default_rng(3)
    M, K, N = 64, 256, 256
    wd = make_weight(rng, K, N, "g64h", O.F16)
    W = weight_to_dev(wd, dev).pack()
    A = to_dev16(randn16(rng, (M, K), O.F16), O.F16, dev)
    C = torch.zeros(M, N, dtype=torch.float16, device=dev)
    with pytest.raises(kh.KhError, match="packed int8 weights need"):
        kh.gemm("store16", A, W, C, M, N, K, K, N, N)
