"""A seeded sweep of kh_gemm launches over random shapes, epilogues, weight formats and activation types
against the oracle. The shapes are drawn so that every launch plan occurs: data-parallel 256-wide tiles,
192- and 128-wide tiles (N that pads less to them, or a partial single wave), stream-K (few tiles, long K),
ragged last row / column tiles, and K from one to many steps. Each case prints its parameters first."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.test_gpu_gemm import EPIS, run_case

pytestmark = pytest.mark.gpu


def _cases(n, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = ["ch", "g128", "16"][i % 3]
        a_dtype = [O.F16, O.BF16][(i // 3) % 2]
        epi = EPIS[int(rng.integers(len(EPIS)))]
        N = 64 * int(rng.choice([1, 2, 3, 5, 6, 8, 12, 16, 20, 24, 48]))
        if epi == "swiglu" and N % 128:
            N += 64  # gate / up pairs
        step = 128 if kind == "g128" else 64
        K = step * int(rng.choice([1, 2, 3, 5, 8, 16, 40]))
        M = int(rng.choice([1, 7, 64, 255, 256, 257, 700, 1500, 3000, 4100]))
        out.append((i, a_dtype, kind, epi, M, N, K))
    return out


@pytest.mark.parametrize("i,a_dtype,kind,epi,M,N,K", _cases(48))
def test_gemm_random_shapes(dev, i, a_dtype, kind, epi, M, N, K):
    # rows are independent: check a subset of rows on the oracle for the largest shapes
    rows = None if M * N * K <= 2e8 else np.unique(np.r_[0:min(M, 64), M - 64:M, np.arange(0, M, 97)])
    run_case(dev, a_dtype, kind, epi, M=M, N=N, K=K, seed=1000 + i, rows=rows)
