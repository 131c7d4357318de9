"""kh_gemm_static (the entry point that allocates nothing: its stream-K workspace is the library's static device
array) against kh_gemm_ws with a caller workspace, through the C ABI, on two calls in a row, the second with a
smaller input; both shapes run stream-K, so the static array's partials and counters are used and reused.
Results must be bitwise equal (same launch plan, same K order of the partial sums), and both within the
per-GEMM budget of the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gemm_ws, make_weight, randn16, rel_l2, to_dev16, weight_to_dev

pytestmark = pytest.mark.gpu


def _call_static(A, W, C, M, N, K, epi, vec):
    from krea_image_amd import kh
    err = ctypes.create_string_buffer(512)
    wc = W.c()
    rc = kh.load().kh_gemm_static(kh._stream(), kh.EPI[epi], kh._ptr(A), kh.dtype_code(A.dtype), ctypes.byref(wc),
                                  kh._ptr(C), M, N, K, K, N, N, kh._ptr(vec), err, 512)
    kh._check(rc, err)


def test_gemm_static_matches_workspace_entry_point(dev):
    from krea_image_amd import kh
    # (M, N, K): 6 x 12 = 72 tiles x 48 K steps, then 2 x 8 = 16 tiles x 64 K steps: both stream-K on 256 CUs
    cases = [(1536, 3072, 3072, "gelu", 71), (512, 2048, 4096, "resid_gate", 72)]
    for M, N, K, epi, seed in cases:
        print(f"[gemm_static] M={M} N={N} K={K} epi={epi}", flush=True)
        rng = np.random.default_rng(seed)
        A16 = randn16(rng, (M, K), O.F16)
        wd = make_weight(rng, K, N, "ch", O.F16)
        A, W = to_dev16(A16, O.F16, dev), weight_to_dev(wd, dev).pack()
        vec = rng.standard_normal(N).astype(np.float32)
        vd = torch.from_numpy(vec).to(dev)
        f32 = epi == "resid_gate"
        C0 = rng.standard_normal((M, N)).astype(np.float32)
        mk = (lambda: torch.from_numpy(C0.copy()).to(dev)) if f32 else \
            (lambda: torch.zeros(M, N, dtype=torch.float16, device=dev))
        Cs, Cw = mk(), mk()
        _call_static(A, W, Cs, M, N, K, epi, vd)
        kh.gemm(epi, A, W, Cw, M, N, K, K, N, N, vd, gemm_ws(dev))
        torch.cuda.synchronize()
        assert torch.equal(Cs.cpu(), Cw.cpu()), "kh_gemm_static differs from kh_gemm_ws"
        rows = np.arange(0, M, 37)
        ref = O.gemm(O.EPI[epi], np.ascontiguousarray(A16[rows]), O.F16, wd["w"], wd["w_dtype"], wd["s"],
                     wd["s_dtype"], wd["group"], C=np.ascontiguousarray(C0[rows]) if f32 else None, vec=vec)
        got = Cs.cpu().numpy()[rows] if f32 else O.to_f32(Cs.cpu().view(torch.int16).numpy().view(np.uint16)[rows],
                                                          O.F16)
        ref = ref if f32 else O.to_f32(ref, O.F16)
        base = C0[rows] if f32 else 0
        assert rel_l2(got - base, ref - base) <= 5e-3
