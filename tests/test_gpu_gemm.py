"""Parity of kh_gemm (HIP, through the C ABI) against the CPU oracle's restatement of Metal::gemm.

Tolerance: <= 0.5 % relative L2 per GEMM (the per-GEMM budget of the north star); the fp32-accumulated
results differ only in summation order, so the measured errors sit far below it.
"""
import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, gemm_ws, make_weight, randn16, rel_l2, to_dev16, weight_to_dev

pytestmark = pytest.mark.gpu
TOL = 5e-3
EPIS = ["store16", "f32", "resid_gate", "resid", "swiglu", "gelu", "bias16", "bias_f32"]
F32_OUT = {"f32", "resid_gate", "resid", "bias_f32"}


def run_case(dev, a_dtype, kind, epi, M, N, K, seed=0, rows=None, ws=True):
    """One GEMM against the oracle; ws=True goes through kh_gemm_ws with a stream-K workspace (stream-K where
    the plan picks it), ws=False through kh_gemm (data-parallel always)."""
    from krea_image_amd import kh
    print(f"[gemm case] a_dtype={a_dtype} w={kind} epi={epi} M={M} N={N} K={K} seed={seed} ws={ws}", flush=True)
    rng = np.random.default_rng(seed)
    A = randn16(rng, (M, K), a_dtype)
    wd = make_weight(rng, K, N, kind, a_dtype)
    vec = rng.standard_normal(N).astype(np.float32) * np.float32(0.1)
    ncol = N // 2 if epi == "swiglu" else N
    C0 = rng.standard_normal((M, ncol)).astype(np.float32) if epi in F32_OUT else None

    Ad = to_dev16(A, a_dtype, dev)
    W = weight_to_dev(wd, dev)
    vd = torch.from_numpy(vec).to(dev)
    if epi in F32_OUT:
        Cd = torch.from_numpy(C0.copy()).to(dev)
    else:
        Cd = torch.zeros(M, ncol, dtype=Ad.dtype, device=dev)
    kh.gemm(epi, Ad, W, Cd, M, N, K, K, N, ncol, vd, gemm_ws(dev) if ws else None)
    torch.cuda.synchronize()
    got = Cd.cpu().numpy() if epi in F32_OUT else O.to_f32(from_dev16(Cd), a_dtype)

    # oracle on all rows (or a row subset: rows are independent)
    sel = np.arange(M) if rows is None else rows
    Cr = None if C0 is None else np.ascontiguousarray(C0[sel])
    ref = O.gemm(O.EPI[epi], np.ascontiguousarray(A[sel]), a_dtype, wd["w"], wd["w_dtype"], wd["s"], wd["s_dtype"],
                 wd["group"], C=Cr, vec=vec)
    ref = ref if epi in F32_OUT else O.to_f32(ref, a_dtype)
    got = got[sel]
    if C0 is not None and epi in ("resid", "resid_gate"):  # compare the increments, not the carried residual
        got, ref = got - C0[sel], ref - C0[sel]
    err = rel_l2(got, ref)
    print(f"    rel_l2={err:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL, f"rel L2 {err:.3e} > {TOL}"
    return err


@pytest.mark.parametrize("a_dtype", [O.F16, O.BF16])
@pytest.mark.parametrize("kind", ["ch", "g128", "16"])
@pytest.mark.parametrize("epi", EPIS)
def test_gemm_small_all_formats(dev, a_dtype, kind, epi):
    # M not a multiple of the 256-row tile, N not a multiple of the 256-column tile
    run_case(dev, a_dtype, kind, epi, M=300, N=320, K=256, seed=zlib.crc32(f"{a_dtype}{kind}{epi}".encode()) % 1000)


@pytest.mark.parametrize("M", [1, 7, 64, 257])
def test_gemm_ragged_rows(dev, M):
    run_case(dev, O.F16, "ch", "bias16", M=M, N=192, K=128, seed=M)


def test_gemm_config1_fp16_bias(dev):
    """X[4096,3072] fp16 x int8 [3072,3072] per-channel fp16 scales + fp16 bias -> fp16."""
    run_case(dev, O.F16, "ch", "bias16", M=4096, N=3072, K=3072, seed=1)


def test_gemm_mlp_up_full_size_rows(dev):
    """Target shape M=4096 K=3072 N=12288 with GELU; the oracle checks 96 rows spread over every tile row."""
    rows = np.sort(np.random.default_rng(5).choice(4096, 96, replace=False))
    run_case(dev, O.F16, "ch", "gelu", M=4096, N=12288, K=3072, seed=2, rows=rows)


def test_gemm_mlp_down_full_size_rows(dev):
    rows = np.sort(np.random.default_rng(6).choice(4096, 96, replace=False))
    run_case(dev, O.F16, "ch", "resid", M=4096, N=3072, K=12288, seed=3, rows=rows)


def test_gemm_reference_shape_swiglu_g128(dev):
    """Reference format: bf16 activations, dit_q8 group-128 f32 scales, SwiGLU over interleaved gate|up."""
    rows = np.sort(np.random.default_rng(7).choice(1024, 64, replace=False))
    run_case(dev, O.BF16, "g128", "swiglu", M=1024, N=4096, K=6144, seed=4, rows=rows)


def test_gemm_strided_output(dev):
    """lda / ldc larger than the logical widths (the reference writes q|k|v|gate column slices)."""
    from krea_image_amd import kh
    rng = np.random.default_rng(11)
    M, N, K, lda, ldc = 200, 128, 192, 256, 512
    A = randn16(rng, (M, lda), O.F16)
    wd = make_weight(rng, K, N, "ch", O.F16)
    Ad = to_dev16(A, O.F16, dev)
    Cd = torch.zeros(M, ldc, dtype=torch.float16, device=dev)
    kh.gemm("store16", Ad, weight_to_dev(wd, dev), Cd[:, 64:], M, N, K, lda, N, ldc)
    torch.cuda.synchronize()
    got = O.to_f32(from_dev16(Cd), O.F16)
    ref = O.to_f32(O.gemm(0, np.ascontiguousarray(A[:, :K]), O.F16, wd["w"], O.I8, wd["s"], O.F16, K), O.F16)
    assert rel_l2(got[:, 64:64 + N], ref) <= TOL
    assert not got[:, :64].any() and not got[:, 64 + N:].any(), "columns outside [64, 64+N) were written"


def test_gemm_rejects_bad_shapes(dev):
    from krea_image_amd import kh
    A = torch.zeros(64, 96, dtype=torch.float16, device=dev)
    W = kh.Weight(torch.zeros(96, 64, dtype=torch.int8, device=dev), torch.ones(64, dtype=torch.float16, device=dev))
    C = torch.zeros(64, 64, dtype=torch.float16, device=dev)
    with pytest.raises(kh.KhError, match="K % 64"):
        kh.gemm("store16", A, W, C, 64, 64, 96, 96, 64, 64)


@pytest.mark.parametrize("epi", EPIS)
def test_gemm_golden_fixture_per_channel(dev, epi):
    """The kernels against tests/golden/gemm_ch.npz (numpy float64, independent of the oracle)."""
    import os
    from krea_image_amd import kh
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemm_ch.npz"), allow_pickle=False)
    M, K = g["A"].shape
    N = g["q"].shape[1]
    ncol = N // 2 if epi == "swiglu" else N
    Ad = to_dev16(g["A"], O.F16, dev)
    W = kh.Weight(torch.from_numpy(g["q"]).to(dev), to_dev16(g["s"], O.F16, dev), K)
    vec = torch.from_numpy(g["vec"]).to(dev)
    if epi in F32_OUT:
        C = torch.from_numpy(g["X0"].copy() if epi in ("resid", "resid_gate") else np.zeros((M, N), np.float32)).to(dev)
    else:
        C = torch.zeros(M, ncol, dtype=torch.float16, device=dev)
    kh.gemm(epi, Ad, W, C, M, N, K, K, N, ncol, vec)
    torch.cuda.synchronize()
    got = C.cpu().numpy() if epi in F32_OUT else C.cpu().float().numpy()
    ref = g["out_" + epi]
    if epi in ("resid", "resid_gate"):
        got, ref = got - g["X0"], ref - g["X0"]
    assert rel_l2(got, ref) < (1e-3 if epi not in F32_OUT else 1e-5), epi


def test_gemm_golden_fixture_group128_bf16(dev):
    import os
    from krea_image_amd import kh
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemm_g128.npz"), allow_pickle=False)
    M, K = g["A"].shape
    N = g["q"].shape[1]
    C = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    kh.gemm("store16", to_dev16(g["A"], O.BF16, dev), kh.Weight(torch.from_numpy(g["q"]).to(dev),
            torch.from_numpy(g["s"]).to(dev), 128), C, M, N, K, K, N, N)
    torch.cuda.synchronize()
    assert rel_l2(C.cpu().float().numpy(), g["out_store16"]) < 8e-3


@pytest.mark.parametrize("epi", ["store16", "resid_gate", "swiglu", "bias_f32"])
@pytest.mark.parametrize("packed", [False, True])
def test_gemm_rows_past_m_untouched(dev, epi, packed):
    """Rows >= M of C are never written (gemm.metal:270,282): C is allocated with 37 extra rows of a sentinel;
    M = 300 ends inside a 256-row tile, so the last tile's clamped rows must not store."""
    from krea_image_amd import kh
    rng = np.random.default_rng(61)
    M, N, K, extra = 300, 512, 256, 37
    A = to_dev16(randn16(rng, (M, K), O.F16), O.F16, dev)
    W = weight_to_dev(make_weight(rng, K, N, "ch", O.F16), dev)
    W = W.pack() if packed else W
    vec = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev)
    ncol = N // 2 if epi == "swiglu" else N
    dt = torch.float32 if epi in F32_OUT else torch.float16
    C = torch.full((M + extra, ncol), 7.0, dtype=dt, device=dev)
    print(f"[rows past M] epi={epi} packed={packed}", flush=True)
    kh.gemm(epi, A, W, C, M, N, K, K, N, ncol, vec)
    torch.cuda.synchronize()
    assert (C[M:].cpu() == 7.0).all(), "rows >= M were written"
    assert not (C[:M].cpu() == 7.0).all()


def test_gemm_activation_offsets_near_2pow31(dev):
    """Largest A the 32-bit activation offsets allow: (M - 1) * lda + K = 2146304000 < 2^31 (A is 4.3 GB of fp16).
    Rows spread over the whole range, the last rows included, against the oracle (the rejection one row past
    the limit is a CPU test: tests/test_abi.py)."""
    from krea_image_amd import kh
    M, K, N = 262000, 8192, 256
    g = torch.Generator(device=dev)
    g.manual_seed(81)
    print(f"[gemm max offsets] M={M} K={K} N={N}", flush=True)
    A = torch.randn(M, K, generator=g, device=dev, dtype=torch.float16)
    rng = np.random.default_rng(81)
    wd = make_weight(rng, K, N, "ch", O.F16)
    W = weight_to_dev(wd, dev).pack()
    C = torch.empty(M, N, dtype=torch.float16, device=dev)
    kh.gemm("store16", A, W, C, M, N, K, K, N, N)
    torch.cuda.synchronize()
    rows = np.concatenate([np.linspace(0, M - 9, 40).astype(np.int64), np.arange(M - 8, M)])
    Ah = A[torch.from_numpy(rows).to(dev)].cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    ref = O.to_f32(O.gemm(0, Ah, O.F16, wd["w"], O.I8, wd["s"], O.F16, K), O.F16)
    got = C[torch.from_numpy(rows).to(dev)].cpu().float().numpy()
    assert rel_l2(got, ref) <= TOL
    del A, C
    torch.cuda.empty_cache()
