"""Parity of the ops around the GEMMs (kh_rms_norm, kh_qk_norm_rope, kh_gemv, kh_make_cond, kh_gemm_f32)
against the CPU oracle, through the C ABI. Tolerances: one 16-bit rounding of the outputs (<= 0.5 % rel L2);
f32 outputs 1e-5 (the GEMV sums in another order than the oracle's float64); the GEMV and the fp32 GEMM repeat
bit for bit."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import from_dev16, rel_l2, to_dev16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("out_dtype", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("center", [0, 1])
@pytest.mark.parametrize("width", [3072, 6144, 136])
def test_rms_norm(dev, out_dtype, center, width):
    from krea_image_amd import kh
    rng = np.random.default_rng(width + center)
    rows = 37
    x = (rng.standard_normal((rows, width)) * 2 + 0.3).astype(np.float32)
    mul = rng.standard_normal(width).astype(np.float32)
    add = rng.standard_normal(width).astype(np.float32)
    tdt = {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}[out_dtype]
    y = torch.empty(rows, width, dtype=tdt, device=dev)
    kh.rms_norm(torch.from_numpy(x).to(dev), torch.from_numpy(mul).to(dev), torch.from_numpy(add).to(dev), y, rows,
                width, width, width, 1e-6, center)
    torch.cuda.synchronize()
    ref = O.rms_norm(x, mul, add, out_dtype, 1e-6, center)
    got = y.cpu().numpy() if out_dtype == O.F32 else O.to_f32(from_dev16(y), out_dtype)
    ref = ref if out_dtype == O.F32 else O.to_f32(ref, out_dtype)
    assert rel_l2(got, ref) < (1e-5 if out_dtype == O.F32 else 5e-3)


@pytest.mark.parametrize("rope_mode", [0, 1, 2])
@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
def test_qk_norm_rope(dev, rope_mode, dtype):
    from krea_image_amd import kh
    rng = np.random.default_rng(rope_mode * 7 + dtype)
    T, Hh, Ww = 5, 6, 7
    rows, nq, nk = T + Hh * Ww, 4, 2
    ld = (nq + 2 * nk) * 128 + 64
    qkv = O.from_f32(rng.standard_normal((rows, ld)).astype(np.float32), dtype)
    wq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    c, s = O.rope_tables(T, Hh, Ww, rope_mode % 2)
    d = to_dev16(qkv, dtype, dev)
    kh.qk_norm_rope(d, torch.from_numpy(wq).to(dev), torch.from_numpy(wk).to(dev), torch.from_numpy(c).to(dev),
                    torch.from_numpy(s).to(dev), rows, ld, 0, nq, nq * 128, nk, 1e-6, rope_mode)
    torch.cuda.synchronize()
    ref, _, _ = O.qk_norm_rope(qkv, dtype, wq, wk, c, s, 0, nq, nq * 128, nk, 1e-6, rope_mode)
    got = from_dev16(d)
    assert rel_l2(O.to_f32(got, dtype), O.to_f32(ref, dtype)) < 5e-3
    assert np.array_equal(got[:, (nq + nk) * 128:], qkv[:, (nq + nk) * 128:])   # v block and tail untouched


def test_qk_norm_rope_big_dim(dev):
    from krea_image_amd import kh
    rng = np.random.default_rng(3)
    rows, nq, nk, ld = 20, 2, 1, 384
    qkv = O.from_f32(rng.standard_normal((rows, ld)).astype(np.float32), O.BF16)
    w = np.ones(128, np.float32)
    c, s = O.rope_tables(0, 4, 5, 0)
    d = to_dev16(qkv, O.BF16, dev)
    qb = torch.zeros(rows, nq, device=dev)
    kb = torch.zeros(rows, nk, device=dev)
    wt = torch.from_numpy(w).to(dev)
    kh.qk_norm_rope(d, wt, wt, torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev), rows, ld, 0, nq, nq * 128,
                    nk, 1e-5, 0, 37, qb, kb)
    torch.cuda.synchronize()
    ref, rqb, rkb = O.qk_norm_rope(qkv, O.BF16, w, w, c, s, 0, nq, nq * 128, nk, 1e-5, 0, 37)
    assert rel_l2(O.to_f32(from_dev16(d), O.BF16), O.to_f32(ref, O.BF16)) < 5e-3
    assert rel_l2(qb.cpu().numpy(), rqb) < 1e-5 and rel_l2(kb.cpu().numpy(), rkb) < 1e-5


@pytest.mark.parametrize("kind", ["ch", "g128", "16", "f32"])
@pytest.mark.parametrize("act", [0, 1, 3, 4, 6])
@pytest.mark.parametrize("rows", [1, 3])
def test_gemv(dev, kind, act, rows):
    """kh_gemv against the oracle (<= 1e-5 relative L2) for every weight format, SiLU / GELU on load and the
    accumulate bit; the output repeats bit for bit (fixed-order reduction, no atomics)."""
    from krea_image_amd import kh
    rng = np.random.default_rng(11 + act + 7 * rows)
    K, N = (3072, 18432) if kind == "ch" else (1024, 1040) if kind == "f32" else (3072, 1024)
    print(f"[gemv] {kind} act={act} rows={rows} K={K} N={N}", flush=True)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    if kind == "ch":
        w = rng.integers(-127, 128, (K, N), dtype=np.int8)
        s = O.from_f32(np.abs(rng.standard_normal(N)).astype(np.float32) * 1e-4, O.F16)
        W = kh.Weight(torch.from_numpy(w).to(dev), to_dev16(s, O.F16, dev), K)
        wargs = (w, O.I8, s, O.F16, K)
    elif kind == "g128":
        w, s = O.quant_q8((rng.standard_normal((K, N)) * 0.02).astype(np.float32), 128)
        W = kh.Weight(torch.from_numpy(w).to(dev), torch.from_numpy(s).to(dev), 128)
        wargs = (w, O.I8, s, O.F32, 128)
    elif kind == "16":
        w = O.from_f32((rng.standard_normal((K, N)) * 0.02).astype(np.float32), O.BF16)
        W = kh.Weight(to_dev16(w, O.BF16, dev))
        wargs = (w, O.BF16, None, O.F32, 0)
    else:
        w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
        W = kh.Weight(torch.from_numpy(w).to(dev))
        wargs = (w, O.F32, None, O.F32, 0)
    y0 = rng.standard_normal((rows, N)).astype(np.float32)
    xd, bd = torch.from_numpy(x).to(dev), torch.from_numpy(bias).to(dev)
    outs = []
    for _ in range(2):
        y = torch.from_numpy(y0.copy()).to(dev)
        kh.gemv(xd, W, y, rows, N, K, N, act, bd)
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1])
    ref = O.gemv(x, *wargs, y=y0.copy(), act=act, bias=bias)
    assert rel_l2(outs[0].numpy(), ref) < 1e-5


@pytest.mark.parametrize("kind", ["g64h", "f16", "chbf"])
@pytest.mark.parametrize("rows", [2, 4])
def test_gemv_ragged(dev, kind, rows):
    """kh_gemv on the shapes the sweep above leaves out: 2 and 4 rows (the four-row instantiation), fp16 weights,
    fp16 group scales (groups of 64) and bf16 per-channel scales, K that is not a multiple of the 128-way K split
    (uneven split, a short last range) and N that leaves the last workgroup's second lane group past the end."""
    from krea_image_amd import kh
    rng = np.random.default_rng(500 + rows)
    if kind == "g64h":
        K, N = 960, 1040
        w, s32 = O.quant_q8((rng.standard_normal((K, N)) * 0.02).astype(np.float32), 64)
        s = O.from_f32(s32, O.F16)
        W = kh.Weight(torch.from_numpy(w).to(dev), to_dev16(s, O.F16, dev), 64)
        wargs = (w, O.I8, s, O.F16, 64)
    elif kind == "chbf":
        K, N = 1000, 1040
        w = rng.integers(-127, 128, (K, N), dtype=np.int8)
        s = O.from_f32(np.abs(rng.standard_normal(N)).astype(np.float32) * 1e-4, O.BF16)
        W = kh.Weight(torch.from_numpy(w).to(dev), to_dev16(s, O.BF16, dev), K)
        wargs = (w, O.I8, s, O.BF16, K)
    else:
        K, N = 1000, 1032
        w = O.from_f32((rng.standard_normal((K, N)) * 0.02).astype(np.float32), O.F16)
        W = kh.Weight(to_dev16(w, O.F16, dev))
        wargs = (w, O.F16, None, O.F32, 0)
    print(f"[gemv ragged] {kind} rows={rows} K={K} N={N}", flush=True)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    y = torch.zeros(rows, N, device=dev)
    kh.gemv(torch.from_numpy(x).to(dev), W, y, rows, N, K, N, 4, torch.from_numpy(bias).to(dev))
    torch.cuda.synchronize()
    ref = O.gemv(x, *wargs, y=np.zeros((rows, N), np.float32), act=4, bias=bias)
    assert rel_l2(y.cpu().numpy(), ref) < 1e-5


def test_gemv_rejects_bad_act(dev):
    from krea_image_amd import kh
    W = kh.Weight(torch.zeros(64, 64, device=dev))
    x, y = torch.zeros(1, 64, device=dev), torch.zeros(1, 64, device=dev)
    with pytest.raises(kh.KhError, match="exclusive"):
        kh.gemv(x, W, y, 1, 64, 64, 64, 5)


def test_make_cond(dev):
    from krea_image_amd import kh
    rng = np.random.default_rng(12)
    D = 3072
    tv, tab = (rng.standard_normal(6 * D).astype(np.float32) for _ in range(2))
    n1, n2 = (rng.standard_normal(D).astype(np.float32) for _ in range(2))
    mods = torch.empty(6 * D, device=dev)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    kh.make_cond(t(tv), t(tab), t(n1), t(n2), D, mods)
    torch.cuda.synchronize()
    assert np.allclose(mods.cpu().numpy().reshape(6, D), O.make_cond(tv, tab, n1, n2), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("mode", [1, 3, 5])
def test_gemm_f32(dev, mode):
    from krea_image_amd import kh
    rng = np.random.default_rng(mode)
    M, K, N = 300, 64, 3072
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) * 0.1).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    C = torch.from_numpy(C0.copy()).to(dev)
    kh.gemm_f32(torch.from_numpy(A).to(dev), torch.from_numpy(W).to(dev), C, M, N, K, K, N, N, mode,
                torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    v = A.astype(np.float64) @ W + b
    if mode & 2:
        v = torch.nn.functional.gelu(torch.from_numpy(v), approximate="tanh").numpy()
    ref = C0 + v if mode & 4 else v
    assert rel_l2(C.cpu().numpy(), ref) < 1e-5


def test_gemm_f32_head_shape_repeatable(dev):
    """The D -> 64 head at 4096 rows (16-row tiles, each output summed over all of K by one thread): against
    float64 and bit for bit across two runs."""
    from krea_image_amd import kh
    rng = np.random.default_rng(33)
    M, K, N = 4096, 3072, 64
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    Ad, Wd, bd = (torch.from_numpy(v).to(dev) for v in (A, W, b))
    outs = []
    for _ in range(2):
        C = torch.empty(M, N, device=dev)
        kh.gemm_f32(Ad, Wd, C, M, N, K, K, N, N, 1, bd)
        torch.cuda.synchronize()
        outs.append(C.cpu())
    assert torch.equal(outs[0], outs[1])
    assert rel_l2(outs[0].numpy(), A.astype(np.float64) @ W + b) < 1e-5
