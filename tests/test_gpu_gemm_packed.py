"""kh_pack_int8 and kh_gemm on packed int8 weights (KH_I8P): the packed buffer against the layout include/kh.h
documents (numpy), and every packed GEMM bitwise against the same GEMM on the input-major weights (which the
oracle tests pin) — data-parallel 256- and 192-wide tiles, stream-K, SwiGLU, ragged M, both scale formats,
column views of a wider matrix — plus one packed case against the oracle directly."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import gemm_ws, make_weight, randn16, rel_l2, to_dev16, weight_to_dev
from tests.test_gpu_gemm import F32_OUT

pytestmark = pytest.mark.gpu


def pack_np(q):
    """(k, n) -> byte (k // 8) 8 ldw + 32 (n // 4) + 4 (k % 8) + n % 4."""
    K, L = q.shape
    return q.reshape(K // 8, 8, L // 4, 4).transpose(0, 2, 1, 3).reshape(K, L)


def test_pack_layout(dev):
    from krea_image_amd import kh
    rng = np.random.default_rng(51)
    q = rng.integers(-128, 128, size=(136, 208), dtype=np.int8)  # K % 64 != 0, ldw % 64 != 0
    print("[pack] K=136 ldw=208", flush=True)
    got = kh.pack_int8(torch.from_numpy(q).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, pack_np(q))
    # round trip through the closed form's inverse
    K, L = q.shape
    back = got.reshape(K // 8, L // 4, 8, 4).transpose(0, 2, 1, 3).reshape(K, L)
    np.testing.assert_array_equal(back, q)


def _both(dev, a_dtype, kind, epi, M, N, K, seed):
    from krea_image_amd import kh
    rng = np.random.default_rng(seed)
    A = to_dev16(randn16(rng, (M, K), a_dtype), a_dtype, dev)
    W = weight_to_dev(make_weight(rng, K, N, kind, a_dtype), dev)
    vec = torch.from_numpy(rng.standard_normal(N).astype(np.float32) * np.float32(0.1)).to(dev)
    ncol = N // 2 if epi == "swiglu" else N
    C0 = torch.from_numpy(rng.standard_normal((M, ncol)).astype(np.float32)).to(dev) if epi in F32_OUT else None
    outs = []
    for w in (W, W.pack()):
        C = C0.clone() if C0 is not None else torch.zeros(M, ncol, dtype=A.dtype, device=dev)
        kh.gemm(epi, A, w, C, M, N, K, K, N, ncol, vec, gemm_ws(dev))
        torch.cuda.synchronize()
        outs.append(C.cpu())
    return outs


# (M, N, K): 256 tiles of 256 x 256 (one data-parallel wave); 4096 x 3072 (192-wide tiles); 1024 x 2048 x 4096
# (stream-K, tiles split ~8 ways); 300 x 320 (ragged M and N, stream-K over 4 tiles)
SHAPES = [(2048, 8192, 1024), (4096, 3072, 1024), (1024, 2048, 4096), (300, 320, 256)]


@pytest.mark.parametrize("shape", SHAPES, ids=["dp256", "dp192", "streamk", "ragged"])
@pytest.mark.parametrize("epi", ["store16", "resid_gate", "gelu", "bias_f32"])
def test_packed_bitwise_per_channel_f16(dev, shape, epi):
    M, N, K = shape
    print(f"[packed] f16 ch {epi} M={M} N={N} K={K}", flush=True)
    a, b = _both(dev, O.F16, "ch", epi, M, N, K, seed=M + N + K)
    assert torch.equal(a, b), "packed and input-major weights give different results"


@pytest.mark.parametrize("shape", SHAPES, ids=["dp256", "dp192", "streamk", "ragged"])
@pytest.mark.parametrize("epi", ["store16", "swiglu", "resid"])
def test_packed_bitwise_group128_bf16(dev, shape, epi):
    M, N, K = shape
    print(f"[packed] bf16 g128 {epi} M={M} N={N} K={K}", flush=True)
    a, b = _both(dev, O.BF16, "g128", epi, M, N, K, seed=M + 2 * N + K)
    assert torch.equal(a, b), "packed and input-major weights give different results"


def test_packed_column_view(dev):
    """Columns [c0, c0 + N) of a packed [K, ldw] matrix start at byte 8 c0, with the same ldw."""
    from krea_image_amd import kh
    rng = np.random.default_rng(53)
    M, K, ldw, c0, N = 512, 512, 768, 256, 320
    Ab = randn16(rng, (M, K), O.F16)
    A = to_dev16(Ab, O.F16, dev)
    wd = make_weight(rng, K, ldw, "ch", O.F16)
    W = weight_to_dev(wd, dev)
    Wp = W.pack()
    s = W.s[c0:c0 + N]
    full = kh.Weight(W.w.view(-1)[c0:], s, K)
    pk = kh.Weight(Wp.w.view(-1)[8 * c0:], s, K, packed=True)
    outs = []
    for w in (full, pk):
        C = torch.zeros(M, N, dtype=torch.float16, device=dev)
        kh.gemm("store16", A, w, C, M, N, K, K, ldw, N)
        torch.cuda.synchronize()
        outs.append(C.cpu())
    assert torch.equal(outs[0], outs[1])
    ref = O.to_f32(O.gemm(0, Ab, O.F16, np.ascontiguousarray(wd["w"][:, c0:c0 + N]), O.I8,
                          np.ascontiguousarray(wd["s"][c0:c0 + N]), O.F16, K), O.F16)
    got = O.to_f32(outs[1].view(torch.int16).numpy().view(np.uint16), O.F16)
    assert rel_l2(got, ref) <= 5e-3


def test_packed_rejections(dev):
    from krea_image_amd import kh
    rng = np.random.default_rng(54)
    wd = make_weight(rng, 256, 256, "g128", O.F16)
    W = weight_to_dev(wd, dev).pack()
    W16 = kh.Weight(W.w, W.s.half(), 128, packed=True)  # group scales in f16: not a packed format
    A = torch.zeros(64, 256, dtype=torch.float16, device=dev)
    C = torch.zeros(64, 256, dtype=torch.float16, device=dev)
    with pytest.raises(kh.KhError, match="packed int8"):
        kh.gemm("store16", A, W16, C, 64, 256, 256, 256, 256, 256)
    x = torch.zeros(1, 256, device=dev)
    y = torch.zeros(1, 256, device=dev)
    with pytest.raises(kh.KhError, match="KH_I8P"):
        kh.gemv(x, W, y, 1, 256, 256, 256)
    with pytest.raises(kh.KhError, match="multiple of 8"):
        kh.pack_int8(torch.zeros(12, 64, dtype=torch.int8, device=dev))


@pytest.mark.parametrize("epi,K,N", [("gelu", 3072, 12288), ("resid", 12288, 3072)], ids=["up", "down"])
def test_packed_bitwise_benchmark_shapes(dev, epi, K, N):
    """The bench's MLP pair at full size (4096 rows): packed == input-major, bitwise."""
    print(f"[packed] bench shape {epi} M=4096 K={K} N={N}", flush=True)
    a, b = _both(dev, O.F16, "ch", epi, 4096, N, K, seed=K + N)
    assert torch.equal(a, b)
