"""The scalar-address form of the attention kernel (attn_kernel AA, chosen per call with KH_ATTN_ADDR=1) against
the default form: it changes only how addresses are formed (scalar block bases, per-lane offsets computed once,
the block max inside the lane-swap asm), so every output must be bitwise equal. Covers both activation types,
4- and 8-wave workgroups, ragged and single-block key ranges, causal masks with a query offset, GQA, the sigmoid
gate, the rank-1 term, and the configs[2] workload (4608 tokens x 24 heads, strided q | k | v). Strides above
2^24 fall back to the default form (host check)."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import randn16, rel_l2, to_dev16, from_dev16

pytestmark = pytest.mark.gpu


def _attn(dev, dtype, Lq, Lk, heads, group, causal, q_pos0, gate, big, seed, waves, addr):
    from krea_image_amd import kh
    rng = np.random.default_rng(seed)
    kvh = heads // group
    Q = to_dev16(randn16(rng, (Lq, heads * 128), dtype), dtype, dev)
    K = to_dev16(randn16(rng, (Lk, kvh * 128), dtype), dtype, dev)
    V = to_dev16(randn16(rng, (Lk, kvh * 128), dtype), dtype, dev)
    G = to_dev16(randn16(rng, (Lq, heads * 128), dtype), dtype, dev) if gate else None
    QB = torch.from_numpy((rng.standard_normal((Lq, heads)) * 3).astype(np.float32)).to(dev) if big else None
    KB = torch.from_numpy((rng.standard_normal((Lk, kvh)) * 3).astype(np.float32)).to(dev) if big else None
    O_ = torch.zeros(Lq, heads * 128, dtype=Q.dtype, device=dev)
    saved = {k: os.environ.get(k) for k in ("KH_ATTN_ADDR", "KH_ATTN_WAVES")}
    os.environ["KH_ATTN_ADDR"] = "1" if addr else "0"
    os.environ["KH_ATTN_WAVES"] = str(waves)
    try:
        kh.attention(Q, K, V, O_, Lq, Lk, heads, heads * 128, kvh * 128, kvh * 128, heads * 128, group, bool(causal),
                     q_pos0, G, heads * 128 if gate else 0, QB, KB)
        torch.cuda.synchronize()
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    return O_.cpu()


CASES = [  # dtype, Lq, Lk, heads, group, causal, q_pos0, gate, big
    (O.F16, 300, 517, 2, 1, 0, 0, False, False),
    (O.BF16, 256, 64, 4, 2, 0, 0, True, False),
    (O.BF16, 200, 1000, 8, 4, 1, 77, True, False),
    (O.F16, 33, 4097, 2, 2, 0, 0, False, True),
    (O.BF16, 513, 513, 4, 1, 1, 0, False, True),
    (O.F16, 1, 1, 1, 1, 0, 0, False, False),
]


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_addr_form_bitwise(dev, case, waves):
    dtype, Lq, Lk, heads, group, causal, q_pos0, gate, big = case
    print(f"[attn addr] waves={waves} case={case}", flush=True)
    a = _attn(dev, dtype, Lq, Lk, heads, group, causal, q_pos0, gate, big, Lq + Lk, waves, False)
    b = _attn(dev, dtype, Lq, Lk, heads, group, causal, q_pos0, gate, big, Lq + Lk, waves, True)
    assert torch.equal(a, b), "the scalar-address form differs from the default form"


def test_addr_form_config2(dev):
    """4608 tokens x 24 heads, q | k | v strided in one buffer, bitwise and against the oracle on a
    head's rows."""
    from krea_image_amd import kh
    L, H = 4608, 24
    D = H * 128
    print(f"[attn addr] configs[2] L={L} heads={H}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(70)
    qkv = torch.randn(L, 3 * D, generator=g, device=dev).half()
    outs = []
    for addr in ("0", "1"):
        os.environ["KH_ATTN_ADDR"] = addr
        try:
            O_ = torch.empty(L, D, dtype=torch.float16, device=dev)
            kh.attention(qkv, qkv[:, D:], qkv[:, 2 * D:], O_, L, L, H, 3 * D, 3 * D, 3 * D, D)
            torch.cuda.synchronize()
            outs.append(O_.cpu())
        finally:
            os.environ.pop("KH_ATTN_ADDR", None)
    assert torch.equal(outs[0], outs[1])
    host = from_dev16(qkv)
    rows = np.r_[0:32, L - 32:L]
    h = 17
    ref = O.to_f32(O.attention(np.ascontiguousarray(host[rows, 128 * h:128 * h + 128]),
                               np.ascontiguousarray(host[:, D + 128 * h:D + 128 * h + 128]),
                               np.ascontiguousarray(host[:, 2 * D + 128 * h:2 * D + 128 * h + 128]), O.F16, 1), O.F16)
    got = O.to_f32(from_dev16(outs[1])[rows, 128 * h:128 * h + 128], O.F16)
    assert rel_l2(got, ref) <= 5e-3
