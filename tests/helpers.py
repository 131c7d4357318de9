"""Shared test helpers: seeded synthetic inputs (numpy), upload to the device, relative L2."""
import numpy as np
import torch

from oracle import oracle as O

NP16 = {O.F16: np.float16}
TORCH16 = {O.F16: torch.float16, O.BF16: torch.bfloat16}


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def randn16(rng, shape, dtype, scale=1.0):
    """N(0, scale^2) rounded to the 16-bit type; returns the uint16 bit pattern."""
    return O.from_f32(rng.standard_normal(shape).astype(np.float32) * np.float32(scale), dtype)


def to_dev16(bits, dtype, dev):
    """uint16 bit pattern -> 16-bit device tensor of that type."""
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev)
    return t.view(TORCH16[dtype])


def from_dev16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def make_weight(rng, K, N, kind, a_dtype):
    """Synthetic weight in one of the three formats (numpy side):
    'ch'  : int8 U{-127..127} [K, N] + fp16 per-output-channel scales |N(0, 0.02)| / 127 (benchmark configs)
    'g128': convert.py q8 of W ~ N(0, 0.02): int8 [K, N] + f32 scales [K/128, N] (reference dit_q8 format)
    'g64h' / 'g256b': the same quantizer with groups of 64 / 256 rows, scales stored as fp16 / bf16
    'chf32' / 'chbf': int8 + per-output-channel scales stored as f32 / bf16
    '16'  : W ~ N(0, 0.02) as 16-bit [K, N]
    Returns dict(w=np array, s=np array or None, w_dtype, s_dtype, group)."""
    if kind == "ch":
        q = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
        s = np.abs(rng.standard_normal(N).astype(np.float32) * np.float32(0.02)) / np.float32(127)
        return dict(w=q, s=O.from_f32(s, O.F16), w_dtype=O.I8, s_dtype=O.F16, group=K)
    if kind == "g128":
        w = rng.standard_normal((K, N)).astype(np.float32) * np.float32(0.02)
        q, s = O.quant_q8(w, 128)
        return dict(w=q, s=s, w_dtype=O.I8, s_dtype=O.F32, group=128)
    if kind in ("g64h", "g256b"):
        # other groups, scales stored as fp16 / bf16 (kh_weight s_dtype KH_F16 / KH_BF16 with group < K)
        group, s_dt = (64, O.F16) if kind == "g64h" else (256, O.BF16)
        w = rng.standard_normal((K, N)).astype(np.float32) * np.float32(0.02)
        q, s = O.quant_q8(w, group)
        return dict(w=q, s=O.from_f32(s, s_dt), w_dtype=O.I8, s_dtype=s_dt, group=group)
    if kind in ("chf32", "chbf"):
        # per-output-channel scales stored as f32 / bf16
        q = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
        s = np.abs(rng.standard_normal(N).astype(np.float32) * np.float32(0.02)) / np.float32(127)
        if kind == "chf32":
            return dict(w=q, s=s, w_dtype=O.I8, s_dtype=O.F32, group=K)
        return dict(w=q, s=O.from_f32(s, O.BF16), w_dtype=O.I8, s_dtype=O.BF16, group=K)
    w = rng.standard_normal((K, N)).astype(np.float32) * np.float32(0.02)
    return dict(w=O.from_f32(w, a_dtype), s=None, w_dtype=a_dtype, s_dtype=O.F32, group=0)


def weight_to_dev(wd, dev):
    from krea_image_amd import kh
    if wd["w_dtype"] == O.I8:
        w = torch.from_numpy(wd["w"]).to(dev)
    else:
        w = to_dev16(wd["w"], wd["w_dtype"], dev)
    s = None
    if wd["s"] is not None:
        if wd["s_dtype"] == O.F32:
            s = torch.from_numpy(wd["s"]).to(dev)
        else:
            s = to_dev16(wd["s"], wd["s_dtype"], dev)
    return kh.Weight(w, s, wd["group"])


def unpack_int8(packed):
    """Inverse of kh_pack_int8's layout (byte (k // 8) 8 ldw + 32 (n // 4) + 4 (k % 8) + n % 4 holds (k, n))."""
    K, L = packed.shape
    return np.ascontiguousarray(packed.reshape(K // 8, L // 4, 8, 4).transpose(0, 2, 1, 3).reshape(K, L))


def host_int8(W):
    """The input-major int8 matrix of a kh.Weight, packed or not, as numpy."""
    q = W.w.cpu().numpy()
    return unpack_int8(q) if getattr(W, "packed", False) else q


_WS = {}


def gemm_ws(dev):
    """One kh_gemm_ws stream-K workspace per device for the tests (kh.gemm_workspace)."""
    from krea_image_amd import kh
    if dev not in _WS:
        _WS[dev] = kh.gemm_workspace(dev)
    return _WS[dev]
