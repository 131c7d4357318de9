"""The engine's packed weight file (.qw): writer, int8 group quantizer and gate/up interleave (the offline
converter's transforms, tools/convert.py:49-130), and the reader over libkh (kh_qw_*: mmap, validate,
upload into one resident device allocation).

Format (tools/convert.py:13-17): b"QWTS" | u32 version (1) | u64 header_len | JSON header | zero pad |
tensor data. header = {"tensors": {name: {dtype, shape, offset, nbytes}}, "meta": {...}}; the data starts
at the first 16 KiB boundary after the header and every tensor offset (relative to it) is 16 KiB aligned,
in the order the tensors were planned. Linear weights are stored input-major Wt[K, N]; int8 weights carry
f32 scales [K / 128, N]; SwiGLU gate / up rows are interleaved per 64-column GEMM tile.

A DiT file (tools/convert.py:174-224, dit_specs / convert_dit) has per layer i:
  L{i}.qkvg [D, 2D + 2 kvD] (q | k | v | gate), L{i}.o [D, D], L{i}.gu [D, 2 FF] (interleaved),
  L{i}.down [FF, D] (each + ".s" when int8), L{i}.qn / kn [128], L{i}.n1 / n2 [D] (stored as 1 + w),
  L{i}.mod [6, D]; and first.w [64, D], first.b [D], last.w [D, 64], last.b [64], last.n [D], last.mod [2, D].
"""
import ctypes
import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, Iterable, List, Optional, Tuple

import numpy as np

from . import kh

ALIGN = 16384   # tensor / data alignment (convert.py ALIGN)
Q_GROUP = 128   # int8 scale group along K (convert.py Q_GROUP)
GEMM_BN = 64    # SwiGLU interleave tile (convert.py GEMM_BN; the GEMM's SwiGLU epilogue pairs within it)
MAGIC = b"QWTS"
VERSION = 1

_NP = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i8": np.int8}
_SIZE = {"f32": 4, "f16": 2, "bf16": 2, "i8": 1}
_CODE = {"f32": kh.F32, "f16": kh.F16, "bf16": kh.BF16, "i8": kh.I8}
_NAME = {v: k for k, v in _CODE.items()}


# ---------------------------------------------------------------------------------------------------------
# converter transforms
def quantize_q8(w_t: np.ndarray, group: int = Q_GROUP) -> Tuple[np.ndarray, np.ndarray]:
    """Wt[K, N] -> int8 [K, N] + f32 scales [K / group, N] (tools/convert.py:92-99): per output column and
    `group`-row block, scale = max(amax, 1e-12) / 127, q = clamp(round_half_even(w / scale), -127, 127),
    all in f32."""
    w = np.asarray(w_t, dtype=np.float32)
    K, N = w.shape
    if K % group:
        raise ValueError(f"K={K} is not a multiple of the group {group}")
    g = w.reshape(K // group, group, N)
    scale = (np.maximum(np.abs(g).max(axis=1), np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(g / scale[:, None, :]), -127, 127).astype(np.int8).reshape(K, N)
    return q, scale


def interleave_gate_up(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """gate / up [F, D] (output-major) -> [2F, D] grouped per GEMM tile: [gate 32 | up 32] x F / 32
    (tools/convert.py:102-107). Column 64 t + i (i < 32) of the transposed weight is gate unit 32 t + i and
    column 64 t + 32 + i is up unit 32 t + i."""
    F, Dm = gate.shape
    h = GEMM_BN // 2
    if up.shape != gate.shape or F % h:
        raise ValueError("gate / up must have the same shape with rows a multiple of 32")
    return np.concatenate([gate.reshape(F // h, h, Dm), up.reshape(F // h, h, Dm)], axis=1).reshape(2 * F, Dm)


def deinterleave_gate_up(gu: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Inverse of interleave_gate_up (tools/convert.py:110-115)."""
    F2, Dm = gu.shape
    v = gu.reshape(F2 // GEMM_BN, GEMM_BN, Dm)
    h = GEMM_BN // 2
    return v[:, :h].reshape(-1, Dm), v[:, h:].reshape(-1, Dm)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns (round to nearest even), as torch's .to(bfloat16) stores them."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u >> 16) & 1) + np.uint32(0x7FFF)
    out = ((u + r) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = 0x7FC0
    return out


# ---------------------------------------------------------------------------------------------------------
# writer
class QwWriter:
    """A .qw file laid out before any data arrives: every tensor's offset follows from (name, dtype, shape) alone,
    so the header is final at open and each tensor is written straight to its own offset (positional writes,
    any order), one at a time: a multi-GB file is never held in memory (the layout of tools/convert.py:49-89).
    The file appears under its name only once every planned tensor has been written (close)."""

    def __init__(self, path: str, specs: Iterable[Tuple[str, str, Tuple[int, ...]]], meta: Optional[dict] = None):
        self.path, self.tmp = path, path + ".partial"
        plan, end = {}, 0
        for name, dtype, shape in specs:
            if dtype not in _SIZE:
                raise ValueError(f"{name}: unknown dtype {dtype}")
            if name in plan:
                raise ValueError(f"{name}: planned twice")
            nbytes = int(np.prod(shape, dtype=np.int64)) * _SIZE[dtype]
            plan[name] = {"dtype": dtype, "shape": [int(s) for s in shape], "offset": end, "nbytes": nbytes}
            end = -(-(end + nbytes) // ALIGN) * ALIGN
        self.header = {"tensors": plan, "meta": meta or {}}
        hj = json.dumps(self.header).encode()
        self.data_start = -(-(16 + len(hj)) // ALIGN) * ALIGN
        self.fd = os.open(self.tmp, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
        os.pwrite(self.fd, MAGIC + struct.pack("<IQ", VERSION, len(hj)) + hj, 0)
        os.ftruncate(self.fd, self.data_start + end)
        self.pending = set(plan)

    def write(self, name: str, a: np.ndarray):
        """`a`: f32 / f16 / int8 values, or uint16 bf16 bit patterns for a bf16 tensor (f32 input is rounded)."""
        info = self.header["tensors"].get(name)
        if info is None:
            raise KeyError(f"{name}: not in the file's plan")
        if name not in self.pending:
            raise RuntimeError(f"{name}: already written")
        a = np.asarray(a)
        if info["dtype"] == "bf16" and a.dtype != np.uint16:
            a = bf16_bits(a)
        a = np.ascontiguousarray(a, dtype=_NP[info["dtype"]])
        if list(a.shape) != info["shape"]:
            raise RuntimeError(f"{name}: shape {list(a.shape)} != planned {info['shape']}")
        buf, pos = memoryview(a).cast("B"), self.data_start + info["offset"]
        while len(buf):
            n = os.pwrite(self.fd, buf, pos)
            buf, pos = buf[n:], pos + n
        self.pending.discard(name)

    def close(self):
        if self.pending:
            raise RuntimeError(f"{self.path}: no data for {sorted(self.pending)[:4]} ({len(self.pending)} tensors)")
        os.close(self.fd)
        os.replace(self.tmp, self.path)


def write_qw(path: str, tensors: List[Tuple[str, str, np.ndarray]], meta: Optional[dict] = None):
    """Write (name, dtype, array) tensors in the given order."""
    w = QwWriter(path, [(n, d, a.shape) for n, d, a in tensors], meta)
    for n, _, a in tensors:
        w.write(n, a)
    w.close()


def dit_specs(D: int, kv_heads: int, FF: int, layers: int, quant: bool, latent: int = 64):
    """(name, dtype, shape) of a DiT file, in the converter's order (tools/convert.py:174-187)."""
    def lin(name, K, N):
        return [(name, "i8", (K, N)), (name + ".s", "f32", (K // Q_GROUP, N))] if quant else [(name, "bf16", (K, N))]
    specs = []
    for i in range(layers):
        p = f"L{i}."
        specs += lin(p + "qkvg", D, 2 * D + 2 * kv_heads * 128) + lin(p + "o", D, D) + lin(p + "gu", D, 2 * FF)
        specs += lin(p + "down", FF, D)
        specs += [(p + "qn", "f32", (128,)), (p + "kn", "f32", (128,)), (p + "n1", "f32", (D,)),
                  (p + "n2", "f32", (D,)), (p + "mod", "f32", (6, D))]
    specs += [("first.w", "f32", (latent, D)), ("first.b", "f32", (D,)), ("last.w", "f32", (D, latent)),
              ("last.b", "f32", (latent,)), ("last.n", "f32", (D,)), ("last.mod", "f32", (2, D))]
    return specs


def write_random_dit(path: str, D: int, kv_heads: int, FF: int, layers: int, quant: bool = True, seed: int = 0,
                     big_gain: Optional[Tuple[int, int, float]] = None, direct_q8: bool = False):
    """A random-init DiT in the converter's layout (the stand-in for dit_q8.qw / dit.qw: no checkpoint is
    available offline). Linear weights ~ N(0, 1/sqrt(K)) in the checkpoint's [out, in] orientation, then
    transposed, fused, interleaved and quantized as convert_dit does (tools/convert.py:190-224).
    direct_q8 (with quant): the int8 values (uniform in [-127, 127]) and f32 group scales (~1 / (73 sqrt(K)),
    so the weights' spread is again ~1/sqrt(K)) are drawn directly, which is what a reference-width file
    (hundreds of millions of weights per layer) needs to be written in seconds; the file layout is the same.
    big_gain = (layer, dim, g): sets qn[dim] = kn[dim] = g in that layer (a high-gain q.k dimension)."""
    rng = np.random.default_rng(seed)
    w = QwWriter(path, dit_specs(D, kv_heads, FF, layers, quant),
                 {"model": "krea2-dit-random", "layers": layers, "q8": quant, "dim": D, "kv_heads": kv_heads,
                  "ff": FF, "seed": seed})
    kvD = kv_heads * 128

    def lin(name, w_out_in):
        if direct_q8 and quant:
            N, K = w_out_in
            w.write(name, rng.integers(-127, 128, (K, N), dtype=np.int8))
            sc = (1.0 + 0.1 * rng.standard_normal((K // Q_GROUP, N), dtype=np.float32)) / np.float32(73 * np.sqrt(K))
            w.write(name + ".s", np.abs(sc).astype(np.float32))
            return
        wt = np.ascontiguousarray(w_out_in.T.astype(np.float32))
        if quant:
            q, s = quantize_q8(wt)
            w.write(name, q)
            w.write(name + ".s", s)
        else:
            w.write(name, wt)

    def mat(o, i):
        return rng.standard_normal((o, i), dtype=np.float32) / np.float32(np.sqrt(i))

    for i in range(layers):
        p = f"L{i}."
        if direct_q8 and quant:  # (out, in) shapes only
            lin(p + "qkvg", (2 * D + 2 * kvD, D))
            lin(p + "o", (D, D))
            lin(p + "gu", (2 * FF, D))
            lin(p + "down", (D, FF))
        else:
            lin(p + "qkvg", np.concatenate([mat(D, D), mat(kvD, D), mat(kvD, D), mat(D, D)]))
            lin(p + "o", mat(D, D))
            lin(p + "gu", interleave_gate_up(mat(FF, D), mat(FF, D)))
            lin(p + "down", mat(D, FF))
        qn = 1.0 + 0.1 * rng.standard_normal(128, dtype=np.float32)
        kn = 1.0 + 0.1 * rng.standard_normal(128, dtype=np.float32)
        if big_gain is not None and big_gain[0] == i:
            qn[big_gain[1]] = kn[big_gain[1]] = big_gain[2]
        w.write(p + "qn", qn)
        w.write(p + "kn", kn)
        w.write(p + "n1", 1.0 + 0.1 * rng.standard_normal(D, dtype=np.float32))
        w.write(p + "n2", 1.0 + 0.1 * rng.standard_normal(D, dtype=np.float32))
        w.write(p + "mod", 0.1 * rng.standard_normal((6, D), dtype=np.float32))
    w.write("first.w", 0.02 * rng.standard_normal((64, D), dtype=np.float32))
    w.write("first.b", 0.01 * rng.standard_normal(D, dtype=np.float32))
    w.write("last.w", 0.02 * rng.standard_normal((D, 64), dtype=np.float32))
    w.write("last.b", 0.01 * rng.standard_normal(64, dtype=np.float32))
    w.write("last.n", 1.0 + 0.1 * rng.standard_normal(D, dtype=np.float32))
    w.write("last.mod", 0.1 * rng.standard_normal((2, D), dtype=np.float32))
    w.close()


def cond_specs(D: int, n_base: int, n_fast: int):
    """(name, dtype, shape) of a cond.qw file (tools/convert.py:287-293)."""
    return [("tmlp1.w", "f32", (256, D)), ("tmlp1.b", "f32", (D,)), ("tmlp2.w", "f32", (D, D)),
            ("tmlp2.b", "f32", (D,)), ("tproj.w", "f32", (D, 6 * D)), ("tproj.b", "f32", (6 * D,)),
            ("base.sigma", "f32", (n_base,)), ("base.t", "f32", (n_base, D)), ("base.tvec", "f32", (n_base, 6 * D)),
            ("fast.sigma", "f32", (n_fast,)), ("fast.t", "f32", (n_fast, D)), ("fast.tvec", "f32", (n_fast, 6 * D))]


def write_random_cond(path: str, D: int, base_sigmas, fast_sigmas, seed: int = 0):
    """A random-init cond.qw in the converter's layout (the stand-in for the real file, which needs the
    checkpoint): f32 tmlp1 / tmlp2 / tproj weights ~ N(0, 1/sqrt(in)) stored input-major, small biases, and
    per-schedule tables whose t / tvec rows are random values (so a table hit is told apart from a computed
    conditioning)."""
    rng = np.random.default_rng(seed)
    base = np.asarray(base_sigmas, np.float32)
    fast = np.asarray(fast_sigmas, np.float32)
    w = QwWriter(path, cond_specs(D, len(base), len(fast)), {"model": "krea2-conditioning-random", "seed": seed})

    def mat(i, o):
        return rng.standard_normal((i, o), dtype=np.float32) / np.float32(np.sqrt(i))

    w.write("tmlp1.w", mat(256, D))
    w.write("tmlp1.b", 0.1 * rng.standard_normal(D, dtype=np.float32))
    w.write("tmlp2.w", mat(D, D))
    w.write("tmlp2.b", 0.1 * rng.standard_normal(D, dtype=np.float32))
    w.write("tproj.w", mat(D, 6 * D))
    w.write("tproj.b", 0.1 * rng.standard_normal(6 * D, dtype=np.float32))
    for tag, sig in (("base", base), ("fast", fast)):
        w.write(tag + ".sigma", sig)
        w.write(tag + ".t", rng.standard_normal((len(sig), D), dtype=np.float32))
        w.write(tag + ".tvec", 0.2 * rng.standard_normal((len(sig), 6 * D), dtype=np.float32))
    w.close()


# ---------------------------------------------------------------------------------------------------------
# reader (libkh)
class _TensorC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * 8), ("offset", ctypes.c_size_t), ("nbytes", ctypes.c_size_t),
                ("host", ctypes.c_void_p), ("dev", ctypes.c_void_p)]


def _bind(lib):
    if getattr(lib, "_qw_bound", False):
        return lib
    vp, i, cp = ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p
    lib.kh_qw_open.argtypes, lib.kh_qw_open.restype = [cp, cp, i], vp
    lib.kh_qw_close.argtypes, lib.kh_qw_close.restype = [vp], None
    lib.kh_qw_count.argtypes, lib.kh_qw_count.restype = [vp], i
    lib.kh_qw_version.argtypes, lib.kh_qw_version.restype = [vp], ctypes.c_uint
    lib.kh_qw_meta.argtypes, lib.kh_qw_meta.restype = [vp], cp
    lib.kh_qw_at.argtypes, lib.kh_qw_at.restype = [vp, i, ctypes.POINTER(_TensorC)], i
    lib.kh_qw_find.argtypes, lib.kh_qw_find.restype = [vp, cp, ctypes.POINTER(_TensorC)], i
    lib.kh_qw_upload.argtypes, lib.kh_qw_upload.restype = [vp, vp, cp, i], i
    lib._qw_bound = True
    return lib


@dataclass
class TensorInfo:
    """engine/src/weights.h:16-21 (TensorInfo), plus the host / device addresses."""
    name: str
    dtype: str
    shape: Tuple[int, ...]
    offset: int
    nbytes: int
    host: int
    dev: Optional[int]


class DevPtr:
    """A raw device address with the data_ptr() interface the kh structures read."""

    def __init__(self, p: int):
        self.p = p

    def data_ptr(self) -> int:
        return self.p


@dataclass
class RawWeight:
    """A kh_weight over device addresses inside an uploaded .qw file."""
    w: int
    s: Optional[int]
    w_dtype: int
    s_dtype: int
    group: int

    def c(self):
        return kh._WeightC(self.w, self.s or 0, self.w_dtype, self.s_dtype, self.group)


class QwFile:
    """WeightFile (engine/src/weights.mm:16-98) over libkh: mmap + header validation in C++, one upload."""

    def __init__(self, path: str):
        self.lib = _bind(kh.load())
        err = ctypes.create_string_buffer(512)
        self.h = self.lib.kh_qw_open(path.encode(), err, 512)
        if not self.h:
            raise kh.KhError(err.value.decode(errors="replace"))
        self.path = path

    def close(self):
        if self.h:
            self.lib.kh_qw_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self) -> int:
        return self.lib.kh_qw_version(self.h)

    @property
    def meta(self) -> dict:
        return json.loads(self.lib.kh_qw_meta(self.h).decode())

    def __len__(self) -> int:
        return self.lib.kh_qw_count(self.h)

    @staticmethod
    def _info(t: _TensorC) -> TensorInfo:
        return TensorInfo(t.name.decode(), _NAME[t.dtype], tuple(t.shape[:t.ndim]), t.offset, t.nbytes, t.host,
                          t.dev or None)

    def names(self) -> List[str]:
        out = []
        t = _TensorC()
        for i in range(len(self)):
            self.lib.kh_qw_at(self.h, i, ctypes.byref(t))
            out.append(t.name.decode())
        return out

    def has(self, name: str) -> bool:
        t = _TensorC()
        return self.lib.kh_qw_find(self.h, name.encode(), ctypes.byref(t)) == 0

    def info(self, name: str) -> TensorInfo:
        t = _TensorC()
        if self.lib.kh_qw_find(self.h, name.encode(), ctypes.byref(t)) != 0:
            raise kh.KhError(f"missing tensor: {name} in {self.path}")
        return self._info(t)

    def array(self, name: str) -> np.ndarray:
        """A host copy (numpy; bf16 as uint16 bit patterns)."""
        ti = self.info(name)
        buf = (ctypes.c_char * ti.nbytes).from_address(ti.host)
        return np.frombuffer(buf, dtype=_NP[ti.dtype]).reshape(ti.shape).copy()

    def upload(self):
        """Copy the data region to the current device (synchronous, once)."""
        import torch
        err = ctypes.create_string_buffer(512)
        rc = self.lib.kh_qw_upload(self.h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), err, 512)
        kh._check(rc, err)
        return self

    def conditioning(self, fast: bool, sigma: float, t, tvec, work) -> bool:
        """kh_conditioning on this (uploaded) cond.qw: t [D] and tvec [6 D] (f32 device tensors) for noise level
        sigma, Conditioning::get / compute (engine/src/model.mm:545-591); work: f32 device scratch of >= 256 + D
        floats (None is enough for a table hit). Returns True when the sigma was found in the schedule's table."""
        hit = ctypes.c_int(0)
        err = ctypes.create_string_buffer(512)
        wp, wb = (None, 0) if work is None else (kh._ptr(work), work.numel() * work.element_size())
        rc = kh.load().kh_conditioning(kh._stream(), self.h, int(fast), float(sigma), kh._ptr(t), kh._ptr(tvec),
                                       wp, wb, ctypes.byref(hit), err, 512)
        kh._check(rc, err)
        return bool(hit.value)

    def dev(self, name: str) -> DevPtr:
        ti = self.info(name)
        if ti.dev is None:
            raise kh.KhError(f"{self.path} is not uploaded")
        return DevPtr(ti.dev)

    def weight(self, name: str, pack: bool = False) -> RawWeight:
        """The GEMM weight `name` (+ `name.s` for int8): Metal's Weight{w, s, q8} (engine/src/metal.h:25-29).
        pack=True rearranges an int8 weight in place into kh_gemm's packed layout (kh_pack_int8 into one scratch
        buffer, copied back: no extra resident memory) on first request; from then on the weight is always
        returned as KH_I8P, so its bytes are never read as the input-major layout again."""
        ti = self.info(name)
        if ti.dtype == "i8":
            si = self.info(name + ".s")
            K = ti.shape[0]
            group = K // si.shape[0] if si.shape[0] else 0
            packed = self.__dict__.setdefault("_packed", set())
            if pack and name not in packed and (group == K or si.dtype == "f32"):
                N = ti.shape[1]
                import torch
                tmp = torch.empty(K * N, dtype=torch.int8, device="cuda")
                kh._call(kh.load().kh_pack_int8, kh._stream(), self.dev(name).p, K, N, kh._ptr(tmp))
                kh._call(kh.load().kh_copy, kh._stream(), self.dev(name).p, kh._ptr(tmp), K * N)
                torch.cuda.current_stream().synchronize()
                packed.add(name)
            return RawWeight(self.dev(name).p, self.dev(name + ".s").p, kh.I8P if name in packed else kh.I8,
                             _CODE[si.dtype], group)
        return RawWeight(self.dev(name).p, None, _CODE[ti.dtype], kh.F32, 0)
