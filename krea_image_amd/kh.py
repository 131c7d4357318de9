"""ctypes binding of libkh.so (include/kh.h) with a torch-tensor front end.

This is the host-side mirror of the reference engine's op layer krea::Metal (engine/src/metal.h:44-167):
the same op names, argument meanings (M, N, K, lda, ldw, ldc, epilogue, vec) and error behaviour (an
unsupported shape raises before anything is launched, engine/src/metal.mm:150-152). Tensors are torch
device tensors used as plain device memory; every op goes through the C ABI on torch's current stream.

The library must be built (krea_image_amd/csrc/Makefile, or __graft_entry__.build()); there is no
fallback path: a missing libkh.so raises ImportError-like KhError on first use.
"""
import ctypes
import os
from dataclasses import dataclass
from typing import Optional

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkh.so")

F32, F16, BF16, I8 = 0, 1, 2, 3
EPI = {"store16": 0, "f32": 1, "resid_gate": 2, "resid": 3, "swiglu": 4, "gelu": 5, "bias16": 6, "bias_f32": 7}
# reference spelling (enum class Epi, engine/src/metal.h:37-38)
Epi = type("Epi", (), {"BF16": 0, "STORE16": 0, "F32": 1, "ResidGate": 2, "Resid": 3, "SwiGLU": 4, "GELU": 5,
                       "BiasBF16": 6, "Bias16": 6, "BiasF32": 7})

_TORCH_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int8: I8}

# C-ABI symbols declared in include/kh.h (checked by tests/test_abi.py)
SYMBOLS = ["kh_version", "kh_gemm", "kh_attention"]


class KhError(RuntimeError):
    pass


class _WeightC(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("w_dtype", ctypes.c_int),
                ("s_dtype", ctypes.c_int), ("group", ctypes.c_int)]


_lib = None


def load():
    """Load libkh.so (no fallback: raises KhError if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise KhError(f"{LIB_PATH} is not built: run `make -C krea_image_amd/csrc` or __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        lib.kh_version.restype = ctypes.c_char_p
        vp, i = ctypes.c_void_p, ctypes.c_int
        lib.kh_gemm.argtypes = [vp, i, vp, i, ctypes.POINTER(_WeightC), vp, i, i, i, i, i, i, vp, ctypes.c_char_p, i]
        lib.kh_gemm.restype = i
        lib.kh_attention.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, i, i, i, i, i, i, i, vp, i, vp, vp,
                                     ctypes.c_char_p, i]
        lib.kh_attention.restype = i
        _lib = lib
    return _lib


def dtype_code(t: torch.dtype) -> int:
    return _TORCH_DT[t]


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(rc, err):
    if rc != 0:
        raise KhError(err.value.decode(errors="replace") or f"libkh error {rc}")


@dataclass
class Weight:
    """Input-major GEMM weight Wt[K, N] (engine/src/metal.h:25-29). w: int8 / fp16 / bf16 device tensor;
    s: scales — [K/group, N] for group < K, [N] for per-output-channel (group = K or 0)."""
    w: torch.Tensor
    s: Optional[torch.Tensor] = None
    group: int = 0

    @property
    def q8(self) -> bool:
        return self.w.dtype == torch.int8

    def c(self) -> _WeightC:
        return _WeightC(self.w.data_ptr(), 0 if self.s is None else self.s.data_ptr(), dtype_code(self.w.dtype),
                        F32 if self.s is None else dtype_code(self.s.dtype), self.group)


def gemm(epi, A: torch.Tensor, W: Weight, C: torch.Tensor, M: int, N: int, K: int, lda: int, ldw: int, ldc: int,
         vec: Optional[torch.Tensor] = None):
    """krea::Metal::gemm (engine/src/metal.mm:146-163): acc = A[M,K] x Wt[K,N], then epilogue `epi`."""
    lib = load()
    if isinstance(epi, str):
        epi = EPI[epi]
    err = ctypes.create_string_buffer(512)
    wc = W.c()
    rc = lib.kh_gemm(_stream(), epi, _ptr(A), dtype_code(A.dtype), ctypes.byref(wc), _ptr(C), M, N, K, lda, ldw, ldc,
                     _ptr(vec), err, 512)
    _check(rc, err)
    return C


def linear(epi, x: torch.Tensor, W: Weight, out: Optional[torch.Tensor] = None, vec=None):
    """Convenience: contiguous x [M, K] @ W -> out (allocated when None, except residual epilogues)."""
    M, K = x.shape
    N = W.w.shape[1]
    if isinstance(epi, str):
        epi = EPI[epi]
    if out is None:
        if epi in (EPI["resid"], EPI["resid_gate"]):
            raise KhError("residual epilogues need the f32 residual tensor as `out`")
        dt = torch.float32 if epi in (EPI["f32"], EPI["bias_f32"]) else x.dtype
        out = torch.empty(M, N // 2 if epi == EPI["swiglu"] else N, dtype=dt, device=x.device)
    return gemm(epi, x, W, out, M, N, K, x.stride(0), W.w.stride(0), out.stride(0), vec)


def attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, O: torch.Tensor, Lq: int, Lk: int, heads: int,
              ldq: int, ldk: int, ldv: int, ldo: int, group: int = 1, causal: bool = False, q_pos0: int = 0,
              G: Optional[torch.Tensor] = None, ldg: int = 0, QB: Optional[torch.Tensor] = None,
              KB: Optional[torch.Tensor] = None):
    """krea::Metal::attention (engine/src/metal.mm:193-202): flash attention, head dim 128. Tensors may be
    column views of a fused projection buffer (their data_ptr is the first element of head 0)."""
    lib = load()
    err = ctypes.create_string_buffer(512)
    rc = lib.kh_attention(_stream(), _ptr(Q), _ptr(K), _ptr(V), _ptr(O), dtype_code(Q.dtype), Lq, Lk, heads, ldq, ldk,
                          ldv, ldo, group, int(causal), q_pos0, _ptr(G), ldg, _ptr(QB), _ptr(KB), err, 512)
    _check(rc, err)
    return O
