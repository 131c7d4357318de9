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

F32, F16, BF16, I8, I8P = 0, 1, 2, 3, 4  # I8P: int8 in the packed layout of pack_int8
EPI = {"store16": 0, "f32": 1, "resid_gate": 2, "resid": 3, "swiglu": 4, "gelu": 5, "bias16": 6, "bias_f32": 7}
# reference spelling (enum class Epi, engine/src/metal.h:37-38)
Epi = type("Epi", (), {"BF16": 0, "STORE16": 0, "F32": 1, "ResidGate": 2, "Resid": 3, "SwiGLU": 4, "GELU": 5,
                       "BiasBF16": 6, "Bias16": 6, "BiasF32": 7})

_TORCH_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int8: I8}

# C-ABI symbols declared in include/kh.h (checked by tests/test_abi.py)
SYMBOLS = ["kh_version", "kh_gemm", "kh_attention", "kh_rms_norm", "kh_qk_norm_rope", "kh_gemv", "kh_make_cond",
           "kh_gemm_f32", "kh_rope_tables", "kh_dit_layer_forward", "kh_dit_forward",
           "kh_qw_open", "kh_qw_close", "kh_qw_count", "kh_qw_version", "kh_qw_meta", "kh_qw_at", "kh_qw_find",
           "kh_qw_upload", "kh_stream_create", "kh_stream_destroy", "kh_stream_sync", "kh_alloc", "kh_free",
           "kh_upload", "kh_download", "kh_vae_conv3x3", "kh_vae_subpix_weights", "kh_vae_conv_up2", "kh_vae_im2col", "kh_vae_norm_silu", "kh_vae_unpack", "kh_vae_softmax",
           "kh_vae_conv_out", "kh_vae_workspace_bytes", "kh_vae_decode", "kh_gemm_qk_norm_rope",
           "kh_pack_int8", "kh_sigmas", "kh_euler_step", "kh_cfg_combine", "kh_copy", "kh_make_fin", "kh_conditioning",
           "kh_gemm_ws", "kh_gemm_workspace_bytes", "kh_gemm_workspace_init", "kh_gemm_static",
           "kh_gemm_plan"]


class KhError(RuntimeError):
    pass


class _WeightC(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("w_dtype", ctypes.c_int),
                ("s_dtype", ctypes.c_int), ("group", ctypes.c_int)]


class DitConfig(ctypes.Structure):
    """kh_dit_config (include/kh.h)."""
    _fields_ = [("dim", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("ff", ctypes.c_int),
                ("mlp", ctypes.c_int), ("attn_gate", ctypes.c_int), ("norm_center", ctypes.c_int),
                ("rope_mode", ctypes.c_int), ("dtype", ctypes.c_int), ("eps", ctypes.c_float)]


class DitLayerC(ctypes.Structure):
    """kh_dit_layer (include/kh.h)."""
    _fields_ = [("qkv", _WeightC), ("o", _WeightC), ("up", _WeightC), ("down", _WeightC), ("ada", _WeightC),
                ("ada_bias", ctypes.c_void_p), ("mod_table", ctypes.c_void_p), ("n1", ctypes.c_void_p),
                ("n2", ctypes.c_void_p), ("qn", ctypes.c_void_p), ("kn", ctypes.c_void_p), ("big_dim", ctypes.c_int)]


class DitStateC(ctypes.Structure):
    """kh_dit_state (include/kh.h)."""
    _fields_ = [("x", ctypes.c_void_p), ("h", ctypes.c_void_p), ("qkv", ctypes.c_void_p), ("ao", ctypes.c_void_p),
                ("mid", ctypes.c_void_p), ("tvec", ctypes.c_void_p), ("mods", ctypes.c_void_p),
                ("cond", ctypes.c_void_p), ("cond_dim", ctypes.c_int), ("cosb", ctypes.c_void_p),
                ("sinb", ctypes.c_void_p), ("qbig", ctypes.c_void_p), ("kbig", ctypes.c_void_p),
                ("gemm_ws", ctypes.c_void_p), ("gemm_ws_bytes", ctypes.c_size_t)]


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
        lib.kh_gemm_ws.argtypes = [vp, i, vp, i, ctypes.POINTER(_WeightC), vp, i, i, i, i, i, i, vp, vp,
                                   ctypes.c_size_t, ctypes.c_char_p, i]
        lib.kh_gemm_ws.restype = i
        lib.kh_gemm_static.argtypes = [vp, i, vp, i, ctypes.POINTER(_WeightC), vp, i, i, i, i, i, i, vp,
                                       ctypes.c_char_p, i]
        lib.kh_gemm_static.restype = i
        lib.kh_gemm_workspace_bytes.argtypes, lib.kh_gemm_workspace_bytes.restype = [], ctypes.c_size_t
        lib.kh_gemm_plan.argtypes = [i, i, i, i, i, i, i, ctypes.POINTER(ctypes.c_int), ctypes.c_char_p, i]
        lib.kh_gemm_plan.restype = i
        lib.kh_gemm_workspace_init.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_char_p, i]
        lib.kh_gemm_workspace_init.restype = i
        lib.kh_attention.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, i, i, i, i, i, i, i, vp, i, vp, vp,
                                     ctypes.c_char_p, i]
        lib.kh_attention.restype = i
        f = ctypes.c_float
        cp = ctypes.c_char_p
        lib.kh_rms_norm.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, i, f, i, cp, i]
        lib.kh_qk_norm_rope.argtypes = [vp, vp, i, vp, vp, vp, vp, i, i, i, i, i, i, f, i, i, vp, vp, cp, i]
        lib.kh_gemv.argtypes = [vp, vp, ctypes.POINTER(_WeightC), vp, i, i, i, i, i, vp, cp, i]
        lib.kh_make_cond.argtypes = [vp, vp, vp, vp, vp, i, vp, cp, i]
        lib.kh_gemm_f32.argtypes = [vp, vp, vp, vp, i, i, i, i, i, i, i, vp, cp, i]
        lib.kh_make_fin.argtypes, lib.kh_make_fin.restype = [vp, vp, vp, vp, i, vp, cp, i], i
        lib.kh_conditioning.argtypes = [vp, vp, i, f, vp, vp, vp, ctypes.c_size_t, ctypes.POINTER(i), cp, i]
        lib.kh_conditioning.restype = i
        lib.kh_gemm_qk_norm_rope.argtypes = ([vp, vp, i, ctypes.POINTER(_WeightC), vp] + [i] * 6 + [vp] * 4 +
                                             [i] * 4 + [ctypes.c_float, i, i, vp, vp, vp, ctypes.c_size_t, cp, i])
        lib.kh_gemm_qk_norm_rope.restype = i
        lib.kh_pack_int8.argtypes, lib.kh_pack_int8.restype = [vp, vp, i, i, vp, cp, i], i
        lib.kh_sigmas.argtypes, lib.kh_sigmas.restype = [i, ctypes.c_float, vp], i
        ll = ctypes.c_longlong
        lib.kh_euler_step.argtypes, lib.kh_euler_step.restype = [vp, vp, vp, ll, ctypes.c_float, cp, i], i
        lib.kh_cfg_combine.argtypes, lib.kh_cfg_combine.restype = [vp, vp, vp, ll, ctypes.c_float, cp, i], i
        lib.kh_rope_tables.argtypes = [i, i, i, i, vp, vp]
        lib.kh_dit_layer_forward.argtypes = [vp, ctypes.POINTER(DitConfig), ctypes.POINTER(DitLayerC),
                                             ctypes.POINTER(DitStateC), i, cp, i]
        lib.kh_dit_forward.argtypes = [vp, ctypes.POINTER(DitConfig), ctypes.POINTER(DitLayerC), i,
                                       ctypes.POINTER(DitStateC), i, cp, i]
        for name in SYMBOLS[2:11]:
            getattr(lib, name).restype = i
        sz = ctypes.c_size_t
        lib.kh_stream_create.argtypes, lib.kh_stream_create.restype = [ctypes.POINTER(vp), cp, i], i
        lib.kh_stream_destroy.argtypes, lib.kh_stream_destroy.restype = [vp], i
        lib.kh_stream_sync.argtypes, lib.kh_stream_sync.restype = [vp, cp, i], i
        lib.kh_alloc.argtypes, lib.kh_alloc.restype = [ctypes.POINTER(vp), sz, cp, i], i
        lib.kh_free.argtypes, lib.kh_free.restype = [vp], i
        lib.kh_upload.argtypes = lib.kh_download.argtypes = [vp, vp, vp, sz, cp, i]
        lib.kh_upload.restype = lib.kh_download.restype = i
        lib.kh_copy.argtypes, lib.kh_copy.restype = [vp, vp, vp, sz, cp, i], i
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
    s: scales — [K/group, N] for group < K, [N] for per-output-channel (group = K or 0).
    packed: w holds int8 in the layout of pack_int8 (kh_gemm reads it as KH_I8P; same results bitwise)."""
    w: torch.Tensor
    s: Optional[torch.Tensor] = None
    group: int = 0
    packed: bool = False

    @property
    def q8(self) -> bool:
        return self.w.dtype == torch.int8

    def c(self) -> _WeightC:
        return _WeightC(self.w.data_ptr(), 0 if self.s is None else self.s.data_ptr(),
                        I8P if self.packed else dtype_code(self.w.dtype),
                        F32 if self.s is None else dtype_code(self.s.dtype), self.group)

    def pack(self) -> "Weight":
        """The same weight in kh_gemm's packed int8 layout (a new device buffer; scales shared)."""
        if self.packed:
            return self
        return Weight(pack_int8(self.w), self.s, self.group, True)


def pack_int8(w: torch.Tensor) -> torch.Tensor:
    """kh_pack_int8: int8 Wt[K, ldw] (contiguous) -> the packed layout, a new tensor of the same shape."""
    if w.dtype != torch.int8 or w.dim() != 2 or not w.is_contiguous():
        raise KhError("pack_int8: expects a contiguous 2-D int8 tensor")
    out = torch.empty_like(w)
    _call(load().kh_pack_int8, _stream(), _ptr(w), w.shape[0], w.shape[1], _ptr(out))
    return out


_F32_OUT_EPI = (1, 2, 3, 7)  # F32, RESID_GATE, RESID, BIAS_F32


def _bytes_after(t) -> int:
    """Bytes of t's storage from t's first element to the end (what a raw-pointer kernel may touch)."""
    if not isinstance(t, torch.Tensor):
        return 1 << 62  # raw device addresses (uploaded weight files) are the caller's responsibility
    st = t.untyped_storage()
    return st.nbytes() - (t.data_ptr() - st.data_ptr())


def _need(t, name: str, rows: int, cols: int, ld: int, esize: int):
    need = ((rows - 1) * ld + cols) * esize if rows > 0 and cols > 0 else 0
    if _bytes_after(t) < need:
        raise KhError(f"gemm: {name} holds {_bytes_after(t)} bytes, the call addresses {need}")


def gemm_workspace(dev=None) -> torch.Tensor:
    """A kh_gemm_ws workspace for the current device (kh_gemm_workspace_bytes, prepared by
    kh_gemm_workspace_init): uint8 device tensor, owned by the caller; one stream at a time may use it."""
    lib = load()
    n = lib.kh_gemm_workspace_bytes()
    ws = torch.empty(max(int(n), 256), dtype=torch.uint8, device=dev or "cuda")
    if n:
        _call(lib.kh_gemm_workspace_init, _stream(), _ptr(ws), ws.numel())
    return ws


def gemm(epi, A: torch.Tensor, W: Weight, C: torch.Tensor, M: int, N: int, K: int, lda: int, ldw: int, ldc: int,
         vec: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None):
    """krea::Metal::gemm (engine/src/metal.mm:146-163): acc = A[M,K] x Wt[K,N], then epilogue `epi`; with `ws`
    (gemm_workspace()) through kh_gemm_ws, which may run stream-K. Tensor arguments are checked on the host
    (dtype of C for the epilogue, storage covering every strided row) so a mis-sized buffer raises instead of
    reaching the device."""
    lib = load()
    if isinstance(epi, str):
        epi = EPI[epi]
    if isinstance(C, torch.Tensor) and isinstance(A, torch.Tensor):
        want = torch.float32 if epi in _F32_OUT_EPI else A.dtype
        if C.dtype != want:
            raise KhError(f"gemm: epilogue {epi} writes {want}, C is {C.dtype}")
        _need(A, "A", M, K, lda, A.element_size())
        _need(C, "C", M, N // 2 if epi == EPI["swiglu"] else N, ldc, C.element_size())
        if W.packed:  # 8-row panels of 8 ldw bytes; columns [0, N) end at byte 8 N of the last panel
            if _bytes_after(W.w) < (K - 8) * ldw + 8 * N:
                raise KhError(f"gemm: W holds {_bytes_after(W.w)} bytes, the call addresses {(K - 8) * ldw + 8 * N}")
        else:
            _need(W.w, "W", K, N, ldw, 1 if W.w.dtype == torch.int8 else 2)
        if vec is not None:
            _need(vec, "vec", 1, N, N, 4)
    err = ctypes.create_string_buffer(512)
    wc = W.c()
    if ws is None:
        rc = lib.kh_gemm(_stream(), epi, _ptr(A), dtype_code(A.dtype), ctypes.byref(wc), _ptr(C), M, N, K, lda, ldw,
                         ldc, _ptr(vec), err, 512)
    else:
        rc = lib.kh_gemm_ws(_stream(), epi, _ptr(A), dtype_code(A.dtype), ctypes.byref(wc), _ptr(C), M, N, K, lda,
                            ldw, ldc, _ptr(vec), _ptr(ws), ws.numel() * ws.element_size(), err, 512)
    _check(rc, err)
    return C


def linear(epi, x: torch.Tensor, W: Weight, out: Optional[torch.Tensor] = None, vec=None, ws=None):
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
    return gemm(epi, x, W, out, M, N, K, x.stride(0), W.w.stride(0), out.stride(0), vec, ws)


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


def _call(fn, *args):
    err = ctypes.create_string_buffer(512)
    rc = fn(*args, err, 512)
    _check(rc, err)


def rms_norm(x: torch.Tensor, mul: torch.Tensor, add: Optional[torch.Tensor], y: torch.Tensor, rows: int, width: int,
             ld_in: int, ld_out: int, eps: float, center: int = 0):
    """krea::Metal::rms_norm (engine/src/metal.h:72-74): y = norm(x) * mul (+ add); center = 1 -> LayerNorm."""
    _call(load().kh_rms_norm, _stream(), _ptr(x), _ptr(mul), _ptr(add), _ptr(y), dtype_code(y.dtype), rows, width,
          ld_in, ld_out, eps, center)
    return y


def qk_norm_rope(qkv: torch.Tensor, wq, wk, cos, sin, rows: int, ld: int, q_off: int, n_q: int, k_off: int, n_k: int,
                 eps: float, rope_mode: int, big_dim: int = -1, qbig=None, kbig=None):
    """krea::Metal::qk_norm_rope (engine/src/metal.h:77-79): per-head RMSNorm + RoPE in place."""
    _call(load().kh_qk_norm_rope, _stream(), _ptr(qkv), dtype_code(qkv.dtype), _ptr(wq), _ptr(wk), _ptr(cos),
          _ptr(sin), rows, ld, q_off, n_q, k_off, n_k, eps, rope_mode, big_dim, _ptr(qbig), _ptr(kbig))
    return qkv


def gemm_qk_norm_rope(A: torch.Tensor, W: Weight, C: torch.Tensor, M: int, N: int, K: int, lda: int, ldw: int,
                      ldc: int, wq, wk, cos, sin, q_off: int, n_q: int, k_off: int, n_k: int, eps: float,
                      rope_mode: int, big_dim: int = -1, qbig=None, kbig=None, ws=None):
    """The QKV projection of DiT::layer (engine/src/model.mm:373-375) as one launch: kh_gemm STORE16 with
    kh_qk_norm_rope fused into its epilogue (C plays qkv); ws: stream-K workspace (gemm_workspace) or None."""
    if C.dtype != A.dtype:
        raise KhError(f"gemm_qk_norm_rope: C must be {A.dtype}")
    _need(A, "A", M, K, lda, A.element_size())
    _need(C, "C", M, N, ldc, C.element_size())
    _need(W.w, "W", K, N, ldw, 1 if W.w.dtype == torch.int8 else 2)
    wc = W.c()
    _call(load().kh_gemm_qk_norm_rope, _stream(), _ptr(A), dtype_code(A.dtype), ctypes.byref(wc), _ptr(C), M, N, K,
          lda, ldw, ldc, _ptr(wq), _ptr(wk), _ptr(cos), _ptr(sin), q_off, n_q, k_off, n_k, eps, rope_mode, big_dim,
          _ptr(qbig), _ptr(kbig), _ptr(ws), 0 if ws is None else ws.numel() * ws.element_size())
    return C


def gemv(x: torch.Tensor, W: Weight, y: torch.Tensor, rows: int, N: int, K: int, ldw: int, act: int = 0, bias=None):
    """gemv_bf16 semantics (engine/kernels/gemm.metal:346-371): y (+)= act(x) W~ + bias; act bit 0 SiLU on load,
    bit 1 accumulate, bit 2 GELU(tanh) on load (the f32 linears of Conditioning::compute)."""
    wc = W.c()
    _call(load().kh_gemv, _stream(), _ptr(x), ctypes.byref(wc), _ptr(y), rows, N, K, ldw, act, _ptr(bias))
    return y


def make_cond(tvec, table, n1, n2, D: int, mods):
    """DiT::make_cond (engine/src/model.mm:317-347) for one layer, on the device."""
    _call(load().kh_make_cond, _stream(), _ptr(tvec), _ptr(table), _ptr(n1), _ptr(n2), D, _ptr(mods))
    return mods


def make_fin(t, lin, nf, D: int, fin):
    """The final-norm half of DiT::make_cond (engine/src/model.mm:340-346): fin [2, D] from t [D], last.mod
    [2, D] and last.n [D], on the device."""
    _call(load().kh_make_fin, _stream(), _ptr(t), _ptr(lin), _ptr(nf), D, _ptr(fin))
    return fin


def gemm_f32(A, W, C, M: int, N: int, K: int, lda: int, ldw: int, ldc: int, mode: int, bias=None):
    """krea::Metal::gemm_f32 (engine/src/metal.h:70-71): mode 1 bias, 2 GELU, 4 accumulate."""
    _call(load().kh_gemm_f32, _stream(), _ptr(A), _ptr(W), _ptr(C), M, N, K, lda, ldw, ldc, mode, _ptr(bias))
    return C


def rope_tables(T: int, H: int, W: int, mode: int):
    """Host RoPE tables (cos, sin) as float32 CPU tensors [T + H*W, 64]."""
    R = T + H * W
    c = torch.empty(R, 64, dtype=torch.float32)
    s = torch.empty(R, 64, dtype=torch.float32)
    if load().kh_rope_tables(T, H, W, mode, ctypes.c_void_p(c.data_ptr()), ctypes.c_void_p(s.data_ptr())) != 0:
        raise KhError("rope_tables: bad arguments")
    return c, s


def sigmas(steps: int, mu: float = 1.15):
    """krea_sigmas (engine/src/model.mm:594-602), on the host: numpy f32 [steps + 1], 1 -> 0."""
    import numpy as np
    out = np.empty(steps + 1, np.float32)
    if load().kh_sigmas(steps, mu, out.ctypes.data) != 0:
        raise KhError(f"sigmas: steps={steps} must be positive")
    return out


def _f32_flat(t, name):
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise KhError(f"{name}: expects a contiguous float32 tensor")
    return t.numel()


def euler_step(z: torch.Tensor, v: torch.Tensor, dt: float):
    """Metal::euler_step (engine/src/metal.mm:232-235): z += dt v in place (f32)."""
    n = _f32_flat(z, "euler_step")
    if _f32_flat(v, "euler_step") != n:
        raise KhError("euler_step: z and v differ in size")
    _call(load().kh_euler_step, _stream(), _ptr(z), _ptr(v), n, dt)
    return z


def cfg_combine(vc: torch.Tensor, vn: torch.Tensor, scale: float):
    """cfg_combine (engine/kernels/norm.metal:259-262): vc += scale (vc - vn) in place (f32)."""
    n = _f32_flat(vc, "cfg_combine")
    if _f32_flat(vn, "cfg_combine") != n:
        raise KhError("cfg_combine: vc and vn differ in size")
    _call(load().kh_cfg_combine, _stream(), _ptr(vc), _ptr(vn), n, scale)
    return vc
