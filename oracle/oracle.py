"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as
the checker of the HIP kernels and as the timed CPU baseline. The product path never imports it.

Arrays are numpy; 16-bit float tensors are passed as uint16 bit patterns (np.float16 arrays are accepted for
fp16 and viewed as uint16). dtype codes follow include/kh.h: 0 f32, 1 f16, 2 bf16, 3 i8.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

F32, F16, BF16, I8 = 0, 1, 2, 3
EPI = {"store16": 0, "f32": 1, "resid_gate": 2, "resid": 3, "swiglu": 4, "gelu": 5, "bias16": 6, "bias_f32": 7}

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.or_f32_to_f16.restype = ctypes.c_uint16
        _lib.or_f32_to_bf16.restype = ctypes.c_uint16
        _lib.or_f16_to_f32.restype = ctypes.c_float
        _lib.or_bf16_to_f32.restype = ctypes.c_float
        _lib.or_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.or_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.or_rms_norm.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int]
        _lib.or_qk_norm_rope.argtypes = ([ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 4 +
                                         [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int, ctypes.c_int] +
                                         [ctypes.c_void_p] * 2)
        vp, i = ctypes.c_void_p, ctypes.c_int
        _lib.or_vae_conv.argtypes = [vp, i, i, i, i, i, vp, vp, vp, i, vp]
        _lib.or_vae_norm_silu.argtypes = [vp, vp, vp, i, i, i]
        _lib.or_vae_unpack.argtypes = [vp] * 6 + [i, i]
        _lib.or_vae_softmax.argtypes = [vp, i, i, i, ctypes.c_float, vp]
        _lib.or_vae_conv_out.argtypes = [vp, i, vp, vp, vp, i, i]
        _lib.or_temb.argtypes = [ctypes.c_float, vp]
        _lib.or_make_fin.argtypes = [vp, vp, vp, i, vp]
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a):
    assert a is None or a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a


# ---- 16-bit conversions (vectorised through the C scalar routines' bulk forms) ----
def to_f32(bits, dtype):
    bits = np.ascontiguousarray(bits)
    if dtype == F32:
        return bits.astype(np.float32)
    if dtype == I8:
        return bits.astype(np.float32)
    out = np.empty(bits.shape, np.float32)
    lib().or_to_f32(_p(bits.view(np.uint16)), dtype, _p(out), ctypes.c_size_t(bits.size))
    return out


def from_f32(x, dtype):
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == F32:
        return x.copy()
    out = np.empty(x.shape, np.uint16)
    lib().or_from_f32(_p(x), dtype, _p(out), ctypes.c_size_t(x.size))
    return out


def round16(x, dtype):
    return to_f32(from_f32(x, dtype), dtype)


# ---- quantizers / layout ----
def quant_q8(w, group):
    """convert.py:92-99. w f32 [K, N] -> (int8 [K, N], f32 scales [K/group, N])."""
    w = np.ascontiguousarray(w, np.float32)
    K, N = w.shape
    q = np.empty((K, N), np.int8)
    s = np.empty((K // group, N), np.float32)
    if lib().or_quant_q8(_p(w), K, N, group, _p(q), _p(s)) != 0:
        raise ValueError("quant_q8: bad shape")
    return q, s


def quant_q8_channel_f16(w):
    """build_ane.py:79-80. w f32 [K, N] -> (int8 [K, N], fp16 bits [N])."""
    w = np.ascontiguousarray(w, np.float32)
    K, N = w.shape
    q = np.empty((K, N), np.int8)
    s = np.empty((N,), np.uint16)
    if lib().or_quant_q8_channel_f16(_p(w), K, N, _p(q), _p(s)) != 0:
        raise ValueError("quant_q8_channel_f16: bad shape")
    return q, s


def interleave_gate_up(gate, up):
    gate, up = np.ascontiguousarray(gate), np.ascontiguousarray(up)
    F, D = gate.shape
    out = np.empty((2 * F, D), gate.dtype)
    if lib().or_interleave_gate_up(_p(gate), _p(up), F, D, gate.itemsize, _p(out)) != 0:
        raise ValueError("interleave: F % 32 != 0")
    return out


def deinterleave_gate_up(gu):
    gu = np.ascontiguousarray(gu)
    F2, D = gu.shape
    g = np.empty((F2 // 2, D), gu.dtype)
    u = np.empty((F2 // 2, D), gu.dtype)
    if lib().or_deinterleave_gate_up(_p(gu), F2 // 2, D, gu.itemsize, _p(g), _p(u)) != 0:
        raise ValueError("deinterleave: F % 32 != 0")
    return g, u


# ---- ops ----
def gemm(epi, A, a_dtype, w, w_dtype, s=None, s_dtype=F32, group=0, C=None, vec=None, N=None, threads=0):
    """Metal::gemm semantics (see oracle.h). A: uint16 bits [M, K]; w: int8 or uint16 bits [K, N].
    C is updated in place for the residual epilogues and returned."""
    A, w = _c(A), _c(w)
    M, K = A.shape
    N = w.shape[1] if N is None else N
    if w_dtype == I8 and group == 0:
        group = K
    if C is None:
        if epi in (EPI["f32"], EPI["bias_f32"], EPI["resid"], EPI["resid_gate"]):
            C = np.zeros((M, N), np.float32)
        else:
            C = np.zeros((M, N // 2 if epi == EPI["swiglu"] else N), np.uint16)
    _c(C)
    ldc = C.shape[1]
    if vec is not None:
        vec = np.ascontiguousarray(vec, np.float32)
    if s is not None:
        s = np.ascontiguousarray(s)
    rc = lib().or_gemm(epi, _p(A), a_dtype, _p(w), w_dtype, _p(s), s_dtype, group, _p(C), M, N, K, A.shape[1],
                       w.shape[1], ldc, _p(vec), threads)
    if rc != 0:
        raise ValueError("oracle gemm: unsupported shape")
    return C


def gemv(x, w, w_dtype, s=None, s_dtype=F32, group=0, y=None, act=0, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    rows, K = x.shape
    N = w.shape[1]
    if w_dtype == I8 and group == 0:
        group = K
    if y is None:
        y = np.zeros((rows, N), np.float32)
    if bias is not None:
        bias = np.ascontiguousarray(bias, np.float32)
    rc = lib().or_gemv(_p(x), _p(_c(w)), w_dtype, _p(s), s_dtype, group, _p(y), rows, N, K, w.shape[1], act,
                       _p(bias))
    if rc != 0:
        raise ValueError("oracle gemv: bad shape")
    return y


def temb(sigma: float) -> np.ndarray:
    """Timestep embedding of Conditioning::compute (engine/src/model.mm:576-581): f32 [256] of bf16(sigma)."""
    e = np.empty(256, np.float32)
    lib().or_temb(float(sigma), _p(e))
    return e


def make_fin(t, lin, nf):
    """Final-norm vectors of DiT::make_cond (engine/src/model.mm:340-346): f32 [2, D]."""
    D = nf.shape[0]
    fin = np.empty((2, D), np.float32)
    lib().or_make_fin(_p(np.ascontiguousarray(t, np.float32)), _p(np.ascontiguousarray(lin, np.float32)),
                      _p(np.ascontiguousarray(nf, np.float32)), D, _p(fin))
    return fin


def conditioning(sigma: float, w1, b1, w2, b2, wp, bp):
    """Conditioning::compute (engine/src/model.mm:571-591): (t [D], tvec [6 D]) f32 from the f32 tmlp1 [256, D],
    tmlp2 [D, D], tproj [D, 6 D] weights (input-major) and biases, as a composition of the oracle's gemv
    (GELU(tanh) on load, act bit 2) on temb(sigma)."""
    e = temb(sigma)[None]
    h = gemv(e, np.ascontiguousarray(w1, np.float32), F32, bias=b1)
    t = gemv(h, np.ascontiguousarray(w2, np.float32), F32, bias=b2, act=4)
    tvec = gemv(t, np.ascontiguousarray(wp, np.float32), F32, bias=bp, act=4)
    return t[0], tvec[0]


def make_cond(tvec, table, n1, n2):
    D = n1.shape[0]
    mods = np.empty((6, D), np.float32)
    tvec = np.ascontiguousarray(tvec, np.float32)
    table = None if table is None else np.ascontiguousarray(table, np.float32)
    lib().or_make_cond(_p(tvec), _p(table), _p(np.ascontiguousarray(n1, np.float32)),
                       _p(np.ascontiguousarray(n2, np.float32)), D, _p(mods))
    return mods


def rms_norm(x, mul, add, out_dtype, eps=1e-5, center=0):
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    y = np.empty((rows, width), np.float32 if out_dtype == F32 else np.uint16)
    lib().or_rms_norm(_p(x), _p(np.ascontiguousarray(mul, np.float32)),
                      _p(None if add is None else np.ascontiguousarray(add, np.float32)), _p(y), out_dtype, rows,
                      width, width, width, eps, center)
    return y


def qk_norm_rope(qkv, dtype, wq, wk, cosb, sinb, q_off, n_q, k_off, n_k, eps=1e-5, rope_mode=0, big_dim=-1):
    """In place on a copy of qkv (uint16 bits [rows, ld]); returns (qkv, qbig, kbig)."""
    qkv = np.array(qkv, copy=True)
    rows, ld = qkv.shape
    qbig = np.zeros((rows, max(n_q, 1)), np.float32)
    kbig = np.zeros((rows, max(n_k, 1)), np.float32)
    lib().or_qk_norm_rope(_p(qkv), dtype, _p(np.ascontiguousarray(wq, np.float32)),
                          _p(np.ascontiguousarray(wk, np.float32)),
                          _p(None if cosb is None else np.ascontiguousarray(cosb, np.float32)),
                          _p(None if sinb is None else np.ascontiguousarray(sinb, np.float32)), rows, ld, q_off, n_q,
                          k_off, n_k, eps, rope_mode, big_dim, _p(qbig), _p(kbig))
    return qkv, qbig, kbig


def sigmas(steps, mu=1.15):
    out = np.empty(steps + 1, np.float32)
    lib().or_sigmas(steps, ctypes.c_float(mu), _p(out))
    return out


def euler_step(z, v, dt):
    z = np.array(z, np.float32, copy=True)
    lib().or_euler_step(_p(z), _p(np.ascontiguousarray(v, np.float32)), ctypes.c_longlong(z.size), ctypes.c_float(dt))
    return z


def cfg_combine(vc, vn, scale):
    vc = np.array(vc, np.float32, copy=True)
    lib().or_cfg_combine(_p(vc), _p(np.ascontiguousarray(vn, np.float32)), ctypes.c_longlong(vc.size),
                         ctypes.c_float(scale))
    return vc


def rope_tables(T, H, W, mode):
    R = T + H * W
    c = np.empty((R, 64), np.float32)
    s = np.empty((R, 64), np.float32)
    lib().or_rope_tables(T, H, W, mode, _p(c), _p(s))
    return c, s


def attention(Q, K, V, dtype, heads, group=1, causal=0, q_pos0=0, G=None, QB=None, KB=None, threads=0):
    """Q [Lq, ldq], K [Lk, ldk], V [Lk, ldv] uint16 bits with heads at column h*128 (kv head h // group)."""
    Q, K, V = _c(Q), _c(K), _c(V)
    Lq, Lk = Q.shape[0], K.shape[0]
    O = np.zeros((Lq, heads * 128), np.uint16)
    lib().or_attention(_p(Q), _p(K), _p(V), _p(O), dtype, Lq, Lk, heads, Q.shape[1], K.shape[1], V.shape[1],
                       heads * 128, group, causal, q_pos0, _p(G), 0 if G is None else G.shape[1],
                       _p(None if QB is None else np.ascontiguousarray(QB, np.float32)),
                       _p(None if KB is None else np.ascontiguousarray(KB, np.float32)), threads)
    return O


# ---- VAE decoder ops (engine/kernels/vae.metal); bf16 tensors as uint16 bit patterns ----
def vae_conv(x, H, W, w, bias, N, ks=3, up=0, res=None):
    """x [Hin*Win, Cin] bf16 -> [H*W, N] bf16; w [ks*ks*Cin, N] bf16, bias [N] f32 (vae.metal:5-128)."""
    x = np.ascontiguousarray(x, np.uint16)
    Cin = x.shape[1]
    y = np.empty((H * W, N), np.uint16)
    lib().or_vae_conv(_p(x), H, W, Cin, ks, up, _p(np.ascontiguousarray(w, np.uint16)),
                      _p(np.ascontiguousarray(bias, np.float32)),
                      _p(None if res is None else np.ascontiguousarray(res, np.uint16)), N, _p(y))
    return y


def vae_subpix_weights(w, Cin, Cout):
    """Sub-pixel weights of nearest-2x + 3x3 (engine/kernels/vae.metal:134-160): W2 [4 Cin, 4 Cout] bf16 bits,
    W2[(2r + s) Cin + ci, (2py + px) Cout + co] = bf16(fp32 sum, in (ky, kx) order, of the taps W[ky, kx] with
    ky in [0, py] for r = 0 and [1 + py, 2] for r = 1, kx likewise)."""
    wf = to_f32(np.asarray(w, np.uint16), BF16).reshape(3, 3, Cin, Cout)
    W2 = np.zeros((4 * Cin, 4 * Cout), np.float32)
    for ph in range(4):
        py, px = ph >> 1, ph & 1
        for t in range(4):
            r, sc = t >> 1, t & 1
            y0, y1 = (1 + py, 2) if r else (0, py)
            x0, x1 = (1 + px, 2) if sc else (0, px)
            acc = np.zeros((Cin, Cout), np.float32)
            for ky in range(y0, y1 + 1):
                for kx in range(x0, x1 + 1):
                    acc = acc + wf[ky, kx]
            W2[t * Cin:(t + 1) * Cin, ph * Cout:(ph + 1) * Cout] = acc
    return from_f32(W2, BF16)


def vae_conv_up2(x, H, W, w2, bias, Cout):
    """conv3x3(nearest2x(x)) as four 2x2 sub-pixel convs (engine/src/vae.mm:137-150, vconv mode 2): x [H W, Cin]
    bf16 low-res, w2 from vae_subpix_weights, bias [Cout] f32 -> y [(2H)(2W), Cout] bf16. Phase (py, px) is a
    3x3 conv of x whose taps at offsets (r + py - 1, s + px - 1) hold W2's 2x2 taps and the rest are zero."""
    x = np.ascontiguousarray(x, np.uint16)
    Cin = x.shape[1]
    w2 = np.asarray(w2, np.uint16)
    y = np.empty((2 * H, 2 * W, Cout), np.uint16)
    for ph in range(4):
        py, px = ph >> 1, ph & 1
        k3 = np.zeros((3, 3, Cin, Cout), np.uint16)
        for t in range(4):
            r, sc = t >> 1, t & 1
            k3[r + py, sc + px] = w2[t * Cin:(t + 1) * Cin, ph * Cout:(ph + 1) * Cout]
        yp = vae_conv(x, H, W, k3.reshape(9 * Cin, Cout), bias, Cout, ks=3)
        y[py::2, px::2] = yp.reshape(H, W, Cout)
    return y.reshape(4 * H * W, Cout)


def vae_norm_silu(x, gamma, silu=1):
    x = np.ascontiguousarray(x, np.uint16)
    y = np.empty_like(x)
    lib().or_vae_norm_silu(_p(x), _p(np.ascontiguousarray(gamma, np.float32)), _p(y), x.shape[0], x.shape[1], silu)
    return y


def vae_unpack(z, mean, stdv, w, b, H16, W16):
    y = np.empty((4 * H16 * W16, 16), np.uint16)
    f = lambda a: np.ascontiguousarray(a, np.float32)  # noqa: E731
    lib().or_vae_unpack(_p(f(z)), _p(f(mean)), _p(f(stdv)), _p(f(w)), _p(f(b)), _p(y), H16, W16)
    return y


def vae_softmax(S, n, scale):
    S = np.ascontiguousarray(S, np.float32)
    P = np.zeros(S.shape, np.uint16)
    lib().or_vae_softmax(_p(S), S.shape[1], S.shape[0], n, scale, _p(P))
    return P


def vae_conv_out(x, w, bias, H, W):
    x = np.ascontiguousarray(x, np.uint16)
    rgba = np.empty((H * W, 4), np.uint8)
    lib().or_vae_conv_out(_p(x), x.shape[1], _p(np.ascontiguousarray(w, np.uint16)),
                          _p(np.ascontiguousarray(bias, np.float32)), _p(rgba), H, W)
    return rgba
