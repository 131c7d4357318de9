"""Pins the CPU oracle (oracle/oracle.c) against references independent of it: numpy / torch in float64,
closed-form special cases, invariants, and the golden fixtures of tests/golden (computed by numpy, not by
the oracle). CPU only."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import rel_l2

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ---------------------------------------------------------------------------------------------- conversions
def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 300,
                        rng.standard_normal(2000).astype(np.float32) * 1e-6,    # subnormals
                        np.array([65504, 65519, 65520, 1e9, -1e9, 0.0, -0.0, 2.0 ** -24, 2.0 ** -25,
                                  3 * 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11], np.float32)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.from_f32(x, O.F16), ref)
    assert np.array_equal(O.to_f32(ref, O.F16), ref.view(np.float16).astype(np.float32))


def test_bf16_conversion_matches_torch_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 1e3,
                        np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8), 3.0e38], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.from_f32(x, O.BF16), ref)
    # ties to even: 1 + 2^-8 -> 1.0, 1 + 3 * 2^-8 -> 1 + 2^-6
    assert O.to_f32(O.from_f32(np.array([1 + 2.0 ** -8], np.float32), O.BF16), O.BF16)[0] == 1.0
    assert O.to_f32(O.from_f32(np.array([1 + 3 * 2.0 ** -8], np.float32), O.BF16), O.BF16)[0] == 1 + 2.0 ** -6


# ---------------------------------------------------------------------------------------------- quantizers
def test_quant_q8_known_answers():
    g = gold("q8.npz")
    q, s = O.quant_q8(g["w"], int(g["group"]))
    assert np.array_equal(q, g["q"]) and np.allclose(s, g["s"], rtol=0, atol=0)
    # hand-computed: column 0 has scale 1 and ties -63.5 -> -64, 0.5 -> 0, 1.5 -> 2, -2.5 -> -2 (half to even)
    assert s[0, 0] == 1.0 and s[0, 2] == 2.0 and s[0, 1] == np.float32(1e-12) / np.float32(127)
    assert list(q[:5, 0]) == [127, -64, 0, 2, -2]
    assert not q[:, 1].any()                       # zero column stays zero
    assert q[0, 2] == -127 and q[1, 2] == 50       # amax from a negative entry: 100 / 2 = 50
    q2, s2 = O.quant_q8(g["w_rand"], 128)
    assert np.array_equal(q2, g["q_rand"]) and np.array_equal(s2, g["s_rand"])


def test_quant_q8_dequant_error_bound():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((512, 96)).astype(np.float32)
    q, s = O.quant_q8(w, 128)
    deq = q.astype(np.float32).reshape(4, 128, 96) * s[:, None, :]
    err = np.abs(deq.reshape(512, 96) - w)
    assert (err <= 0.5 * np.repeat(s, 128, axis=0) * (1 + 1e-6)).all()   # half a quantum, by construction
    assert np.abs(q).max() == 127


def test_quant_q8_channel_f16_matches_numpy():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((256, 40)) * 0.05).astype(np.float32)
    q, s16 = O.quant_q8_channel_f16(w)
    s = np.maximum(np.abs(w).max(axis=0), np.float32(1e-12)) / np.float32(127)   # build_ane.py:79-80
    assert np.array_equal(q, np.clip(np.rint(w / s), -127, 127).astype(np.int8))
    assert np.array_equal(s16, s.astype(np.float16).view(np.uint16))


def test_interleave_gate_up_map_and_roundtrip():
    F, Dm = 96, 5
    gate = np.arange(F * Dm, dtype=np.int32).reshape(F, Dm)
    up = -gate - 1
    gu = O.interleave_gate_up(gate, up)
    for t in range(F // 32):
        for i in range(32):
            assert np.array_equal(gu[64 * t + i], gate[32 * t + i])
            assert np.array_equal(gu[64 * t + 32 + i], up[32 * t + i])
    g2, u2 = O.deinterleave_gate_up(gu)
    assert np.array_equal(g2, gate) and np.array_equal(u2, up)
    with pytest.raises(ValueError):
        O.interleave_gate_up(gate[:40], up[:40])


# ---------------------------------------------------------------------------------------------- GEMM
def _acc64(A, a_dtype, w, w_dtype, s, s_dtype, group):
    a = O.to_f32(A, a_dtype).astype(np.float64)
    if w_dtype == O.I8:
        wq = w.astype(np.float64)
        sv = O.to_f32(s, s_dtype).astype(np.float64) if s_dtype != O.F32 else s.astype(np.float64)
        K = w.shape[0]
        if group == K:
            return (a @ wq) * sv.reshape(-1)[None, :]
        wt = (wq.reshape(K // group, group, -1) * sv[:, None, :]).astype(np.float32).reshape(K, -1)
        return a @ O.round16(wt, a_dtype).astype(np.float64)
    return a @ O.to_f32(w, w_dtype).astype(np.float64)


@pytest.mark.parametrize("epi", list(O.EPI))
def test_gemm_golden_per_channel(epi):
    g = gold("gemm_ch.npz")
    M, K = g["A"].shape
    N = g["q"].shape[1]
    C = g["X0"].copy() if epi in ("resid", "resid_gate") else None
    out = O.gemm(O.EPI[epi], g["A"], O.F16, g["q"], O.I8, g["s"], O.F16, K, C=C, vec=g["vec"])
    got = out if out.dtype == np.float32 else O.to_f32(out, O.F16)
    ref = g["out_" + epi]
    if epi in ("resid", "resid_gate"):
        got, ref = got - g["X0"], ref - g["X0"]
    assert rel_l2(got, ref) < (1e-3 if epi not in ("f32", "bias_f32", "resid", "resid_gate") else 1e-5), epi


def test_gemm_golden_group128_bf16():
    g = gold("gemm_g128.npz")
    K = g["A"].shape[1]
    out = O.to_f32(O.gemm(0, g["A"], O.BF16, g["q"], O.I8, g["s"], O.F32, 128), O.BF16)
    assert rel_l2(out, g["out_store16"]) < 8e-3    # one bf16 rounding of each output (2^-9 relative)
    assert K == 256


@pytest.mark.parametrize("kind", ["g64h", "g256b", "chf32", "chbf"])
@pytest.mark.parametrize("a_dtype", [O.F16, O.BF16])
def test_gemm_fp64_brute_force_scale_formats(kind, a_dtype):
    """The other scale storage formats (fp16 / bf16 group scales at groups 64 and 256; per-channel f32 / bf16)
    against the float64 restatement: per-channel scales multiply the exact integer sum, group scales dequantize
    each weight once (q s in f32, rounded to the activation type; gemm.metal:190-196)."""
    from tests.helpers import make_weight
    rng = np.random.default_rng(19)
    M, K, N = 21, 512, 192
    A = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), a_dtype)
    wd = make_weight(rng, K, N, kind, a_dtype)
    got = O.gemm(O.EPI["f32"], A, a_dtype, wd["w"], wd["w_dtype"], wd["s"], wd["s_dtype"], wd["group"])
    ref = _acc64(A, a_dtype, wd["w"], wd["w_dtype"], wd["s"], wd["s_dtype"], wd["group"])
    assert rel_l2(got, ref) < 1e-6


@pytest.mark.parametrize("kind", ["ch", "g128", "16"])
@pytest.mark.parametrize("a_dtype", [O.F16, O.BF16])
def test_gemm_fp64_brute_force(kind, a_dtype):
    rng = np.random.default_rng(9)
    M, K, N = 33, 256, 128
    A = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), a_dtype)
    if kind == "ch":
        w = rng.integers(-127, 128, (K, N), dtype=np.int8)
        s, s_dtype, group, w_dtype = O.from_f32(np.abs(rng.standard_normal(N)).astype(np.float32) * 1e-3, O.F16), O.F16, K, O.I8
    elif kind == "g128":
        w, s = O.quant_q8((rng.standard_normal((K, N)) * 0.02).astype(np.float32), 128)
        s_dtype, group, w_dtype = O.F32, 128, O.I8
    else:
        w = O.from_f32((rng.standard_normal((K, N)) * 0.02).astype(np.float32), a_dtype)
        s, s_dtype, group, w_dtype = None, O.F32, 0, a_dtype
    got = O.gemm(O.EPI["f32"], A, a_dtype, w, w_dtype, s, s_dtype, group)
    ref = _acc64(A, a_dtype, w, w_dtype, s, s_dtype, group)
    assert rel_l2(got, ref) < 1e-6


def test_gemm_identity_and_permutation_weights():
    rng = np.random.default_rng(12)
    K = 128
    A = O.from_f32(rng.standard_normal((20, K)).astype(np.float32), O.F16)
    eye = np.eye(K, dtype=np.int8)
    ones = O.from_f32(np.ones(K, np.float32), O.F16)
    out = O.gemm(0, A, O.F16, eye, O.I8, ones, O.F16, K)
    assert np.array_equal(out, A)                               # exact: one product per output
    perm = rng.permutation(K)
    P = np.zeros((K, K), np.int8)
    P[perm, np.arange(K)] = 1                                   # out[:, n] = A[:, perm[n]]
    out = O.gemm(0, A, O.F16, P, O.I8, ones, O.F16, K)
    assert np.array_equal(out, A[:, perm])


def test_gemm_k_split_additivity():
    rng = np.random.default_rng(13)
    M, K, N = 16, 256, 64
    A = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), O.BF16)
    w = O.from_f32((rng.standard_normal((K, N)) * 0.1).astype(np.float32), O.BF16)
    full = O.gemm(1, A, O.BF16, w, O.BF16)
    lo = O.gemm(1, np.ascontiguousarray(A[:, :128]), O.BF16, np.ascontiguousarray(w[:128]), O.BF16)
    x = lo.copy()
    O.gemm(3, np.ascontiguousarray(A[:, 128:]), O.BF16, np.ascontiguousarray(w[128:]), O.BF16, C=x)  # resid: x += acc
    assert rel_l2(x, full) < 1e-6


def test_epilogue_functions_match_torch():
    """gelu_tanh / silu of the oracle against torch's own implementations, through 1x1 GEMMs with weight 1."""
    x = np.linspace(-12, 12, 4096, dtype=np.float32)
    K = 64
    A = np.zeros((x.size, K), np.float32)
    A[:, 0] = x
    A16 = O.from_f32(A, O.BF16)
    xa = O.to_f32(A16[:, 0], O.BF16)
    w = np.zeros((K, 64), np.int8)
    w[0, :] = 1
    s = np.ones((1, 64), np.float32)
    g = O.to_f32(O.gemm(O.EPI["gelu"], A16, O.BF16, w, O.I8, s, O.F32, K), O.BF16)[:, 0]
    ref = torch.nn.functional.gelu(torch.from_numpy(xa).double(), approximate="tanh").numpy()
    assert np.max(np.abs(g - ref) / np.maximum(np.abs(ref), 1e-3)) < 8e-3  # bf16 store
    sw = O.to_f32(O.gemm(O.EPI["swiglu"], A16, O.BF16, w, O.I8, s, O.F32, K), O.BF16)[:, 0]
    ref = (torch.nn.functional.silu(torch.from_numpy(xa).double()) * torch.from_numpy(xa).double()).numpy()
    assert np.max(np.abs(sw - ref) / np.maximum(np.abs(ref), 1e-3)) < 8e-3


def test_gemm_rejects_bad_shapes():
    A = np.zeros((4, 100), np.uint16)
    with pytest.raises(ValueError):
        O.gemm(0, A, O.F16, np.zeros((100, 64), np.int8), O.I8, np.ones(64, np.uint16), O.F16, group=64)


# ---------------------------------------------------------------------------------------------- GEMV, make_cond
def test_gemv_silu_int8_channel():
    rng = np.random.default_rng(14)
    K, N = 256, 96
    x = rng.standard_normal((2, K)).astype(np.float32)
    q = rng.integers(-127, 128, (K, N), dtype=np.int8)
    s = (np.abs(rng.standard_normal(N)) * 1e-3).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    y = O.gemv(x, q, O.I8, s, O.F32, K, act=1, bias=b)
    xs = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    ref = (xs @ q.astype(np.float64)) * s + b
    assert rel_l2(y, ref) < 1e-6
    y2 = O.gemv(x, q, O.I8, s, O.F32, K, y=y.copy(), act=3, bias=b)    # accumulate
    assert rel_l2(y2, 2 * ref) < 1e-6


def test_gemv_gelu_on_load_f32_weights():
    """act bit 2: GELU(tanh) of x on load (Conditioning::compute's gelu between its linears), torch's
    gelu(approximate="tanh") in float64 as the reference; f32 weights."""
    rng = np.random.default_rng(41)
    K, N = 192, 40
    x = (2 * rng.standard_normal((3, K))).astype(np.float32)
    w = rng.standard_normal((K, N)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    y = O.gemv(x, w, O.F32, act=4, bias=b)
    g = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    assert rel_l2(y, g @ w.astype(np.float64) + b) < 1e-6


def _bf16(v: float) -> float:
    return float(torch.tensor(v, dtype=torch.float32).to(torch.bfloat16).float())


def test_temb_closed_forms():
    """engine/src/model.mm:576-581. sigma = 0: every cos term is 1 and every sin term 0. Any sigma: the values
    are cos / sin of bf16(sigma) * 1000 * 10000^(-i/128) (argument formed in float32 as the reference writes
    it; numpy float64 trig), and within 2e-4 of the all-float64 formula (the float32 argument's rounding)."""
    e = O.temb(0.0)
    assert np.array_equal(e[:128], np.ones(128, np.float32)) and np.array_equal(e[128:], np.zeros(128, np.float32))
    i = np.arange(128, dtype=np.float32)
    for sig in (1.0, 0.8123, 0.3333, 0.0421):
        ts = np.float32(_bf16(sig))
        # float32 exponent, then a correctly rounded float32 exp (float64 exp, one rounding)
        ex = (-np.float32(np.log(10000.0)) * i) / np.float32(128.0)
        fr = np.exp(ex.astype(np.float64)).astype(np.float32)
        arg = (ts * np.float32(1000.0)) * fr
        got = O.temb(sig)
        assert np.abs(got[:128] - np.cos(arg.astype(np.float64))).max() <= 2e-6
        assert np.abs(got[128:] - np.sin(arg.astype(np.float64))).max() <= 2e-6
        a64 = _bf16(sig) * 1000.0 * np.exp(-np.log(1e4) * np.arange(128) / 128.0)
        assert np.abs(got - np.concatenate([np.cos(a64), np.sin(a64)])).max() <= 2e-4
    # the model sees bf16(sigma): sigmas in one bf16 interval give the same embedding
    assert np.array_equal(O.temb(0.8125), O.temb(0.81251))


def test_conditioning_composition_matches_float64():
    """Conditioning::compute (model.mm:582-590) as the oracle composes it, against numpy float64 with torch's
    tanh-GELU: h = W1 e + b1, t = W2 gelu(h) + b2, tvec = Wp gelu(t) + bp."""
    rng = np.random.default_rng(42)
    D = 64
    w1, w2, wp = (rng.standard_normal(s).astype(np.float32) / np.sqrt(s[0]) for s in ((256, D), (D, D), (D, 6 * D)))
    b1, b2, bp = (0.1 * rng.standard_normal(n).astype(np.float32) for n in (D, D, 6 * D))
    t, tvec = O.conditioning(0.6, w1, b1, w2, b2, wp, bp)
    gelu = lambda v: torch.nn.functional.gelu(torch.from_numpy(v), approximate="tanh").numpy()  # noqa: E731
    e = O.temb(0.6).astype(np.float64)
    h = e @ w1 + b1
    t64 = gelu(h) @ w2 + b2
    tv64 = gelu(t64) @ wp + bp
    assert rel_l2(t, t64) < 1e-5 and rel_l2(tvec, tv64) < 1e-5


def test_make_fin_restatement():
    """model.mm:340-346: fin = [nf (1 + t + lin0) ; t + lin1]; t = lin = 0 gives [nf ; 0]."""
    rng = np.random.default_rng(43)
    D = 96
    t, nf = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    lin = rng.standard_normal((2, D)).astype(np.float32)
    f = O.make_fin(t, lin, nf)
    assert np.array_equal(f[0], nf * ((np.float32(1) + t) + lin[0])) and np.array_equal(f[1], t + lin[1])
    z = O.make_fin(np.zeros(D, np.float32), np.zeros((2, D), np.float32), nf)
    assert np.array_equal(z[0], nf) and not z[1].any()


def test_make_cond_special_cases():
    rng = np.random.default_rng(15)
    D = 64
    n1, n2 = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    m = O.make_cond(np.zeros(6 * D, np.float32), None, n1, n2)
    assert np.array_equal(m[0], n1) and np.array_equal(m[3], n2)
    assert not m[1].any() and not m[2].any() and not m[4].any() and not m[5].any()
    tv = rng.standard_normal(6 * D).astype(np.float32)
    tab = rng.standard_normal(6 * D).astype(np.float32)
    a = O.make_cond(tv, tab, n1, n2)
    b = O.make_cond(tv + tab, None, n1, n2)                     # the table adds to tvec before modulation
    assert np.allclose(a, b, rtol=1e-6, atol=1e-6)
    m = O.make_cond(np.full(6 * D, -1.0, np.float32), None, n1, n2)  # scale -1 cancels the norm weight
    assert not m[0].any() and not m[3].any()


def test_make_cond_one_hot_rows():
    """model.mm:329-338, pinned row by row. DiT::layer (model.mm:374-382) consumes mods row 0 as the first norm's
    multiplier, row 1 as its additive shift, row 2 as the attention gate, rows 3/4/5 likewise for the MLP half.
    A unit impulse at tvec[j*D+k] must move exactly mods[j][k]: by n1[k] (j = 0), n2[k] (j = 3) or 1 (otherwise);
    any swap of rows (shift/gate, v4/v5) or of n1/n2 fails here."""
    rng = np.random.default_rng(151)
    D = 48
    n1 = (1.5 + rng.random(D)).astype(np.float32)       # distinct from 1 and from each other
    n2 = (-3.0 - rng.random(D)).astype(np.float32)
    base = O.make_cond(np.zeros(6 * D, np.float32), None, n1, n2)
    for j in range(6):
        for k in (0, 7, D - 1):
            tv = np.zeros(6 * D, np.float32)
            tv[j * D + k] = 1.0
            d = O.make_cond(tv, None, n1, n2) - base
            want = np.zeros((6, D), np.float32)
            want[j, k] = n1[k] if j == 0 else n2[k] if j == 3 else 1.0
            assert np.array_equal(d, want), (j, k)
            # the per-layer table enters exactly where tvec does
            dt = O.make_cond(np.zeros(6 * D, np.float32), tv, n1, n2) - base
            assert np.array_equal(dt, want), ("table", j, k)


def test_make_fin_one_hot_rows():
    """model.mm:340-346 pinned by impulses: t[k] moves fin[0][k] by nf[k] and fin[1][k] by 1; lin row 0 moves only
    fin[0][k] (by nf[k]); lin row 1 moves only fin[1][k] (by 1). A lin row swap or a dropped t term fails."""
    rng = np.random.default_rng(152)
    D = 40
    nf = (2.0 + rng.random(D)).astype(np.float32)
    z = np.zeros(D, np.float32)
    base = O.make_fin(z, np.zeros((2, D), np.float32), nf)
    assert np.array_equal(base[0], nf) and not base[1].any()
    for k in (0, 11, D - 1):
        t = z.copy()
        t[k] = 1.0
        d = O.make_fin(t, np.zeros((2, D), np.float32), nf) - base
        want = np.zeros((2, D), np.float32)
        want[0, k], want[1, k] = nf[k], 1.0
        assert np.array_equal(d, want), ("t", k)
        for r in (0, 1):
            lin = np.zeros((2, D), np.float32)
            lin[r, k] = 1.0
            d = O.make_fin(z, lin, nf) - base
            want = np.zeros((2, D), np.float32)
            want[r, k] = nf[k] if r == 0 else 1.0
            assert np.array_equal(d, want), ("lin", r, k)


# ---------------------------------------------------------------------------------------------- norms, RoPE
@pytest.mark.parametrize("center", [0, 1])
def test_rms_and_layer_norm_match_torch(center):
    rng = np.random.default_rng(16)
    x = (rng.standard_normal((17, 384)) * 3 + 0.5).astype(np.float32)
    mul = rng.standard_normal(384).astype(np.float32)
    add = rng.standard_normal(384).astype(np.float32)
    y = O.to_f32(O.rms_norm(x, mul, add, O.BF16, eps=1e-6, center=center), O.BF16)
    xt = torch.from_numpy(x).double()
    if center:
        ref = torch.nn.functional.layer_norm(xt, (384,), eps=1e-6)
    else:
        ref = torch.nn.functional.rms_norm(xt, (384,), eps=1e-6)
    ref = (ref * torch.from_numpy(mul).double() + torch.from_numpy(add).double()).numpy()
    assert rel_l2(y, ref) < 4e-3
    yf = O.rms_norm(x, mul, None, O.F32, eps=1e-6, center=center)
    assert rel_l2(yf, ref - add) < 1e-6


def test_rope_tables_special_positions():
    T, H, W = 3, 5, 7
    for mode in (0, 1):
        c, s = O.rope_tables(T, H, W, mode)
        assert np.all(c[:T] == 1) and np.all(s[:T] == 0)        # text rows sit at the origin
        r = T + 2 * W + 5                                        # image token (i, j) = (2, 5)
        pi, pj = (16, 40) if mode == 0 else (0, 32)              # first pair of the row / column axis (omega 1)
        assert np.isclose(c[r, pi], np.cos(2.0)) and np.isclose(s[r, pi], np.sin(2.0))
        assert np.isclose(c[r, pj], np.cos(5.0)) and np.isclose(s[r, pj], np.sin(5.0))
        if mode == 0:
            assert np.all(c[:, :16] == 1)                        # frame axis: always position 0
            assert np.isclose(c[r, 17], np.cos(2.0 * 1000.0 ** (-2.0 / 48)))
        else:
            assert np.isclose(c[r, 33], np.cos(5.0 * 10000.0 ** (-2.0 / 64)))


def test_qk_norm_rope_complex_form_and_norm():
    rng = np.random.default_rng(17)
    rows, nq, nk = 9, 2, 1
    ld = (nq + nk) * 128 + 64
    qkv = O.from_f32(rng.standard_normal((rows, ld)).astype(np.float32), O.F16)
    wq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    c, s = O.rope_tables(1, 2, 4, 1)
    out, _, _ = O.qk_norm_rope(qkv, O.F16, wq, wk, c, s, 0, nq, nq * 128, nk, eps=1e-6, rope_mode=0)
    x = O.to_f32(qkv, O.F16).astype(np.float64)
    got = O.to_f32(out, O.F16).astype(np.float64)
    for h in range(nq + nk):
        xh = x[:, h * 128:(h + 1) * 128]
        wh = wq if h < nq else wk
        n = xh / np.sqrt((xh ** 2).mean(axis=1, keepdims=True) + 1e-6) * wh
        z = (n[:, 0::2] + 1j * n[:, 1::2]) * (c + 1j * s)          # pair (2i, 2i+1) rotated by angle i
        ref = np.stack([z.real, z.imag], axis=-1).reshape(rows, 128)
        assert rel_l2(got[:, h * 128:(h + 1) * 128], ref) < 2e-3
        assert np.allclose(np.linalg.norm(got[:, h * 128:(h + 1) * 128], axis=1), np.linalg.norm(n, axis=1),
                           rtol=3e-3)
    assert np.array_equal(out[:, -64:], qkv[:, -64:])             # columns outside the heads untouched


def test_qk_rope_rotate_half_equals_pairs_under_permutation():
    rng = np.random.default_rng(18)
    rows = 6
    x = rng.standard_normal((rows, 128)).astype(np.float32)
    perm = np.empty(128, np.int64)                                  # pairs layout -> rotate-half layout
    perm[0::2], perm[1::2] = np.arange(64), np.arange(64) + 64
    c, s = O.rope_tables(0, 2, 3, 1)
    w = np.ones(128, np.float32)
    a, _, _ = O.qk_norm_rope(O.from_f32(x[:, perm], O.BF16), O.BF16, w, w, c, s, 0, 1, 0, 0, rope_mode=0)
    b, _, _ = O.qk_norm_rope(O.from_f32(x, O.BF16), O.BF16, w, w, c, s, 0, 1, 0, 0, rope_mode=1)
    assert np.array_equal(a, b[:, perm])


def test_qk_norm_big_dim_split():
    rng = np.random.default_rng(19)
    qkv = O.from_f32(rng.standard_normal((4, 256)).astype(np.float32), O.BF16)
    w = np.ones(128, np.float32)
    out, qb, kb = O.qk_norm_rope(qkv, O.BF16, w, w, None, None, 0, 1, 128, 1, rope_mode=2, big_dim=5)
    ref, _, _ = O.qk_norm_rope(qkv, O.BF16, w, w, None, None, 0, 1, 128, 1, rope_mode=2)
    assert not O.to_f32(out[:, 5], O.BF16).any() and not O.to_f32(out[:, 133], O.BF16).any()
    assert np.allclose(qb[:, 0], O.to_f32(ref[:, 5], O.BF16), rtol=4e-3)
    assert np.allclose(kb[:, 0], O.to_f32(ref[:, 133], O.BF16), rtol=4e-3)


# ---------------------------------------------------------------------------------------------- attention
def test_attention_golden_gqa_causal_gated():
    g = gold("attn.npz")
    H, G = int(g["heads"]), int(g["group"])
    o = O.to_f32(O.attention(g["Q"], g["K"], g["V"], O.F16, H, group=G), O.F16)
    assert rel_l2(o, g["out"]) < 3e-3                                # P and O rounded to fp16
    oc = O.to_f32(O.attention(g["Q"], g["K"], g["V"], O.F16, H, group=G, causal=1, q_pos0=int(g["q_pos0"])), O.F16)
    assert rel_l2(oc, g["out_causal"]) < 3e-3
    og = O.to_f32(O.attention(g["Q"], g["K"], g["V"], O.F16, H, group=G, G=g["G"]), O.F16)
    assert rel_l2(og, g["out_gated"]) < 3e-3


def test_attention_matches_torch_sdpa():
    rng = np.random.default_rng(20)
    L, H = 50, 2
    q, k, v = (O.from_f32(rng.standard_normal((L, H * 128)).astype(np.float32), O.BF16) for _ in range(3))
    o = O.to_f32(O.attention(q, k, v, O.BF16, H), O.BF16)
    t = [torch.from_numpy(O.to_f32(a, O.BF16)).double().view(L, H, 128).transpose(0, 1) for a in (q, k, v)]
    ref = torch.nn.functional.scaled_dot_product_attention(*t).transpose(0, 1).reshape(L, H * 128).numpy()
    assert rel_l2(o, ref) < 8e-3


def test_attention_invariants():
    rng = np.random.default_rng(21)
    L, H = 24, 1
    q = O.from_f32(rng.standard_normal((L, 128)).astype(np.float32), O.F16)
    k = O.from_f32(rng.standard_normal((L, 128)).astype(np.float32), O.F16)
    vrow = rng.standard_normal(128).astype(np.float32)
    v = O.from_f32(np.tile(vrow, (L, 1)), O.F16)                 # uniform V -> every output row is that row
    o = O.to_f32(O.attention(q, k, v, O.F16, H), O.F16)
    assert np.allclose(o, O.to_f32(v[:1], O.F16), rtol=2e-3, atol=2e-3)
    # one dominant key: q . k_7 >> others -> output = v_7
    kk = np.zeros((L, 128), np.float32)
    kk[7] = 8.0
    qq = np.full((L, 128), 8.0, np.float32)
    vv = rng.standard_normal((L, 128)).astype(np.float32)
    o = O.to_f32(O.attention(O.from_f32(qq, O.F16), O.from_f32(kk, O.F16), O.from_f32(vv, O.F16), O.F16, H), O.F16)
    assert np.allclose(o, O.to_f32(O.from_f32(vv[7:8], O.F16), O.F16), rtol=2e-3, atol=2e-3)
