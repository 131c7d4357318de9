"""Writes the golden fixtures of tests/golden/*.npz.

The reference (shinoss/krea_image) ships no tests, fixtures or golden vectors for this path, and its GPU
path is Metal-only, so these fixtures are computed here INDEPENDENTLY of oracle/oracle.c: plain numpy in
float64 from the closed forms the reference implements, on seeded inputs:

  q8_*.npz       tools/convert.py:92-99 quantizer on hand-picked groups (ties, zeros, clamps) and random data
  gemm_*.npz     engine/kernels/gemm.metal epilogues over the three weight formats, fp64 accumulation
  attn_*.npz     engine/kernels/attention.metal semantics: softmax(QK^T/sqrt(128)) V (* sigmoid(G)), fp64

Inputs are stored exactly as the kernels consume them (16-bit bit patterns, int8, f32); expected outputs are
float64 before the final 16-bit rounding, so tests can compare with a tolerance that names the roundings.

    python tests/golden/make_golden.py     # rewrites the fixtures (deterministic)
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16_val(bits):
    return bits.view(np.float16).astype(np.float64)


def gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def silu(x):
    return x / (1.0 + np.exp(-x))


def q8_fixture():
    # hand-picked group of 128 rows x 3 columns: amax 127 -> scale exactly 1, so x.5 inputs are exact ties
    # (round half to even); column 2 has its amax on a negative entry (scale 2)
    K, N, G = 128, 3, 128
    w = np.zeros((K, N), np.float32)
    w[0, 0], w[1, 0], w[2, 0], w[3, 0], w[4, 0] = 127.0, -63.5, 0.5, 1.5, -2.5
    w[:, 1] = 0.0                                   # all-zero column: scale clamps to 1e-12 / 127
    w[0, 2], w[1, 2] = -254.0, 100.0
    # numpy reference of convert.py:92-99 in float32 arithmetic (the converter runs in fp32)
    scale = np.maximum(np.abs(w).max(axis=0), np.float32(1e-12)) / np.float32(127.0)
    q = np.clip(np.rint(w / scale[None, :]), -127, 127).astype(np.int8)
    rng = np.random.default_rng(3)
    wr = (rng.standard_normal((256, 64)) * 0.02).astype(np.float32)
    g = wr.reshape(2, 128, 64)
    sr = (np.maximum(np.abs(g).max(axis=1), np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    qr = np.clip(np.rint(g / sr[:, None, :]), -127, 127).astype(np.int8).reshape(256, 64)
    np.savez(os.path.join(HERE, "q8.npz"), w=w, q=q, s=scale.astype(np.float32), group=G, w_rand=wr, q_rand=qr,
             s_rand=sr)


def gemm_fixture():
    rng = np.random.default_rng(11)
    M, K, N = 70, 256, 128
    A = f16_bits(rng.standard_normal((M, K)))
    q = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
    s = f16_bits(np.abs(rng.standard_normal(N)) * 0.02 / 127)
    vec = (rng.standard_normal(N) * 0.1).astype(np.float32)
    X0 = rng.standard_normal((M, N)).astype(np.float32)
    acc = f16_val(A) @ (q.astype(np.float64) * f16_val(s)[None, :])     # per-channel format
    up = acc.reshape(M, N // 64, 2, 32)
    out = {
        "store16": acc, "f32": acc, "gelu": gelu_tanh(acc), "bias16": acc + vec, "bias_f32": acc + vec,
        "resid": X0 + acc, "resid_gate": X0 + acc * vec,
        "swiglu": (silu(up[:, :, 0, :]) * up[:, :, 1, :]).reshape(M, N // 2),
    }
    np.savez(os.path.join(HERE, "gemm_ch.npz"), A=A, q=q, s=s, vec=vec, X0=X0, **{"out_" + k: v for k, v in out.items()})
    # group-128 format with bf16 activations: W~ = bf16(q * s) per element, fp64 accumulation
    import torch
    Ab = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16)
    wf = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    g = wf.reshape(K // 128, 128, N)
    sg = (np.maximum(np.abs(g).max(axis=1), np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    qg = np.clip(np.rint(g / sg[:, None, :]), -127, 127).astype(np.int8).reshape(K, N)
    wt = torch.from_numpy((qg.astype(np.float32).reshape(K // 128, 128, N) * sg[:, None, :]).reshape(K, N))
    wt = wt.to(torch.bfloat16).double().numpy()
    accg = Ab.double().numpy() @ wt
    np.savez(os.path.join(HERE, "gemm_g128.npz"), A=Ab.view(torch.int16).numpy().view(np.uint16), q=qg, s=sg,
             out_store16=accg)


def attn_fixture():
    rng = np.random.default_rng(5)
    L, Lk, H, G = 40, 56, 4, 2          # 4 query heads over 2 kv heads
    Q = f16_bits(rng.standard_normal((L, H * 128)))
    Kt = f16_bits(rng.standard_normal((Lk, (H // G) * 128)))
    V = f16_bits(rng.standard_normal((Lk, (H // G) * 128)))
    Gt = f16_bits(rng.standard_normal((L, H * 128)))
    q, k, v, gt = f16_val(Q), f16_val(Kt), f16_val(V), f16_val(Gt)
    out = np.zeros((L, H * 128))
    outc = np.zeros((L, H * 128))
    for h in range(H):
        kh = h // G
        s = q[:, h * 128:(h + 1) * 128] @ k[:, kh * 128:(kh + 1) * 128].T / np.sqrt(128.0)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h * 128:(h + 1) * 128] = p @ v[:, kh * 128:(kh + 1) * 128]
        # causal with q_pos0 = Lk - L: query i sees keys j <= i + q_pos0
        mask = np.arange(Lk)[None, :] <= (np.arange(L)[:, None] + (Lk - L))
        sc = np.where(mask, s, -np.inf)
        pc = np.exp(sc - sc.max(axis=1, keepdims=True))
        pc /= pc.sum(axis=1, keepdims=True)
        outc[:, h * 128:(h + 1) * 128] = pc @ v[:, kh * 128:(kh + 1) * 128]
    gated = out / (1.0 + np.exp(-gt))
    np.savez(os.path.join(HERE, "attn.npz"), Q=Q, K=Kt, V=V, G=Gt, heads=H, group=G, out=out, out_causal=outc,
             out_gated=gated, q_pos0=Lk - L)


if __name__ == "__main__":
    q8_fixture()
    gemm_fixture()
    attn_fixture()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
