"""The packed weight file (.qw, tools/convert.py:13-17,49-130; reader engine/src/weights.mm:16-98): libkh's
C++ reader against files assembled byte by byte here (independent of the package's writer), the writer
round trip, rejection of malformed files, and the converter transforms (int8 group quantizer against the
oracle and its closed form, gate/up interleave against the epilogue's column rule). CPU only."""
import json
import os
import struct

import numpy as np
import pytest

from krea_image_amd import kh
from krea_image_amd import qw
from oracle import oracle as O


def raw_file(path, tensors, meta=None, version=1, pad_header=True):
    """Assemble a .qw file by hand: tensors = [(name, dtype, shape, bytes)] at consecutive 16 KiB offsets."""
    hdr, blobs, off = {}, [], 0
    for name, dt, shape, data in tensors:
        hdr[name] = {"dtype": dt, "shape": list(shape), "offset": off, "nbytes": len(data)}
        blobs.append((off, data))
        off += (len(data) + 16383) // 16384 * 16384
    hj = json.dumps({"tensors": hdr, "meta": meta or {}}).encode()
    start = (16 + len(hj) + 16383) // 16384 * 16384 if pad_header else 16 + len(hj)
    buf = bytearray(start + off)
    buf[:16 + len(hj)] = b"QWTS" + struct.pack("<IQ", version, len(hj)) + hj
    for o, d in blobs:
        buf[start + o:start + o + len(d)] = d
    with open(path, "wb") as f:
        f.write(bytes(buf))


def test_reader_on_hand_built_file(tmp_path):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.array([-127, 0, 5, 127], dtype=np.int8)
    c = np.array([0x3F80, 0xC000, 0x7FC0], dtype=np.uint16)  # bf16 1, -2, nan
    p = str(tmp_path / "hand.qw")
    raw_file(p, [("L0.w", "f32", (3, 4), a.tobytes()), ("L0.q", "i8", (4,), b.tobytes()),
                 ("x", "bf16", (3,), c.tobytes())], meta={"model": "t", "layers": 1, "u": "é中"})
    with qw.QwFile(p) as f:
        assert len(f) == 3 and f.version == 1
        assert f.names() == ["L0.q", "L0.w", "x"]
        assert f.meta == {"model": "t", "layers": 1, "u": "é中"}
        ti = f.info("L0.w")
        assert (ti.dtype, ti.shape, ti.offset, ti.nbytes) == ("f32", (3, 4), 0, 48)
        assert f.info("L0.q").offset == 16384 and f.info("x").offset == 32768
        np.testing.assert_array_equal(f.array("L0.w"), a)
        np.testing.assert_array_equal(f.array("L0.q"), b)
        np.testing.assert_array_equal(f.array("x"), c)
        assert not f.has("nope")
        with pytest.raises(kh.KhError, match="missing tensor"):
            f.info("nope")


def test_writer_round_trip_and_layout(tmp_path):
    rng = np.random.default_rng(0)
    t = [("A", "f32", rng.standard_normal((5, 7)).astype(np.float32)),
         ("A.s", "f16", rng.standard_normal(33).astype(np.float16)),
         ("B", "i8", rng.integers(-127, 128, (128, 64), dtype=np.int8)),
         ("C", "bf16", rng.standard_normal((2, 3)).astype(np.float32))]
    p = str(tmp_path / "w.qw")
    qw.write_qw(p, t, {"k": [1, 2.5, None, True]})
    raw = open(p, "rb").read()
    assert raw[:4] == b"QWTS" and struct.unpack("<I", raw[4:8])[0] == 1
    hlen = struct.unpack("<Q", raw[8:16])[0]
    hdr = json.loads(raw[16:16 + hlen])
    start = (16 + hlen + 16383) // 16384 * 16384
    assert all(v["offset"] % 16384 == 0 for v in hdr["tensors"].values())
    assert len(raw) % 16384 == 0 and len(raw) >= start
    with qw.QwFile(p) as f:
        assert f.meta == {"k": [1, 2.5, None, True]}
        for name, dt, a in t[:3]:
            np.testing.assert_array_equal(f.array(name), a)
        np.testing.assert_array_equal(f.array("C"), qw.bf16_bits(t[3][2]))
        np.testing.assert_array_equal(f.array("C"), O.from_f32(t[3][2], O.BF16))


@pytest.mark.parametrize("case,msg", [
    ("magic", "bad magic"),
    ("hlen", "header length"),
    ("json", "header JSON"),
    ("dtype", "unknown dtype"),
    ("nbytes", "nbytes"),
    ("past_end", "past the end"),
    ("shape", "bad shape"),
    ("no_tensors", "tensors"),
])
def test_reader_rejects_malformed(tmp_path, case, msg):
    p = str(tmp_path / f"{case}.qw")
    good = [("w", "f32", (4,), b"\0" * 16)]
    if case == "magic":
        raw_file(p, good)
        d = bytearray(open(p, "rb").read())
        d[:4] = b"QWTX"
        open(p, "wb").write(bytes(d))
    elif case == "hlen":
        raw_file(p, good)
        d = bytearray(open(p, "rb").read())
        d[8:16] = struct.pack("<Q", 1 << 40)
        open(p, "wb").write(bytes(d))
    elif case == "json":
        raw_file(p, good)
        d = bytearray(open(p, "rb").read())
        d[16] = ord("[")
        d[17] = ord("{")
        open(p, "wb").write(bytes(d))
    elif case == "dtype":
        raw_file(p, [("w", "f64", (2,), b"\0" * 16)])
    elif case == "nbytes":
        raw_file(p, [("w", "f32", (5,), b"\0" * 16)])
    elif case == "past_end":
        hj = json.dumps({"tensors": {"w": {"dtype": "i8", "shape": [100000], "offset": 0, "nbytes": 100000}}}).encode()
        open(p, "wb").write(b"QWTS" + struct.pack("<IQ", 1, len(hj)) + hj + b"\0" * 100)
    elif case == "shape":
        raw_file(p, [("w", "f32", (-4,), b"")])
    elif case == "no_tensors":
        hj = b'{"meta": {}}'
        open(p, "wb").write(b"QWTS" + struct.pack("<IQ", 1, len(hj)) + hj)
    with pytest.raises(kh.KhError, match=msg):
        qw.QwFile(p)


def test_reader_missing_file(tmp_path):
    with pytest.raises(kh.KhError, match="cannot open"):
        qw.QwFile(str(tmp_path / "absent.qw"))


def test_quantize_q8_matches_oracle_and_closed_form():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((256, 96)).astype(np.float32)
    w[:128, 5] = 0.0                      # all-zero group: scale clamps to 1e-12 / 127, q = 0
    w[7, 9] = 1e3                         # outlier sets its group's scale
    q, s = qw.quantize_q8(w)
    qo, so = O.quant_q8(w, 128)
    np.testing.assert_array_equal(q, qo)
    np.testing.assert_array_equal(s, so)
    assert s.shape == (2, 96) and s.dtype == np.float32
    assert np.all(np.abs(q) <= 127) and q[7, 9] == 127
    assert np.all(q[:128, 5] == 0) and s[0, 5] == np.float32(1e-12) / np.float32(127)
    # every group's max |q| is 127 (the amax element maps exactly to the end of the range)
    g = np.abs(q.astype(np.int32)).reshape(2, 128, 96).max(axis=1)
    assert np.all((g == 127) | (s == np.float32(1e-12) / np.float32(127)))
    # dequantization error at most half a step per element
    err = np.abs(q.astype(np.float32).reshape(2, 128, 96) * s[:, None, :] - w.reshape(2, 128, 96))
    assert np.all(err <= 0.5 * s[:, None, :] * (1 + 1e-6))


def test_quantize_q8_rounds_half_to_even():
    # scale = 127 / 127 = 1 exactly: q = round_half_even(w)
    w = np.zeros((128, 1), np.float32)
    w[:6, 0] = [127.0, 0.5, 1.5, 2.5, -0.5, -2.5]
    q, s = qw.quantize_q8(w)
    assert s[0, 0] == 1.0
    assert list(q[:6, 0]) == [127, 0, 2, 2, 0, -2]


def test_interleave_gate_up_column_rule():
    F, D = 96, 8
    gate = np.arange(F * D, dtype=np.float32).reshape(F, D)
    up = -gate - 1
    gu = qw.interleave_gate_up(gate, up)
    assert gu.shape == (2 * F, D)
    for t in range(F // 32):
        for i in range(32):
            np.testing.assert_array_equal(gu[64 * t + i], gate[32 * t + i])
            np.testing.assert_array_equal(gu[64 * t + 32 + i], up[32 * t + i])
    np.testing.assert_array_equal(gu, O.interleave_gate_up(gate, up))
    g2, u2 = qw.deinterleave_gate_up(gu)
    np.testing.assert_array_equal(g2, gate)
    np.testing.assert_array_equal(u2, up)


def test_random_dit_file_layout(tmp_path):
    p = str(tmp_path / "dit.qw")
    qw.write_random_dit(p, D=256, kv_heads=1, FF=256, layers=2, quant=True, seed=1, big_gain=(1, 5, 20.0))
    from krea_image_amd import dit
    with qw.QwFile(p) as f:
        names = f.names()
        assert len(names) == 2 * 13 + 6
        assert f.info("L0.qkvg").shape == (256, 2 * 256 + 2 * 128) and f.info("L0.qkvg").dtype == "i8"
        assert f.info("L0.qkvg.s").shape == (2, 768) and f.info("L0.qkvg.s").dtype == "f32"
        assert f.info("L1.gu").shape == (256, 512) and f.info("L1.down").shape == (256, 256)
        assert f.info("L0.mod").shape == (6, 256) and f.info("last.mod").shape == (2, 256)
        sh = dit.shape_from_qw(f)
        assert (sh.dim, sh.heads, sh.kv_heads, sh.ff, sh.layers, sh.mlp, sh.attn_gate) == (256, 2, 1, 256, 2, 1, 1)
        assert dit.big_dims(f, 2, gain=256.0) == [-1, 5]
        assert f.meta["layers"] == 2
