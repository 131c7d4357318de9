"""Robustness of the .qw reader (csrc/kh_qw.cpp: mmap, header length, JSON parser, tensor table checks) against
malformed and adversarial files, under AddressSanitizer and UndefinedBehaviorSanitizer on the host (CPU only:
kh_qw_open parses and validates without touching a GPU). A seeded corpus of mutations of a valid file: header
bit flips, truncations, bad header lengths, out-of-range / wrong-type numbers, shapes and offsets, deep nesting,
bad string escapes, random bytes, overlapping or out-of-file tensors, and structural changes. Passing means no
sanitizer report and no crash; which files are accepted is covered by tests/test_qw.py."""
import json
import os
import random
import shutil
import struct
import subprocess

import numpy as np
import pytest

from krea_image_amd import qw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


def _corpus(d, n, seed):
    base = os.path.join(d, "base.qw")
    qw.write_qw(base, [("a", "f32", np.ones((3, 5), np.float32)), ("b.s", "bf16", np.ones((4,), np.float32)),
                       ("c", "i8", np.ones((2, 2, 2), np.int8)), ("d", "f16", np.ones((1,), np.float16))],
                meta={"k": [1, 2.5, "xé", None, True], "n": {"deep": {"x": -0.0}}})
    B = open(base, "rb").read()
    hlen = struct.unpack("<Q", B[8:16])[0]
    H = json.loads(B[16:16 + hlen])
    data = B[(16 + hlen + qw.ALIGN - 1) // qw.ALIGN * qw.ALIGN:]
    rng = random.Random(seed)
    weird = [-1, 0, 2 ** 31, 2 ** 32 + 1, 2 ** 63 - 1, 2 ** 64, -2 ** 63, 1e300, 1.5, "3", None, [], {},
             18446744073709551615]

    def with_header(hj):
        hjb = hj if isinstance(hj, bytes) else hj.encode("utf-8", "surrogatepass")
        start = (16 + len(hjb) + qw.ALIGN - 1) // qw.ALIGN * qw.ALIGN
        hdr = B[:8] + struct.pack("<Q", len(hjb)) + hjb
        return hdr + bytes(start - len(hdr)) + data

    paths = [base]
    for i in range(n):
        k = rng.randrange(9)
        if k == 0:  # bit flips in the header
            f = bytearray(B)
            for _ in range(rng.randint(1, 8)):
                j = rng.randrange(8, 16 + hlen)
                f[j] ^= 1 << rng.randrange(8)
            f = bytes(f)
        elif k == 1:  # truncation
            f = B[:rng.randrange(0, len(B))]
        elif k == 2:  # header length field
            f = bytearray(B)
            f[8:16] = struct.pack("<Q", rng.choice([0, 1, hlen - 1, hlen + 1, len(B), 2 ** 63, 2 ** 64 - 1,
                                                    rng.randrange(2 ** 64)]))
            f = bytes(f)
        elif k == 3:  # one field of one tensor set to an odd value
            h = json.loads(json.dumps(H))
            t = rng.choice(list(h["tensors"].values()))
            fld = rng.choice(["offset", "shape", "dtype", "nbytes"])
            if fld == "shape":
                t["shape"] = rng.choice([[rng.choice(weird)], [2 ** 40, 2 ** 40], list(range(9)), [], [1] * 20, "x"])
            else:
                t[fld] = rng.choice(weird + ["f32", "f64", "", "i8"])
            f = with_header(json.dumps(h))
        elif k == 4:  # deep nesting
            depth = rng.choice([10, 100, 1000, 100000])
            f = with_header(json.dumps(H)[:-1] + ', "z": ' + "[" * depth + "]" * depth + "}")
        elif k == 5:  # string escapes and control characters
            s = rng.choice(['"\\u', '"\\ud800"', '"\\udc00\\ud800"', '"\\x41"', '"\\u00"', '"\x01"', '"\\', '"abc',
                            '"\\ud83d\\ude00"'])
            f = with_header(json.dumps(H)[:-1] + ', "s": ' + s + "}")
        elif k == 6:  # random bytes as the header
            f = with_header(bytes(rng.randrange(256) for _ in range(rng.randrange(0, 300))))
        elif k == 7:  # a tensor moved onto another or past the end of the file
            h = json.loads(json.dumps(H))
            ts = list(h["tensors"].values())
            ts[0]["offset"] = rng.choice([ts[1]["offset"], 2 ** 62, len(B), qw.ALIGN * 3, 1])
            f = with_header(json.dumps(h))
        else:  # structure
            h = json.loads(json.dumps(H))
            c = rng.randrange(5)
            if c == 0:
                h["tensors"] = rng.choice([[], "x", 3, None])
            elif c == 1:
                del h["tensors"]
            elif c == 2:
                h["tensors"]["new"] = {"dtype": "f32", "shape": [2], "offset": 0}
            elif c == 3:
                h = rng.choice([[], 3, "x", None])
            else:
                h["tensors"][""] = h["tensors"].pop("a")
            f = with_header(json.dumps(h))
        p = os.path.join(d, f"f{i}.qw")
        with open(p, "wb") as fh:
            fh.write(f)
        paths.append(p)
    return paths


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_qw_reader_survives_adversarial_files_under_sanitizers(tmp_path):
    exe = str(tmp_path / "qwfuzz")
    subprocess.run([HIPCC, "-O1", "-g", "-std=c++17", "-Xarch_host", "-fsanitize=address", "-Xarch_host",
                    "-fsanitize=undefined", "-Xarch_host", "-fno-sanitize-recover=undefined", "-fno-gpu-sanitize",
                    "--offload-arch=gfx950", "-x", "hip", os.path.join(ROOT, "krea_image_amd", "csrc", "kh_qw.cpp"),
                    "-x", "c++", os.path.join(ROOT, "tests", "qw_fuzz_driver.cpp"), "-o", exe],
                   check=True, capture_output=True)
    paths = _corpus(str(tmp_path), 2500, seed=12)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], input="\n".join(paths) + "\n", capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    opened, rejected = (int(w) for w in r.stdout.split()[1::2])
    assert opened + rejected == len(paths) and opened >= 1 and rejected > len(paths) // 2
