"""The GGUF reader (libosmos_amd/csrc/gguf.cpp) under the address and undefined-behaviour sanitizers, on mutated
files: valid models (scalars of every width, string and integer arrays, four tensor types, two alignments, an empty
model) with bytes flipped, runs replaced by boundary values at count and length positions, truncations and
insertions. Every file must be refused or read to a model the driver can walk; a sanitizer report fails the test."""
import os
import random
import shutil
import struct
import subprocess

import pytest

import gguf_writer as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KV = [("general.architecture", W.STR, "qwen3moe"), ("a.u", W.U32, 7), ("a.arr", W.ARR, [1, 2, 3], W.I32),
      ("a.sarr", W.ARR, ["x", "yy", ""], W.STR), ("a.f", W.F64, 1.5), ("a.b", W.BOOL, 1), ("a.q", W.U64, 2 ** 63 + 5)]
TS = [("t0", 0, [8, 4], None, None), ("t1", 12, [256, 2], None, None), ("t2", 18, [512], None, None),
      ("t3", 30, [16], None, None)]


def mutate(rng, b):
    b = bytearray(b)
    for _ in range(rng.randint(1, 6)):
        r, p = rng.random(), rng.randrange(len(b))
        if r < 0.4:
            b[p] = rng.randrange(256)
        elif r < 0.6:
            b = b[:p]
        elif r < 0.75 and p + 8 <= len(b):
            b[p:p + 8] = struct.pack("<Q", rng.choice([0, 1, 2 ** 31, 2 ** 32 - 1, 2 ** 63, 2 ** 64 - 1,
                                                       rng.randrange(2 ** 64)]))
        elif r < 0.9 and p + 4 <= len(b):
            b[p:p + 4] = struct.pack("<I", rng.choice([0, 9, 13, 255, 2 ** 32 - 1, rng.randrange(40)]))
        else:
            b[p:p] = bytes(rng.randrange(256) for _ in range(rng.randint(1, 16)))
        if not b:
            break
    return bytes(b)


@pytest.mark.skipif(not shutil.which("g++"), reason="no host C++ compiler")
def test_reader_under_sanitizers(tmp_path):
    exe = tmp_path / "drv"
    r = subprocess.run(["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-I", os.path.join(ROOT, "include"), "-x", "c++", os.path.join(ROOT, "libosmos_amd", "csrc",
                        "gguf.cpp"), "-x", "c++", os.path.join(ROOT, "tests", "gguf_fuzz_driver.cpp"), "-o", str(exe)],
                       capture_output=True, text=True)
    if r.returncode and "asan" in r.stderr.lower() and "cannot find" in r.stderr.lower():
        pytest.skip("no sanitizer runtime for the host compiler")
    assert r.returncode == 0, r.stderr[-2000:]
    bases = [W.model(TS, KV)[0], W.model(TS[:2], KV[:3], align=64)[0], W.model([], [])[0]]
    rng = random.Random(1)
    files = []
    for i in range(3000):
        p = tmp_path / ("f%04d.gguf" % i)
        p.write_bytes(mutate(rng, rng.choice(bases)) if i >= len(bases) else bases[i])
        files.append(str(p))
    r = subprocess.run([str(exe)] + files, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    loaded = int(r.stdout.split()[1])
    assert len(bases) <= loaded < len(files)  # (the valid models load; most mutations are refused)
