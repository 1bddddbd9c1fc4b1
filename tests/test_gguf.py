"""The GGUF reader (include/osmos/model/gguf.h, libosmos_amd/csrc/gguf.cpp) on the CPU, against files written here
byte by byte (tests/gguf_writer.py) and against the reference's own test of its reader (tests/test_gguf.c, compiled in
place and linked with this library) where /root/reference is present. The cases follow the reference test's
(tests/test_gguf.c:138-434): a round trip of every value type and tensor placement, split models, every truncation,
corruptions, the MXFP8 / F8_E4M3 reading, NVFP4's blocks; plus gguf_int and gguf_bytes."""
import ctypes
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import gguf_writer as W
from libosmos_amd import capi
from libosmos_amd.gguf import GgufError, Model

REF = "/root/reference"
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def write(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def refused(path):
    L = capi.lib()
    err = ctypes.create_string_buffer(capi.GGUF_ERR)
    g = L.gguf_create(path.encode(), err)
    assert not g, "accepted"
    msg = err.value.decode()
    assert msg, "refused with no reason"
    return msg


THREE = [("a.f32", 0, [8, 2], None, None), ("b.q4k", 12, [256, 3], None, None), ("c.iq1_m", 29, [256, 1, 2], None, None)]
KV = [("t.u8", W.U8, 200), ("t.i32", W.I32, -7), ("t.f32", W.F32, 1.5), ("t.bool", W.BOOL, 1), ("t.str", W.STR, "deepseek"),
      ("t.strs", W.ARR, ["x", "", "yz"], W.STR), ("t.u32s", W.ARR, [10, 11, 12, 13], W.U32), ("t.u64", W.U64, 1 << 40),
      ("t.i8", W.I8, -3), ("t.i16", W.I16, -300), ("t.u16", W.U16, 60000), ("t.i64", W.I64, -(1 << 50)),
      ("t.f64", W.F64, 2.25), ("t.i64s", W.ARR, [-1, 2 ** 62], W.I64), ("t.u64s", W.ARR, [1, 2 ** 63 + 5], W.U64)]


@pytest.mark.parametrize("align", [None, 64])
def test_round_trip(tmp_path, align):
    blob, base = W.model(THREE, KV, align=align)
    p = write(tmp_path, "one.gguf", blob)
    with Model(p) as m:
        assert m.paths == [p] and m.sizes == [len(blob)]
        assert m.kv["t.u8"] == 200 and m.kv["t.i32"] == -7 and m.kv["t.f32"] == 1.5 and m.kv["t.bool"] is True
        assert m.kv["t.str"] == "deepseek" and m.kv["t.strs"] == ["x", "", "yz"]
        assert list(m.kv["t.u32s"]) == [10, 11, 12, 13] and m.kv["t.u64"] == 1 << 40
        assert m.kv["t.i16"] == -300 and m.kv["t.u16"] == 60000 and m.kv["t.i64"] == -(1 << 50) and m.kv["t.f64"] == 2.25
        a = align or 32
        assert base % a == 0
        at = 0
        for name, type_, dims, _, _ in THREE:
            t = m.tensors[name]
            nb = W.tensor_bytes(type_, dims)
            assert t["type"] == type_ and t["dims"] == dims and t["bytes"] == nb and t["file"] == 0
            assert t["offset"] == base + at and t["offset"] % a == 0
            want = bytes((i * 7 + len(name)) & 255 for i in range(nb))
            assert bytes(m.raw(name)) == want
            at = (at + nb + a - 1) // a * a
    L = capi.lib()
    g = L.gguf_create(p.encode(), None)
    assert g and not L.gguf_kv(g, b"absent") and not L.gguf_tensor(g, b"absent")
    t = L.gguf_tensor(g, b"c.iq1_m").contents
    assert t.type == 29 and t.n_dims == 3 and t.dims[0] == 256 and t.dims[2] == 2 and t.bytes == 112
    L.gguf_destroy(g)


def test_gguf_int_and_bytes(tmp_path):
    p = write(tmp_path, "kv.gguf", W.model(THREE[:1], KV)[0])
    L = capi.lib()
    g = L.gguf_create(p.encode(), None)
    v = ctypes.c_int64()

    def geti(key, i=0):
        k = L.gguf_kv(g, key.encode())
        return v.value if L.gguf_int(k, i, ctypes.byref(v)) else None
    assert geti("t.u8") == 200 and geti("t.i8") == -3 and geti("t.i16") == -300 and geti("t.u64") == 1 << 40
    assert geti("t.i64") == -(1 << 50) and geti("t.u32s", 3) == 13 and geti("t.i64s", 1) == 2 ** 62
    assert geti("t.u64s", 0) == 1 and geti("t.u64s", 1) is None  # (above INT64_MAX)
    assert geti("t.u32s", 4) is None  # (past the array)
    assert geti("t.f32") is None and geti("t.str") is None and geti("t.strs", 0) is None  # (not integers)
    L.gguf_destroy(g)
    assert L.gguf_bytes(18, 512) == 196 and L.gguf_bytes(0, 5) == 20 and L.gguf_bytes(30, 3) == 6
    assert L.gguf_bytes(18, 100) == 0  # (not whole blocks)
    assert L.gguf_bytes(1, 32) == 0 and L.gguf_bytes(99, 256) == 0  # (types no file here may hold: F16, unknown)
    assert L.gguf_bytes(40, 128) == 72 and L.gguf_bytes(43, 64) == 66 and L.gguf_bytes(0x12B, 7) == 7


def shard(no, count, tensors):
    return W.model(tensors, [("split.no", W.U16, no), ("split.count", W.U16, count)])[0]


def test_split(tmp_path):
    p1 = write(tmp_path, "m-00001-of-00002.gguf", shard(0, 2, THREE[:2]))
    p2 = write(tmp_path, "m-00002-of-00002.gguf", shard(1, 2, THREE[2:]))
    with Model(p1) as m:
        assert m.paths == [p1, p2] and len(m.tensors) == 3 and m.tensors["c.iq1_m"]["file"] == 1
        assert bytes(m.raw("c.iq1_m"))[:4] == bytes((i * 7 + 7) & 255 for i in range(4))
    with Model(p1, header_only=True) as h:  # the first shard alone: its own tensors, the whole metadata
        assert len(h.paths) == 1 and set(h.tensors) == {"a.f32", "b.q4k"} and h.kv["split.count"] == 2
    with pytest.raises(GgufError, match="-00001-of-"):
        Model(p2)  # (a later shard is not a model's start)
    os.remove(p2)
    assert "00002" in refused(p1)  # (the missing shard, by name)
    write(tmp_path, "m-00002-of-00002.gguf", shard(0, 2, THREE[2:]))
    assert "another split" in refused(p1)  # (split.no 0 in the second shard)
    assert "first shard" in refused(write(tmp_path, "odd.gguf", shard(0, 2, THREE[:2])))  # (no -00001-of- at all)
    for odd in ("n-00001-of-00003.gguf", "n-00001-of-2"):  # (named for another count: refused by name, nothing opened)
        assert "-00001-of-00002" in refused(write(tmp_path, odd, shard(0, 2, THREE[:2])))
    write(tmp_path, "d-00001-of-00002.gguf", shard(0, 2, THREE[:2]))
    write(tmp_path, "d-00002-of-00002.gguf", shard(1, 2, THREE[:1]))
    assert "twice" in refused(str(tmp_path / "d-00001-of-00002.gguf"))  # (a name in both shards)


def test_truncated(tmp_path):
    blob, base = W.model(THREE, KV[:4])
    for n in list(range(0, base + 1)) + [base + 1, len(blob) - 1]:
        p = write(tmp_path, "t.gguf", blob[:n])
        refused(p)
    with Model(write(tmp_path, "t.gguf", blob)) as m:
        assert len(m.tensors) == 3


def test_corrupt(tmp_path):
    good = THREE[:2]
    cases = {
        "magic": W.model(good, magic=b"GGUX")[0],
        "version 2": W.model(good, version=2)[0],
        "unknown type": W.model([("x", 1, [32], b"\0" * 64, None)])[0],  # F16: no file type here
        "unknown type id": W.model([("x", 77, [32], b"\0" * 64, None)])[0],
        "osmos id": W.model([("x", 0x12B, [32], b"\0" * 32, None)])[0],  # (0x100 | 43: no file's)
        "misaligned": W.model([("x", 0, [8], None, 4)])[0],
        "not whole blocks": W.model([("x", 18, [200], b"\0" * 98, None)])[0],
        "alignment 24": W.model(good, align=24)[0],
        "split.count a string": W.model(good, [("split.count", W.STR, "2")])[0],
        "overlap": W.model([("x", 0, [16], None, 0), ("y", 0, [16], None, 32)])[0],
        "name twice": W.model([("x", 0, [8], None, None), ("x", 0, [8], None, None)])[0],
    }
    for what, blob in cases.items():
        msg = refused(write(tmp_path, "c.gguf", blob))
        if what.startswith("unknown type") or what == "osmos id":
            assert "does not know" in msg, (what, msg)
        if what == "overlap":
            assert "overlap" in msg
    # dims: none, five, a zero
    for dims in ([], [8, 1, 1, 1, 1], [8, 0]):
        refused(write(tmp_path, "d.gguf", one_tensor_dims(dims)))
    # an unknown value type (13), an array of one, a string past the end, counts past the file
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W.s("k")
    for tail in (struct.pack("<I", 13) + b"\0" * 8, struct.pack("<IIQ", 9, 13, 1) + b"\0" * 8,
                 struct.pack("<I", 0x61737961) + b"\0" * 8, struct.pack("<IIQ", 9, 0x61737961, 1) + b"\0" * 8,
                 struct.pack("<IQ", 8, 1 << 40), struct.pack("<IIQ", 9, 4, 1 << 40)):
        refused(write(tmp_path, "v.gguf", head + tail + b"\0" * 32))
    refused(write(tmp_path, "n.gguf", b"GGUF" + struct.pack("<IQQ", 3, 1 << 50, 0) + b"\0" * 64))
    # a tensor whose bytes leave the file
    blob, base = W.model([("x", 0, [64], None, None)])
    assert "leave" in refused(write(tmp_path, "l.gguf", blob[:-4]))


def one_tensor_dims(dims):
    """a file of one F32 tensor "x" with these n_dims and dims, then 64 zero bytes"""
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + W.s("x")
    info = struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", 0, 0)
    return head + info + b"\0" * 64


def test_mxfp8_as_f8(tmp_path):
    vals = 64
    # MXFP8 blocks that fit their room: read as MXFP8
    blob, _ = W.model([("e", 43, [vals], None, None)])
    with Model(write(tmp_path, "m.gguf", blob)) as m:
        assert m.tensors["e"]["type"] == 43 and m.tensors["e"]["bytes"] == vals // 32 * 33
    # a 43 whose MXFP8 bytes would leave its room but whose values fit at a byte each: ggml's F8_E4M3 (0x12B)
    blob, base = W.model([("e", 43, [vals], b"\1" * vals, None)], data=b"\1" * vals)
    with Model(write(tmp_path, "f8.gguf", blob)) as m:
        assert m.tensors["e"]["type"] == 0x12B and m.tensors["e"]["bytes"] == vals
    blob, _ = W.model([("e", 43, [vals], b"\1" * (vals - 1), None)], data=b"\1" * (vals - 1))
    assert "leave" in refused(write(tmp_path, "f8short.gguf", blob))


def test_nvfp4(tmp_path):
    blob, _ = W.model([("w", 40, [128], None, None), ("s", 0, [4], None, None)])
    with Model(write(tmp_path, "n.gguf", blob)) as m:
        assert m.tensors["w"]["bytes"] == 72 and m.tensors["s"]["bytes"] == 16
    refused(write(tmp_path, "n2.gguf", W.model([("w", 40, [96], b"\0" * 72, None)])[0]))  # (not whole 64-blocks)


def test_mutations(tmp_path):
    """every byte of a valid file's header flipped in turn: refused, or read to a model whose tensors all lie in
    their file with their type's bytes - never a crash"""
    blob, base = W.model(THREE, KV[:3])
    L = capi.lib()
    for i in range(base):
        b = bytearray(blob)
        b[i] ^= 0x5A
        p = write(tmp_path, "mut.gguf", bytes(b))
        g = L.gguf_create(p.encode(), None)
        if g:
            m = g.contents
            for j in range(m.n_tensors):
                t = m.tensors[j]
                n = 1
                for d in range(t.n_dims):
                    n *= t.dims[d]
                assert t.offset + t.bytes <= len(blob) and L.gguf_bytes(t.type, n) == t.bytes
            L.gguf_destroy(g)


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "tests", "test_gguf.c")) or not shutil.which("gcc"),
                    reason="the reference's sources are not on this machine")
def test_reference_test_against_this_reader(tmp_path):
    """the reference's own test of its reader (tests/test_gguf.c), compiled in place with this library's gguf.h and
    linked with libosmos_mi355x.so in place of the reference's gguf.c: it must pass unchanged"""
    exe = str(tmp_path / "test_gguf")
    cmd = ["gcc", "-O1", "-std=gnu11", "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(REF, "include"),
           os.path.join(REF, "tests", "test_gguf.c"), capi.LIB_PATH, "-Wl,-rpath," + os.path.dirname(capi.LIB_PATH),
           "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "[test_gguf] ok" in r.stdout, r.stdout + r.stderr
