"""TEST INFRASTRUCTURE ONLY: ctypes bindings for the CPU oracle (oracle/_build/liborc.so) and, where it was built,
the reference's own compiled CPU path (oracle/_ref/libref.so, oracle/ref.mk). Imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg - as the checker or the CPU baseline, never by the product.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_SO = os.path.join(HERE, "_build", "liborc.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

_c = ctypes
P = _c.c_void_p
U32 = _c.c_uint32
U64 = _c.c_uint64
I32 = _c.c_int
F32 = _c.c_float
B = _c.c_bool

_orc = None
_ref = None


def build():
    """Compile the oracle (and, where /root/reference is present, the reference's CPU path)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORC_SO):
            build()
        lib = _c.CDLL(ORC_SO)
        _sig(lib, "orc_init", None)
        _sig(lib, "orc_f16", F32, U32)
        _sig(lib, "orc_lane_exp", F32, F32)
        _sig(lib, "orc_lane_swiglu", F32, F32, F32, F32, F32)
        _sig(lib, "orc_q8_round", B, P, U32, U32, U32, P, P)
        _sig(lib, "orc_q8_rows", B, U32, P, U32, U32, U32, P, P, U32, P, U32)
        _sig(lib, "orc_q8_rows_mt", B, U32, P, U32, U32, P, P, U32, P, U32, I32)
        _sig(lib, "orc_lane_sub", F32, U32, P, U32, P)
        _sig(lib, "orc_dequant", B, U32, P, U64, P)
        _sig(lib, "orc_mv_rows", B, U32, P, U32, U32, U32, P, U32, U32, P, U32)
        _sig(lib, "orc_mmq_x8_rows", B, P, U32, P, U32, U32, P, P, P)
        _sig(lib, "orc_mmq_rows", B, P, U32, U32, U32, P, P, P, U32, P)
        _sig(lib, "orc_mmq_x8_at", U64, U32, U32, U32)
        _sig(lib, "orc_mmq_dx_at", U64, U32, U32, U32)
        _sig(lib, "orc_f16_round", F32, F32)
        _sig(lib, "orc_mm_shape", None, U32, U32, B, _c.POINTER(U32), _c.POINTER(U32))
        _sig(lib, "orc_mm_rows", B, U32, P, U32, U32, U32, P, U32, U32, B, P, U32)
        _sig(lib, "orc_lane_layer", B, U32, U32, U32, U32, F32, P, P, U32, P, P, P, P, P, U32, P)
        _sig(lib, "orc_gather_sum_add", None, P, P, P, U32, U32, U32, P)
        _sig(lib, "orc_route", None, P, U32, U32, U32, P, P)
        _sig(lib, "orc_moe_sum", None, P, P, P, U32, U32, U32, P, P, P)
        _sig(lib, "orc_table", P, I32, _c.POINTER(U32))
        lib.orc_init()
        _orc = lib
    return _orc


def ref():
    """The reference's compiled CPU path, or None where it was not built (e.g. a GPU box without the build)."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_SO):
            return None
        lib = _c.CDLL(REF_SO)
        _sig(lib, "ref_q8_ready", B)
        _sig(lib, "ref_lane_exp", F32, F32)
        _sig(lib, "ref_lane_swiglu", F32, F32, F32, F32, F32)
        _sig(lib, "ref_q8_round", B, P, U32, U32, U32, P, P)
        _sig(lib, "ref_q8_rows", B, U32, P, U32, U32, U32, P, P, U32, P, U32)
        _sig(lib, "ref_q8_rows_mt", B, U32, P, U32, U32, P, P, U32, P, U32, I32)
        _sig(lib, "ref_mv_rows", B, U32, P, U32, U32, U32, P, U32, U32, P, U32)
        _sig(lib, "ref_lane_layer_mt", B, U32, U32, U32, P, P, P, P, P, U32, U32, P, P, P, P, I32, I32)
        _sig(lib, "ref_lane_layer_rot", B, U32, U32, U32, P, P, P, P, P, U32, U32, P, P, P, P, I32, I32, U32)
        _ref = lib
    return _ref


def ptr(a):
    return a.ctypes.data_as(P) if a is not None else None


# ---- numpy-level helpers over the oracle ----

def q8_round(x, lib=None):
    """x [rows, cols] fp32 -> (q int8 [rows, cols], d fp32 [rows, cols/32]); lib: None (the oracle) or ref()"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.zeros((rows, cols), np.int8)
    d = np.zeros((rows, cols // 32), np.float32)
    f = orc().orc_q8_round if lib is None else lib.ref_q8_round
    assert f(ptr(x), rows, cols, cols, ptr(q), ptr(d))
    return q, d


def q8_rows(type_, w, rows, cols, q, d, lib=None):
    """w: bytes of a [rows, cols] matrix; q [n, cols] int8, d [n, cols/32] -> y [n, rows]"""
    q = np.ascontiguousarray(q, dtype=np.int8)
    d = np.ascontiguousarray(d, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = q.shape[0]
    y = np.zeros((n, rows), np.float32)
    if lib is None:
        ok = orc().orc_q8_rows(type_, ptr(w), cols, 0, rows, ptr(q), ptr(d), n, ptr(y), rows)
    else:
        ok = lib.ref_q8_rows(type_, ptr(w), cols, 0, rows, ptr(q), ptr(d), n, ptr(y), rows)
    assert ok
    return y


def mv_rows(type_, w, rows, cols, x, lib=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = x.shape[0]
    y = np.zeros((n, rows), np.float32)
    f = orc().orc_mv_rows if lib is None else lib.ref_mv_rows
    assert f(type_, ptr(w), cols, 0, rows, ptr(x), cols, n, ptr(y), rows)
    return y


def dequant(type_, w, values):
    out = np.zeros(values, np.float32)
    assert orc().orc_dequant(type_, ptr(np.ascontiguousarray(w, dtype=np.uint8)), values, ptr(out))
    return out


def mmq_x8_rows(x, idx, cols):
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    slots = len(idx)
    padded = (slots + 15) // 16 * 16
    x8 = np.zeros(padded * cols, np.int8)
    dx = np.zeros(padded * (cols // 32), np.float32)
    sx = np.zeros(padded * (cols // 32), np.float32)
    assert orc().orc_mmq_x8_rows(ptr(x), x.shape[1], ptr(idx), slots, cols, ptr(x8), ptr(dx), ptr(sx))
    return x8, dx, sx


def mmq_rows(w, rows, cols, x8, dx, sx, slot):
    y = np.zeros(rows, np.float32)
    assert orc().orc_mmq_rows(ptr(np.ascontiguousarray(w, dtype=np.uint8)), cols, 0, rows, ptr(x8), ptr(dx), ptr(sx),
                              slot, ptr(y))
    return y


def mm_rows(type_, w, rows, cols, x, group=False):
    """the f16 matmul's order (mm_run, or mm_group's shape): w bytes of [rows, cols], x [n, cols] -> y [n, rows]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[0]
    y = np.zeros((n, rows), np.float32)
    assert orc().orc_mm_rows(type_, ptr(np.ascontiguousarray(w, dtype=np.uint8)), cols, 0, rows, ptr(x), cols, n,
                             group, ptr(y), rows)
    return y


def mm_shape(type_, cols, group=False):
    sl, w = U32(), U32()
    orc().orc_mm_shape(type_, cols, group, _c.byref(sl), _c.byref(w))
    return sl.value, w.value
