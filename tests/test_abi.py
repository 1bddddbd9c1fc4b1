"""The drop-in boundary, on the CPU: libosmos_mi355x.so loads and exports every function include/**/*.h declares,
exports nothing else, and refuses shapes before touching the GPU (refused calls queue nothing, so they run here).
(reference: include/osmos/gpu/*.h's refusal rules, e.g. kernels/q8.hip:83,94-95,114-116)"""
import os
import re
import subprocess

import pytest

from libosmos_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for d, _, files in os.walk(os.path.join(ROOT, "include")):
        for f in files:
            if f.endswith(".h"):
                text = open(os.path.join(d, f)).read()
                text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
                text = re.sub(r"//[^\n]*", "", text)
                text = re.sub(r"static inline[^{]*\{[^}]*\}", "", text, flags=re.S)
                for m in re.finditer(r"^\s*(?:const\s+)?(?:bool|void|uint32_t|uint64_t|int|Gguf|GgufTensor|GgufKv|CpuLane)\s*\**\s*"
                                     r"([a-z_0-9]+)\s*\(", text, re.M):
                    names.add(m.group(1))
    return names


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


@pytest.fixture(scope="module")
def built():
    if not os.path.exists(capi.LIB_PATH):
        pytest.fail("libosmos_mi355x.so not built (python -m libosmos_amd.build)")
    return capi.lib()


def test_exports_match_headers(built):
    d, e = declared(), exported()
    assert d, "no declarations found"
    assert d <= e, "declared but not exported: %s" % sorted(d - e)
    assert e <= d, "exported but not declared: %s" % sorted(e - d)


def test_refusals_without_gpu(built):
    L = built
    assert not L.q8_round(None, 1, 32, 32, None, None, None)
    assert not L.q8_group_tok(16, None, None, None, None, 1, 1, 16, 512, None, None, None, 16, None)
    assert not L.mv_run(99, None, 16, 512, None, 1, None, None)
    assert not L.quant_known(99)
    assert L.quant_known(18)


def test_layer_refuses_before_queueing(built):
    """osmos_lane_layer / _gate_up / _down check every shape first - a down matrix of rows that are not whole blocks
    (ff 384 in IQ3_XXS's 256-value blocks), a gate/up type that is not a lane type - so a refused call queues nothing
    (no launch happens: these run without a GPU)"""
    L = built
    p = 1 << 20  # (16-aligned stand-in addresses: never read, the calls refuse first)
    P = capi.ctypes.c_void_p

    def layer(tg, td, dim, ff):
        return capi.OsmosLaneLayer(tg, td, dim, ff, 8, 2, float("inf"), p, p, p, 1 << 16, 1 << 16, 1 << 16)
    for d in (layer(18, 18, 3072, 384), layer(18, 16, 2048, 384), layer(1, 18, 2048, 512), layer(18, 99, 2048, 512)):
        ws = L.osmos_lane_workspace(capi.ctypes.byref(d), 1)
        assert not L.osmos_lane_layer(capi.ctypes.byref(d), P(p), 1, P(p), P(p), P(p), P(p), P(p), max(ws, 1 << 20), None)
        assert not L.osmos_lane_gate_up(capi.ctypes.byref(d), P(p), 1, P(p), P(p), P(p), None)
        assert not L.osmos_lane_down(capi.ctypes.byref(d), P(p), 1, P(p), P(p), P(p), None)
