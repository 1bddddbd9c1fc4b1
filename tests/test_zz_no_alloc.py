"""osmos_lane_layer_noalloc (the layer with its workspace in the library's static device array) through the C ABI:
the bits of osmos_lane_layer (caller workspace) on two calls in a row - the second with fewer tokens, so it runs on
the array the first left behind - and a layer whose workspace exceeds OSMOS_LANE_SCRATCH_BYTES refused."""
import ctypes
import math

import numpy as np
import pytest

from libosmos_amd import capi, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def _case(n_exp, k, dim, ff, seed):
    t3 = synth.ID["IQ3_XXS"]
    gate = synth.iq_blocks(t3, n_exp * ff, dim, seed).reshape(n_exp, -1)
    up = synth.iq_blocks(t3, n_exp * ff, dim, seed + 1).reshape(n_exp, -1)
    down = synth.iq_blocks(t3, n_exp * dim, ff, seed + 2).reshape(n_exp, -1)
    return t3, gate, up, down


def test_noalloc_matches_workspace_layer(g):
    import torch
    n_exp, k, dim, ff = 64, 8, 2048, 512
    t3, gate, up, down = _case(n_exp, k, dim, ff, 81)
    G, U, D = g.dev(gate), g.dev(up), g.dev(down)
    desc = capi.OsmosLaneLayer(t3, t3, dim, ff, n_exp, k, math.inf, G.data_ptr(), U.data_ptr(), D.data_ptr(),
                               G[0].numel(), U[0].numel(), D[0].numel())
    L = capi.lib()
    rng = np.random.default_rng(82)
    for n_tok in (32, 3):  # the second call smaller: it reads nothing stale from the first's scratch
        x = g.dev(rng.normal(0, 1, (n_tok, dim)).astype(np.float32))
        ids = g.dev(np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32))
        w = g.dev(rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32))
        add = g.dev(rng.normal(0, 1, (n_tok, dim)).astype(np.float32))
        need = L.osmos_lane_workspace(ctypes.byref(desc), n_tok)
        ws = torch.zeros(need + 256, dtype=torch.uint8, device="cuda")
        wsp = ws.data_ptr() + (-ws.data_ptr()) % 256
        want = torch.full((n_tok, dim), float("nan"), device="cuda")
        got = torch.full((n_tok, dim), float("nan"), device="cuda")
        print("noalloc layer", n_tok, flush=True)
        assert L.osmos_lane_layer(ctypes.byref(desc), g.a(x), n_tok, g.a(ids), g.a(w), g.a(add), g.a(want),
                                  ctypes.c_void_p(wsp), need, None)
        assert L.osmos_lane_layer_noalloc(ctypes.byref(desc), g.a(x), n_tok, g.a(ids), g.a(w), g.a(add), g.a(got),
                                          None)
        wh, gh = g.host(want), g.host(got)
        assert np.isfinite(wh).all()
        assert (g.bits(gh) == g.bits(wh)).all(), n_tok


def test_noalloc_refuses_past_its_scratch(g):
    n_exp, k, dim, ff = 4, 32, 2048, 8192  # 64 tokens: h alone is 64 MB, past the 16 MB array
    t3 = synth.ID["IQ3_XXS"]
    L = capi.lib()
    p = g.dev(np.zeros(1 << 16, np.uint8))
    desc = capi.OsmosLaneLayer(t3, t3, dim, ff, n_exp, k, math.inf, p.data_ptr(), p.data_ptr(), p.data_ptr(), 256,
                               256, 256)
    assert L.osmos_lane_workspace(ctypes.byref(desc), 64) > (16 << 20)
    q = ctypes.c_void_p(p.data_ptr())
    assert not L.osmos_lane_layer_noalloc(ctypes.byref(desc), q, 64, q, q, q, q, None)


def test_noalloc_captured_replays(g):
    """called once eagerly (the array's address looked up), then captured in a graph and replayed three times, each
    replay against osmos_lane_layer's bits on new inputs copied into the captured buffers, with eager layer calls on
    the same array between replays"""
    import torch
    n_exp, k, dim, ff, n_tok = 64, 8, 2048, 512, 4
    t3, gate, up, down = _case(n_exp, k, dim, ff, 91)
    G, U, D = g.dev(gate), g.dev(up), g.dev(down)
    desc = capi.OsmosLaneLayer(t3, t3, dim, ff, n_exp, k, math.inf, G.data_ptr(), U.data_ptr(), D.data_ptr(),
                               G[0].numel(), U[0].numel(), D[0].numel())
    L = capi.lib()
    rng = np.random.default_rng(92)
    x = torch.zeros(n_tok, dim, device="cuda")
    ids = torch.zeros(n_tok, k, dtype=torch.int32, device="cuda")
    w = torch.zeros(n_tok, k, device="cuda")
    add = torch.zeros(n_tok, dim, device="cuda")
    got = torch.zeros(n_tok, dim, device="cuda")
    need = L.osmos_lane_workspace(ctypes.byref(desc), n_tok)
    ws = torch.zeros(need + 256, dtype=torch.uint8, device="cuda")
    wsp = ctypes.c_void_p(ws.data_ptr() + (-ws.data_ptr()) % 256)

    def fill():
        x.copy_(torch.from_numpy(rng.normal(0, 1, (n_tok, dim)).astype(np.float32)))
        ids.copy_(torch.from_numpy(np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)))
        w.copy_(torch.from_numpy(rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32)))
        add.copy_(torch.from_numpy(rng.normal(0, 1, (n_tok, dim)).astype(np.float32)))

    def want():
        out = torch.full((n_tok, dim), float("nan"), device="cuda")
        assert L.osmos_lane_layer(ctypes.byref(desc), g.a(x), n_tok, g.a(ids), g.a(w), g.a(add), g.a(out), wsp, need,
                                  None)
        torch.cuda.synchronize()
        return g.host(out)

    args = (ctypes.byref(desc), g.a(x), n_tok, g.a(ids), g.a(w), g.a(add), g.a(got))
    fill()
    print("noalloc eager then capture", flush=True)
    assert L.osmos_lane_layer_noalloc(*args, None)
    torch.cuda.synchronize()
    assert (g.bits(g.host(got)) == g.bits(want())).all()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        graph.capture_begin()
        assert L.osmos_lane_layer_noalloc(*args, ctypes.c_void_p(s.cuda_stream))
        graph.capture_end()
    torch.cuda.synchronize()
    for rep in range(3):
        fill()
        torch.cuda.synchronize()
        got.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        gh = g.host(got)
        ref = want()
        assert np.isfinite(ref).all()
        assert (g.bits(gh) == g.bits(ref)).all(), rep
        # eager noalloc work on the same array between replays
        assert L.osmos_lane_layer_noalloc(*args, None)
        torch.cuda.synchronize()
