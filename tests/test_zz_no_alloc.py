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
