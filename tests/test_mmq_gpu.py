"""mmq on the MI355X's int8 matrix cores through the C ABI (mmq_x8_rows, mmq_group): bit for bit against the pinned
oracle at 1 / 16 / 37 / 64 tokens and every column tiling, a token's bits its own whatever the batch.
(reference test: tests/gpu/test_mmq_gpu.hip:66-233)"""
import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def x8_dev(g, x, idx, cols):
    import torch
    slots = len(idx)
    padded = (slots + 15) // 16 * 16
    x8 = torch.zeros(padded * cols, dtype=torch.int8, device="cuda")
    dx = torch.zeros(padded * (cols // 32), dtype=torch.float32, device="cuda")
    sx = torch.zeros(padded * (cols // 32), dtype=torch.float32, device="cuda")
    g.call("mmq_x8_rows", g.a(g.dev(x)), x.shape[1], g.a(g.dev(np.asarray(idx, np.int32))), slots, cols, g.a(x8),
           g.a(dx), g.a(sx), None)
    return x8, dx, sx


@pytest.mark.parametrize("cols,pad", [(2048, 32), (7168, 32), (2048, 1)])
def test_x8_rows(g, cols, pad):
    """the oracle's codes, dx and sx; a row stride of cols + 1 (rows not 16-aligned) takes the one-value-a-lane form"""
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (9, cols + pad)).astype(np.float32)
    x[3, 96:128] = 0
    idx = [0, 3, -1, 8, 2, 3, 7]
    x8, dx, sx = x8_dev(g, x, idx, cols)
    o8, odx, osx = orc.mmq_x8_rows(x, idx, cols)
    assert (g.host(x8) == o8).all()
    assert (g.bits(g.host(dx)) == g.bits(odx)).all() and (g.bits(g.host(sx)) == g.bits(osx)).all()


@pytest.mark.parametrize("cols", [2048, 1280])
def test_group(g, cols):
    """three matrices at 1, 16 and 37 tokens (two-tile passes and a last one-tile pass), then 64 tokens; then 5 and 33;
    all the oracle's"""
    import torch
    rows = 64
    t = synth.ID["Q4_K"]
    rng = np.random.default_rng(8)
    for counts in ([1, 16, 37], [64], [5, 33]):
        n_mat = len(counts)
        ws = [synth.random_blocks(t, rows, cols, 60 + m) for m in range(n_mat)]
        soff = np.concatenate([[0], np.cumsum([(c + 15) // 16 * 16 for c in counts])[:-1]]).astype(np.uint32)
        slots = int(soff[-1] + (counts[-1] + 15) // 16 * 16)
        x = rng.normal(0, 1, (slots, cols)).astype(np.float32)
        idx = np.arange(slots, dtype=np.int32)
        x8, dx, sx = x8_dev(g, x, idx, cols)
        o8, odx, osx = orc.mmq_x8_rows(x, idx, cols)
        yoff = np.array([int(so) * rows for so in soff], np.uint32)
        y = torch.full((slots * rows,), float("nan"), device="cuda")
        print("mmq_group", counts, cols, flush=True)
        g.call("mmq_group", t, g.a(g.table([g.dev(w) for w in ws])), g.a(g.dev(np.array(counts, np.int32))), n_mat,
               max(counts), rows, cols, g.a(x8), g.a(dx), g.a(sx), g.a(g.dev(soff)), g.a(y), g.a(g.dev(yoff)), rows,
               None)
        yh = g.host(y).reshape(slots, rows)
        for m, c in enumerate(counts):
            for k in range(c):
                s = int(soff[m]) + k
                want = orc.mmq_rows(ws[m], rows, cols, o8, odx, osx, s)
                assert (g.bits(yh[s]) == g.bits(want)).all(), (counts, m, k)
            for k in range(c, (c + 15) // 16 * 16):
                assert np.isnan(yh[int(soff[m]) + k]).all()  # the slots past the count not written


def test_refusals(g):
    from libosmos_amd import capi
    L = capi.lib()
    p = capi.addr(g.dev(np.zeros(64, np.int64)))
    assert not L.mmq_known(16) and L.mmq_known(12)
    assert not L.mmq_group(16, p, p, 1, 1, 16, 256, p, p, p, p, p, p, 16, None)
    assert not L.mmq_group(12, p, p, 1, 1, 20, 256, p, p, p, p, p, p, 20, None)
    assert not L.mmq_group(12, p, p, 1, 1, 16, 250, p, p, p, p, p, p, 16, None)
    assert not L.mmq_x8_rows(p, 16, p, 1, 48, p, p, p, None)


def test_group_dense_passes_split(g):
    """one matrix over 200 tokens (7 passes of two tiles, spread over workgroups along z): the oracle's bits on a row
    subset, and each of three tokens alone the same bits as in the batch"""
    import torch
    rows, cols, n = 128, 2048, 200
    t = synth.ID["Q4_K"]
    w = synth.random_blocks(t, rows, cols, 91)
    x = np.random.default_rng(92).normal(0, 1, (n, cols)).astype(np.float32)
    idx = np.arange(n, dtype=np.int32)
    x8, dx, sx = x8_dev(g, x, idx, cols)
    o8, odx, osx = orc.mmq_x8_rows(x, idx, cols)
    z = np.zeros(1, np.uint32)
    y = torch.full((n * rows,), float("nan"), device="cuda")
    print("mmq_group dense 200", flush=True)
    g.call("mmq_group", t, g.a(g.table([g.dev(w)])), g.a(g.dev(np.array([n], np.int32))), 1, n, rows, cols, g.a(x8),
           g.a(dx), g.a(sx), g.a(g.dev(z)), g.a(y), g.a(g.dev(z)), rows, None)
    yh = g.host(y).reshape(n, rows)
    for k in range(0, n, 7):
        want = orc.mmq_rows(w, rows, cols, o8, odx, osx, k)
        assert (g.bits(yh[k]) == g.bits(want)).all(), k
    for k in (0, 101, 199):
        a8, adx, asx = x8_dev(g, x, [k], cols)
        y1 = torch.full((rows,), float("nan"), device="cuda")
        g.call("mmq_group", t, g.a(g.table([g.dev(w)])), g.a(g.dev(np.array([1], np.int32))), 1, 1, rows, cols,
               g.a(a8), g.a(adx), g.a(asx), g.a(g.dev(z)), g.a(y1), g.a(g.dev(z)), rows, None)
        assert (g.bits(g.host(y1)) == g.bits(yh[k])).all(), k
