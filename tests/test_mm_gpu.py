"""The f16 matrix products on the MI355X through the C ABI (mm_x16, mm_x16_rows, mm_run, mm_group, mm_known, mm_fits,
mm_col_tiles) and the experts' activation into the down's f16 (q4x_swiglu_rows).

What pins them (the reference's own checks, tests/gpu/test_mm_gpu.hip:1-5,321-341): a token's outputs the same bits
alone, among others and reordered (batch invariance); each output within (cols/16 + 20) u sum |w16 x16| of the double
sum over the f16 weights (the oracle's exact decode, rounded to nearest f16) and the f16 activations it reads; the
x16 layout and rounding exactly (numpy's f16 conversion is round-to-nearest-even). mm_group's tiles the bits of
mm_run's. q4x_swiglu_rows: silu(g) u in f32 (libm exp: parity unpinned to the bit, within an f16 ulp), then f16.
"""
import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc

pytestmark = pytest.mark.gpu

MM_TYPES = ["Q8_0", "Q4_0", "IQ4_NL", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS",
            "IQ1_S", "IQ1_M", "IQ4_XS"]
U = 2.0 ** -24


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def x16_layout(x, n16=None):
    """numpy restatement of the tiled f16 layout: token t's column c at (t/16) 16 cols + (c/16) 256 + (t%16) 16 + c%16"""
    n, cols = x.shape
    n16 = n16 or (n + 15) // 16 * 16
    full = np.zeros((n16, cols), np.float16)
    full[:n] = x.astype(np.float16)
    return full.reshape(n16 // 16, 16, cols // 16, 16).transpose(0, 2, 1, 3).reshape(-1)


def mm_x16(g, x):
    import torch
    n, cols = x.shape
    xt = g.dev(x)
    x16 = torch.zeros((n + 15) // 16 * 16 * cols, dtype=torch.float16, device="cuda")
    ov = torch.zeros(1, dtype=torch.int32, device="cuda")
    g.call("mm_x16", g.a(xt), cols, n, cols, g.a(x16), g.a(ov), None)
    return x16, int(g.host(ov)[0])


def run(g, name, w, rows, cols, x16, n):
    import torch
    y = torch.full((n, rows), float("nan"), device="cuda")
    g.call("mm_run", synth.ID[name], g.a(g.dev(w)), rows, cols, g.a(x16), n, g.a(y), rows, None)
    return g.host(y)


def bound_check(name, w, rows, cols, x, y):
    wf = orc.dequant(synth.ID[name], w, rows * cols).reshape(rows, cols).astype(np.float16).astype(np.float64)
    xf = x.astype(np.float16).astype(np.float64)
    want = xf @ wf.T
    mag = np.abs(xf) @ np.abs(wf).T
    err = np.abs(y.astype(np.float64) - want)
    assert np.isfinite(y).all()
    assert (err <= (cols / 16 + 20) * U * mag).all(), (name, float((err / np.maximum(mag * U, 1e-300)).max()))


def test_x16_layout_and_overflow(g):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 3, (21, 64)).astype(np.float32)
    x16, ov = mm_x16(g, x)
    assert ov == 0
    assert (g.host(x16).view(np.uint16) == x16_layout(x).view(np.uint16)).all()
    x[3, 5] = 70000.0  # past f16's range
    _, ov = mm_x16(g, x)
    assert ov == 1
    # rows: slots from rows of x, -1 zero
    import torch
    idx = np.array([4, -1, 0, 20, 4], np.int32)
    xt = g.dev(x)
    x16 = torch.full((16 * 64,), float("nan"), dtype=torch.float16, device="cuda")
    ov = torch.zeros(1, dtype=torch.int32, device="cuda")
    g.call("mm_x16_rows", g.a(xt), 64, g.a(g.dev(idx)), 5, 64, g.a(x16), g.a(ov), None)
    sel = np.stack([x[i] if i >= 0 else np.zeros(64, np.float32) for i in idx])
    assert (g.host(x16).view(np.uint16) == x16_layout(sel).view(np.uint16)).all()
    assert int(g.host(ov)[0]) == 0


def test_queries():
    from libosmos_amd import capi
    L = capi.lib()
    for name in MM_TYPES:
        t = synth.ID[name]
        assert L.mm_known(t)
        assert L.mm_fits(t, 64, 512) and not L.mm_fits(t, 60, 512) and not L.mm_fits(t, 64, 0)
        assert L.mm_col_tiles(t, 1) == 1 and L.mm_col_tiles(t, 17) == 2 and L.mm_col_tiles(t, 64) == 4
        assert L.mm_col_tiles(t, 512) == 8
    assert not L.mm_known(0) and L.mm_col_tiles(0, 16) == 0
    assert not L.mm_fits(synth.ID["Q4_K"], 64, 128)  # not whole 256-value blocks


@pytest.mark.parametrize("name", MM_TYPES)
def test_mm_run_bound_and_invariance(g, name):
    rows, cols = 96, 512
    w = synth.random_blocks(synth.ID[name], rows, cols, 7)
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (37, cols)).astype(np.float32)
    print("mm", name, flush=True)
    x16, _ = mm_x16(g, x)
    y = run(g, name, w, rows, cols, x16, 37)
    bound_check(name, w, rows, cols, x, y)
    # a token's bits its own: alone, and in a reordered batch
    for t in (0, 17, 36):
        one16, _ = mm_x16(g, x[t:t + 1])
        assert (g.bits(run(g, name, w, rows, cols, one16, 1)[0]) == g.bits(y[t])).all()
    perm = rng.permutation(37)
    p16, _ = mm_x16(g, x[perm])
    yp = run(g, name, w, rows, cols, p16, 37)
    assert (g.bits(yp) == g.bits(y[perm])).all()


@pytest.mark.parametrize("name", ["IQ3_XXS", "Q4_K", "IQ2_XXS"])
def test_mm_run_wide(g, name):
    """DeepSeek-sized columns (7168) and 80 tokens (5 tiles: two launches' worth of 4-tile blocks)"""
    rows, cols = 64, 7168
    w = synth.iq_blocks(synth.ID[name], rows, cols, 9) if name.startswith("IQ") else synth.random_blocks(
        synth.ID[name], rows, cols, 9)
    x = np.random.default_rng(5).normal(0, 1, (80, cols)).astype(np.float32)
    x16, _ = mm_x16(g, x)
    y = run(g, name, w, rows, cols, x16, 80)
    bound_check(name, w, rows, cols, x, y)



@pytest.mark.parametrize("name", ["Q8_0", "Q6_K", "IQ3_XXS", "Q4_K"])
def test_mm_many_tokens_and_tall(g, name):
    """150 tokens (10 token tiles: 2 a workgroup for the 128-value slabs of Q8_0 / Q6_K / IQ3_XXS, 4 for Q4_K's) within the bound and each token's bits its own; then mm_group over 16 matrices of 4096 rows (the
    4-row-tile form, or for Q6_K's 2-byte staging words - 9 blocks a row - one row tile) - each matrix the bits of
    mm_run on it alone"""
    import torch
    t = synth.ID[name]
    gen = synth.iq_blocks if name.startswith("IQ") else synth.random_blocks
    rows, cols = 64, 512
    w = gen(t, rows, cols, 31)
    x = np.random.default_rng(12).normal(0, 1, (150, cols)).astype(np.float32)
    print("mm many tokens", name, flush=True)
    x16, _ = mm_x16(g, x)
    y = run(g, name, w, rows, cols, x16, 150)
    bound_check(name, w, rows, cols, x, y)
    for k in (0, 77, 149):
        one16, _ = mm_x16(g, x[k:k + 1])
        assert (g.bits(run(g, name, w, rows, cols, one16, 1)[0]) == g.bits(y[k])).all(), k
    # tall: 16 matrices x 64 row blocks of 64 = 1024 row blocks, 3 tokens each
    n_mat, rows, cols, per = 16, 4096, 2304, 3  # (2304: the tuned K split for mm_run too; 9 blocks a row)
    mats = [gen(t, rows, cols, 40 + e) for e in range(n_mat)]
    rng = np.random.default_rng(13)
    xs = [rng.normal(0, 1, (per, cols)).astype(np.float32) for _ in range(n_mat)]
    x16 = np.concatenate([x16_layout(xs[e], 16) for e in range(n_mat)])
    xoff = (np.arange(n_mat) * 16 * cols).astype(np.uint32)
    yoff = (np.arange(n_mat) * per * rows).astype(np.uint32)
    cnt = np.full(n_mat, per, np.int32)
    y = torch.full((n_mat * per, rows), float("nan"), device="cuda")
    wd = [g.dev(m) for m in mats]
    x16d = g.dev(x16.view(np.uint16)).view(torch.float16)
    print("mm tall group", name, flush=True)
    g.call("mm_group", t, g.a(g.table(wd)), g.a(g.dev(cnt)), n_mat, per, rows, cols, g.a(x16d), g.a(g.dev(xoff)), cols,
           g.a(y), g.a(g.dev(yoff)), rows, None)
    got = g.host(y)
    for e in (0, 7, 15):
        one16, _ = mm_x16(g, xs[e])
        alone = run(g, name, mats[e], rows, cols, one16, per)
        assert (g.bits(got[e * per:(e + 1) * per]) == g.bits(alone)).all(), e

def test_mm_group(g):
    """three experts' gathered tokens (5, 16, 23: whole tiles each) over one x16, outputs at their own offsets: each
    the bits of mm_run on that expert alone; an expert with 0 tokens writes nothing"""
    import torch
    name, rows, cols = "IQ3_XXS", 64, 1024
    t = synth.ID[name]
    mats = [synth.iq_blocks(t, rows, cols, 20 + e) for e in range(4)]
    cnt = np.array([5, 16, 23, 0], np.int32)
    rng = np.random.default_rng(8)
    xs = [rng.normal(0, 1, (max(c, 1), cols)).astype(np.float32) for c in cnt]
    tiles = [(c + 15) // 16 for c in cnt]
    x16 = np.concatenate([x16_layout(xs[e][:max(cnt[e], 1)], 16 * max(tiles[e], 1)) for e in range(4)])
    xoff = np.cumsum([0] + [16 * max(tt, 1) * cols for tt in tiles])[:4].astype(np.uint32)
    yoff = np.cumsum([0] + [int(c) * rows for c in cnt])[:4].astype(np.uint32)
    y = torch.full((int(cnt.sum()) + 1, rows), float("nan"), device="cuda")
    wd = [g.dev(m) for m in mats]
    x16d = g.dev(x16.view(np.uint16)).view(torch.float16)
    g.call("mm_group", t, g.a(g.table(wd)), g.a(g.dev(cnt)), 4, 23, rows, cols, g.a(x16d), g.a(g.dev(xoff)), cols,
           g.a(y), g.a(g.dev(yoff)), rows, None)
    got = g.host(y)
    for e in range(3):
        one16, _ = mm_x16(g, xs[e][:cnt[e]])
        alone = run(g, name, mats[e], rows, cols, one16, int(cnt[e]))
        assert (g.bits(got[yoff[e] // rows:yoff[e] // rows + cnt[e]]) == g.bits(alone)).all(), e
    assert np.isnan(got[-1]).all()  # the empty expert's place untouched


def test_refusals(g):
    import torch
    from libosmos_amd import capi
    L = capi.lib()
    x16 = torch.zeros(16 * 256, dtype=torch.float16, device="cuda")
    y = torch.zeros(16, 64, device="cuda")
    w = g.dev(synth.random_blocks(synth.ID["Q4_K"], 64, 256, 1))
    assert not L.mm_run(0, capi.addr(w), 64, 256, capi.addr(x16), 1, capi.addr(y), 64, None)  # unknown type
    assert not L.mm_run(synth.ID["Q4_K"], capi.addr(w), 60, 256, capi.addr(x16), 1, capi.addr(y), 64, None)
    assert not L.mm_run(synth.ID["Q4_K"], capi.addr(w), 64, 256, capi.addr(x16), 0, capi.addr(y), 64, None)
    assert not L.mm_run(synth.ID["Q4_K"], capi.addr(w), 64, 256, capi.addr(x16), 2049, capi.addr(y), 64, None)
    xf = torch.zeros(4, 30, device="cuda")
    assert not L.mm_x16(capi.addr(xf), 30, 4, 30, capi.addr(x16), None, None)  # cols not a multiple of 16


def test_swiglu_rows(g):
    import torch
    rng = np.random.default_rng(12)
    ff, rows_ = 64, 6
    gg = rng.normal(0, 3, (rows_, ff)).astype(np.float32)
    uu = rng.normal(0, 3, (rows_, ff)).astype(np.float32)
    idx = np.array([2, -1, 5, 0, 2], np.int32)
    x16 = torch.full((16 * ff,), float("nan"), dtype=torch.float16, device="cuda")
    ov = torch.zeros(1, dtype=torch.int32, device="cuda")
    g.call("q4x_swiglu_rows", g.a(g.dev(gg)), g.a(g.dev(uu)), ff, g.a(g.dev(idx)), 5, g.a(x16), g.a(ov), None)
    got = g.host(x16).reshape(-1)
    silu = (gg.astype(np.float64) / (1.0 + np.exp(-gg.astype(np.float64)))).astype(np.float32)
    h = (silu * uu).astype(np.float32)
    sel = np.stack([h[i] if i >= 0 else np.zeros(ff, np.float32) for i in idx])
    want = x16_layout(sel)
    # the slots written: within an f16 ulp of the f32 reference (exp's last bit is libm's), zeros exact
    live = np.zeros((16, ff), bool)
    live[:5] = True
    livev = x16_layout(live.astype(np.float32)).astype(bool)
    a16, b16 = got[livev].astype(np.float32), want[livev].astype(np.float32)
    ulp = np.spacing(np.abs(want[livev]).astype(np.float16)).astype(np.float32)
    assert (np.abs(a16 - b16) <= ulp).all()
    zero = np.zeros((16, ff), np.float32)
    zero[1] = 1.0  # slot 1 (idx -1): exact zeros
    zv = x16_layout(zero).astype(bool)
    assert (got[zv] == 0).all()
    assert np.isnan(got[~livev]).all()  # the tile's rows past the slots untouched
    assert int(g.host(ov)[0]) == 0


@pytest.mark.parametrize("name,cols,group", [("Q8_0", 2048, False), ("Q8_0", 320, False), ("Q4_K", 2048, False),
                                             ("Q5_K", 512, False), ("Q6_K", 1536, False), ("Q6_K", 1536, True),
                                             ("Q4_0", 512, False), ("IQ4_NL", 512, False), ("Q2_K", 1024, False),
                                             ("Q3_K", 1024, False), ("IQ2_XXS", 1024, False), ("IQ2_XS", 1024, True),
                                             ("IQ2_S", 1024, False), ("IQ1_S", 1024, False), ("IQ1_M", 1024, True),
                                             ("IQ3_XXS", 2048, True), ("IQ4_XS", 512, False)])
def test_mm_partition_order(g, name, cols, group):
    """the reference's K split, bit for bit: on data where every matrix-core step is exact (tests/mmorder.py) mm_run
    (or mm_group) gives the oracle's bits - the partitions' chains and their ordered sum - which differ from a single
    chain's in K order"""
    import torch
    from tests import mmorder
    t = synth.ID[name]
    w, x, ordered, chain = mmorder.case(name, cols, group, 7)
    want = orc.mm_rows(t, w, 16, cols, x, group)
    x16, _ = mm_x16(g, x)
    n = x.shape[0]
    print("mm order", name, cols, group, flush=True)
    if group:
        y = torch.full((n, 16), float("nan"), device="cuda")
        z = np.zeros(1, np.uint32)
        g.call("mm_group", t, g.a(g.table([g.dev(w)])), g.a(g.dev(np.array([n], np.int32))), 1, n, 16, cols, g.a(x16),
               g.a(g.dev(z)), cols, g.a(y), g.a(g.dev(z)), 16, None)
        got = g.host(y)
    else:
        got = run(g, name, w, 16, cols, x16, n)
    assert (g.bits(got) == g.bits(want)).all()


def test_swiglu_side_and_rows_agree(g):
    """q4x_swiglu's F32 output within an ulp-level bound of float64 SiLU (exp is the device library's: parity
    unpinned to the bit); its f16 side copy byte for byte mm_x16's of that output; and q4x_swiglu_rows on the same
    rows the same bytes as q4x_swiglu then mm_x16_rows (the reference's own check, tests/gpu/test_q4x_moe_gpu.hip:117-
    130); in place (y = g) the same values"""
    import ctypes
    import torch
    from libosmos_amd import capi
    rng = np.random.default_rng(21)
    rows_, ff = 37, 96
    gg = rng.normal(0, 3, (rows_, ff)).astype(np.float32)
    uu = rng.normal(0, 3, (rows_, ff)).astype(np.float32)
    n = rows_ * ff
    y = torch.full((rows_, ff), float("nan"), device="cuda")
    x16 = torch.full((48 * ff,), float("nan"), dtype=torch.float16, device="cuda")
    ov = torch.zeros(1, dtype=torch.int32, device="cuda")
    side = capi.Q4xX16(x16.data_ptr(), ov.data_ptr(), ff, 3)  # rows 3 .. 39 of the tiled x16
    gd, ud = g.dev(gg), g.dev(uu)
    g.call("q4x_swiglu", g.a(gd), g.a(ud), n, g.a(y), ctypes.byref(side), None)
    yh = g.host(y)
    ref = gg.astype(np.float64) / (1.0 + np.exp(-gg.astype(np.float64))) * uu.astype(np.float64)
    assert (np.abs(yh - ref) <= 4 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-30).all()
    # the side copy: mm_x16 of y, placed at rows 3 ..
    want16 = torch.zeros(48 * ff, dtype=torch.float16, device="cuda")
    ov2 = torch.zeros(1, dtype=torch.int32, device="cuda")
    padded = np.zeros((40, ff), np.float32)
    padded[3:] = yh
    g.call("mm_x16", g.a(g.dev(padded)), ff, 40, ff, g.a(want16), g.a(ov2), None)
    got16 = g.host(x16).reshape(-1).view(np.uint16)
    w16 = g.host(want16).reshape(-1).view(np.uint16)
    live = np.zeros((48, ff), np.float32)
    live[3:40] = 1.0
    lv = x16_layout(live, 48).astype(bool)
    assert (got16[lv] == w16[lv]).all()
    assert np.isnan(g.host(x16).reshape(-1)[~lv]).all()
    assert int(g.host(ov)[0]) == 0
    # q4x_swiglu_rows over the same rows = q4x_swiglu then mm_x16_rows, byte for byte
    idx = np.array([5, -1, 0, 36, 5, 17], np.int32)
    r16 = torch.zeros(16 * ff, dtype=torch.float16, device="cuda")
    g.call("q4x_swiglu_rows", g.a(gd), g.a(ud), ff, g.a(g.dev(idx)), len(idx), g.a(r16), g.a(ov), None)
    m16 = torch.zeros(16 * ff, dtype=torch.float16, device="cuda")
    g.call("mm_x16_rows", g.a(y), ff, g.a(g.dev(idx)), len(idx), ff, g.a(m16), g.a(ov2), None)
    assert (g.host(r16).view(np.uint16) == g.host(m16).view(np.uint16)).all()
    # in place
    g.call("q4x_swiglu", g.a(gd), g.a(ud), n, g.a(gd), None, None)
    assert (g.bits(g.host(gd)) == g.bits(yh)).all()


def test_f16_overflow_rule():
    """the side copies' and mm_x16's overflow flag is the reference's rule (kernels/mm.h:47-50): a value past 65504 or
    not a number, judged before rounding - 65510 rounds to 65504 and is still flagged; 65504 itself is not"""
    import ctypes
    import torch
    from libosmos_amd import capi
    from tests import gpu_util as g
    ff = 16
    for v, flagged in ((65504.0, False), (65510.0, True), (-70000.0, True), (float("nan"), True), (1.0, False)):
        x = np.ones((1, ff), np.float32)
        x[0, 5] = v
        x16 = torch.zeros(16 * ff, dtype=torch.float16, device="cuda")
        ov = torch.zeros(1, dtype=torch.int32, device="cuda")
        g.call("mm_x16", g.a(g.dev(x)), ff, 1, ff, g.a(x16), g.a(ov), None)
        assert bool(g.host(ov)[0]) == flagged, v
        ov.zero_()
        side = capi.Q4xX16(x16.data_ptr(), ov.data_ptr(), ff, 0)
        one = g.dev(np.full((1, ff), 1e30, np.float32))  # silu(1e30) = 1e30: u = v / 1e30 gives y = v
        uu = g.dev((x / np.float32(1e30)).astype(np.float32))
        y = torch.zeros(1, ff, device="cuda")
        g.call("q4x_swiglu", g.a(one), g.a(uu), ff, g.a(y), ctypes.byref(side), None)
        if np.isfinite(v):
            assert bool(g.host(ov)[0]) == (abs(float(g.host(y)[0, 5])) > 65504.0), v


def test_spin_holds_the_stream():
    """q4x_spin holds its stream for at least the asked time (events around it), and refuses nothing"""
    import torch
    from tests import gpu_util as g
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    g.call("q4x_spin", 2000, None)
    b.record()
    torch.cuda.synchronize()
    assert a.elapsed_time(b) >= 1.9
