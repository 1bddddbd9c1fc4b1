"""Q5_KR (Q5_K repacked in tiles of 16 rows) and the f16 decode on the MI355X through the C ABI: quant_repack_q5k's
bytes those of the numpy restatement (tests/q5kr.py), and - the reference's own check, tests/gpu/test_mm_gpu.hip:
290-309 - mm_run, mm_group and mv_strided giving QUANT_Q5_KR the bits they give Q5_K (1 .. 150 tokens, the short
and tuned K splits, the tall four-row-tile form); quant_dequant_f16 the f16 (nearest, ties to even: numpy's
conversion) of quant_dequant's values for every type; the refusals the reference's header names."""
import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc
from tests import q5kr
from tests.test_mm_gpu import MM_TYPES, mm_x16, run, x16_layout

pytestmark = pytest.mark.gpu

Q5K = synth.ID["Q5_K"]
Q5KR = 0x100 | Q5K


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def repack(g, w, rows, cols):
    import torch
    out = torch.full((rows * (cols // 256) * 180,), 0xA5, dtype=torch.uint8, device="cuda")
    g.call("quant_repack_q5k", g.a(g.dev(w)), rows, cols, g.a(out), None)
    return out


@pytest.mark.parametrize("rows,cols", [(16, 256), (48, 768), (4096, 2304)])
def test_repack_bytes(g, rows, cols):
    print("repack", rows, cols, flush=True)
    w = synth.random_blocks(Q5K, rows, cols, rows + cols)
    got = g.host(repack(g, w, rows, cols))
    assert (got == q5kr.repack(np.asarray(w, np.uint8).reshape(-1), rows, cols)).all()


def test_repack_refusals(g):
    from libosmos_amd import capi
    L = capi.lib()
    w = g.dev(synth.random_blocks(Q5K, 32, 512, 1))
    import torch
    d = torch.zeros(32 * 2 * 180, dtype=torch.uint8, device="cuda")
    p, q = capi.addr(w), capi.addr(d)
    assert not L.quant_repack_q5k(p, 24, 512, q, None)  # rows not whole tiles
    assert not L.quant_repack_q5k(p, 32, 500, q, None)  # cols not whole blocks
    assert not L.quant_repack_q5k(p, 32, 512, p, None)  # in place
    assert not L.quant_repack_q5k(p, 0, 512, q, None) and not L.quant_repack_q5k(None, 32, 512, q, None)
    assert not L.quant_dequant(Q5KR, q, 512, q, None) and not L.quant_known(Q5KR)  # not a dequant type
    assert L.mm_known(Q5KR) and L.mm_fits(Q5KR, 64, 512) and not L.mm_fits(Q5KR, 60, 512)
    assert L.mm_col_tiles(Q5KR, 17) == 2
    x = torch.zeros(512, device="cuda")
    y = torch.zeros(64, device="cuda")
    assert not L.mv_strided(Q5KR, q, 24, 512, capi.addr(x), 512, 1, capi.addr(y), 24, None)  # rows not whole tiles
    tab = g.table([d])
    assert not L.mv_group(Q5KR, capi.addr(tab), 1, 32, 512, capi.addr(x), 0, 1, capi.addr(y), None)  # mv_strided's alone


@pytest.mark.parametrize("cols", [512, 2304])
def test_mm_run_bits_of_q5k(g, cols):
    rows = 96
    w = synth.random_blocks(Q5K, rows, cols, 3)
    wr = repack(g, w, rows, cols)
    x = np.random.default_rng(2).normal(0, 1, (150, cols)).astype(np.float32)
    for n in (1, 16, 37, 150):
        print("mm q5kr", cols, n, flush=True)
        x16, _ = mm_x16(g, x[:n])
        want = run(g, "Q5_K", w, rows, cols, x16, n)
        import torch
        y = torch.full((n, rows), float("nan"), device="cuda")
        g.call("mm_run", Q5KR, g.a(wr), rows, cols, g.a(x16), n, g.a(y), rows, None)
        assert (g.bits(g.host(y)) == g.bits(want)).all(), n


def test_mm_group_tall_bits_of_q5k(g):
    """16 matrices of 4096 rows (1024 row blocks of 64: the four-row-tile form), 3 tokens each"""
    import torch
    n_mat, rows, cols, per = 16, 4096, 512, 3
    mats = [synth.random_blocks(Q5K, rows, cols, 60 + e) for e in range(n_mat)]
    rng = np.random.default_rng(14)
    xs = [rng.normal(0, 1, (per, cols)).astype(np.float32) for _ in range(n_mat)]
    x16 = g.dev(np.concatenate([x16_layout(xs[e], 16) for e in range(n_mat)]).view(np.uint16)).view(torch.float16)
    xoff = g.dev((np.arange(n_mat) * 16 * cols).astype(np.uint32))
    yoff = g.dev((np.arange(n_mat) * per * rows).astype(np.uint32))
    cnt = g.dev(np.full(n_mat, per, np.int32))
    out = {}
    for t, wd in ((Q5K, [g.dev(m) for m in mats]), (Q5KR, [repack(g, m, rows, cols) for m in mats])):
        print("mm_group", hex(t), flush=True)
        y = torch.full((n_mat * per, rows), float("nan"), device="cuda")
        g.call("mm_group", t, g.a(g.table(wd)), g.a(cnt), n_mat, per, rows, cols, g.a(x16), g.a(xoff), cols, g.a(y),
               g.a(yoff), rows, None)
        out[t] = g.host(y)
    assert np.isfinite(out[Q5K]).all()
    assert (g.bits(out[Q5KR]) == g.bits(out[Q5K])).all()


def test_mv_strided_bits_of_q5k(g):
    import torch
    rows, cols = 80, 1024
    w = synth.random_blocks(Q5K, rows, cols, 8)
    wd, wr = g.dev(w), repack(g, w, rows, cols)
    xs, ys = cols + 64, rows + 16
    x = np.random.default_rng(6).normal(0, 1, (64, xs)).astype(np.float32)
    xd = g.dev(x)
    for n in (1, 2, 3, 4, 5, 8, 11, 64):
        print("mv q5kr", n, flush=True)
        got = {}
        for t, m in ((Q5K, wd), (Q5KR, wr)):
            y = torch.full((n, ys), float("nan"), device="cuda")
            g.call("mv_strided", t, g.a(m), rows, cols, g.a(xd), xs, n, g.a(y), ys, None)
            got[t] = g.host(y)[:, :rows]
        assert (g.bits(got[Q5KR]) == g.bits(got[Q5K])).all(), n
        # and the oracle's bits (the matvec's own check)
        assert (g.bits(got[Q5KR]) == g.bits(orc.mv_rows(Q5K, w, rows, cols, x[:n, :cols]))).all(), n


@pytest.mark.parametrize("name", MM_TYPES + ["BF16"])
def test_dequant_f16(g, name):
    import torch
    t = synth.ID[name]
    rows, cols = 8, 512
    if name == "BF16":
        f = np.random.default_rng(3).normal(0, 0.1, (rows, cols)).astype(np.float32)
        w = (f.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    elif name.startswith("IQ"):
        w = synth.iq_blocks(t, rows, cols, 9)
    else:
        w = synth.random_blocks(t, rows, cols, 9)
    values = rows * cols
    out = torch.full((values,), float("nan"), dtype=torch.float16, device="cuda")
    g.call("quant_dequant_f16", t, g.a(g.dev(w)), values, g.a(out), None)
    want = orc.dequant(t, np.asarray(w).reshape(-1), values).astype(np.float16)
    assert (g.host(out).view(np.uint16) == want.view(np.uint16)).all()
