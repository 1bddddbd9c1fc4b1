"""The lane's int8 expert products on the MI355X through the C ABI (q8_round, q8_group_tok, q8_gate_up): bit for bit
against the reference CPU path's golden vectors (tests/golden) and the pinned oracle on seeded inputs - every type,
16 and 32 lanes, 1 .. 8 tokens, token rows through xin, rows past a count summed and not stored, batch invariance.
(reference tests: tests/test_cpu_q8.c, tests/gpu/test_q8_gpu.hip:129-244, tests/gpu/test_cpu_q8_gpu.hip)"""
import os

import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF_TYPES = ["IQ2_XXS", "IQ2_XS", "IQ1_M", "IQ1_S", "IQ2_S", "IQ3_XXS", "Q2_K"]
ALL_TYPES = REF_TYPES + ["Q4_0", "Q4_K", "Q3_K"]
COLS = [512, 768, 2048, 4352, 5120, 7168]


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "golden_lane.npz"))


def test_q8_round_golden(g, gold):
    for cols in COLS:
        x = gold["x_%d" % cols]
        xs = cols + 32
        xp = np.zeros((x.shape[0], xs), np.float32)
        xp[:, :cols] = x
        xd = g.dev(xp)
        q = g.dev(np.zeros((x.shape[0], cols), np.int8))
        d = g.dev(np.zeros((x.shape[0], cols // 32), np.float32))
        print("q8_round cols", cols, flush=True)
        g.call("q8_round", g.a(xd), x.shape[0], cols, xs, g.a(q), g.a(d), None)
        assert (g.host(q) == gold["q_%d" % cols]).all()
        assert (g.bits(g.host(d)) == g.bits(gold["d_%d" % cols])).all()


def test_q8_round_random(g):
    rng = np.random.default_rng(0)
    x = (rng.normal(0, 1, (37, 3072)) * rng.uniform(0.01, 100, (37, 1))).astype(np.float32)
    x[3, 64:96] = 0
    q = g.dev(np.zeros((37, 3072), np.int8))
    d = g.dev(np.zeros((37, 96), np.float32))
    g.call("q8_round", g.a(g.dev(x)), 37, 3072, 3072, g.a(q), g.a(d), None)
    qo, do = orc.q8_round(x)
    assert (g.host(q) == qo).all() and (g.bits(g.host(d)) == g.bits(do)).all()


def test_q8_round_unaligned(g):
    """x rows not 16-aligned (an odd row stride, a start one float in): the one-value-a-lane form, the same bits"""
    import torch
    rng = np.random.default_rng(5)
    rows, cols, xs = 9, 512, 517
    x = (rng.normal(0, 1, (rows, cols)) * rng.uniform(0.01, 10, (rows, 1))).astype(np.float32)
    buf = np.zeros(1 + rows * xs, np.float32)
    for r in range(rows):
        buf[1 + r * xs:1 + r * xs + cols] = x[r]
    xd = g.dev(buf)
    q = g.dev(np.zeros((rows, cols), np.int8))
    d = g.dev(np.zeros((rows, cols // 32), np.float32))
    from libosmos_amd import capi
    assert capi.lib().q8_round(capi.ctypes.c_void_p(xd.data_ptr() + 4), rows, cols, xs, g.a(q), g.a(d), None)
    torch.cuda.synchronize()
    qo, do = orc.q8_round(x)
    assert (g.host(q) == qo).all() and (g.bits(g.host(d)) == g.bits(do)).all()


@pytest.mark.parametrize("name", REF_TYPES)
def test_group_tok_golden(g, gold, name):
    """6 rows x 3 tokens of each shape: the reference cpu_q8_rows's bits"""
    import torch
    t = synth.ID[name]
    for cols in COLS:
        w = g.dev(gold["w_%s_%d" % (name, cols)])
        q, d = g.dev(gold["q_%d" % cols]), g.dev(gold["d_%d" % cols])
        y = torch.full((3, 6), float("nan"), device="cuda")
        tab = g.table([w])
        cnt, xrow = g.dev(np.array([3], np.int32)), g.dev(np.array([0], np.int32))
        print("group_tok golden", name, cols, flush=True)
        g.call("q8_group_tok", t, g.a(tab), g.a(cnt), g.a(xrow), None, 1, 3, 6, cols, g.a(q), g.a(d), g.a(y), 6, None)
        assert (g.bits(g.host(y)) == g.bits(gold["y_%s_%d" % (name, cols)])).all(), cols


def _case(name, cols, rows, counts, seed, use_xin):
    """matrices of `name` each over counts[m] tokens; returns host arrays and the oracle's outputs"""
    t = synth.ID[name]
    n_tok = sum(counts)
    rng = np.random.default_rng(seed)
    ws = [synth.random_blocks(t, rows, cols, seed * 10 + m) for m in range(len(counts))]
    xrow = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    n_in = 5
    x = rng.normal(0, 1, (n_in if use_xin else n_tok, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    xin = rng.integers(0, n_in, n_tok).astype(np.int32) if use_xin else None
    want = np.zeros((n_tok, rows), np.float32)
    for m, c in enumerate(counts):
        for k in range(c):
            r = xrow[m] + k
            src = xin[r] if use_xin else r
            want[r] = orc.q8_rows(t, ws[m], rows, cols, q[src:src + 1], d[src:src + 1])[0]
    return t, ws, xrow, q, d, xin, want


@pytest.mark.parametrize("name", ALL_TYPES)
@pytest.mark.parametrize("cols", [768, 4608])
def test_group_tok_tokens(g, name, cols):
    """3 matrices at 1, 5 and 8 tokens (max_cnt 8), a ragged row count, inputs by token (xin): the oracle's bits; then
    the same tokens one launch each at max_cnt 1 - a token's bits its own (batch invariance)"""
    import torch
    rows = 75
    counts = [1, 5, 8]
    t, ws, xrow, q, d, xin, want = _case(name, cols, rows, counts, 7, True)
    wd = [g.dev(w) for w in ws]
    tab = g.table(wd)
    n_tok = sum(counts)
    y = torch.full((n_tok, rows + 3), float("nan"), device="cuda")
    print("group_tok", name, cols, flush=True)
    g.call("q8_group_tok", t, g.a(tab), g.a(g.dev(np.array(counts, np.int32))), g.a(g.dev(xrow)), g.a(g.dev(xin)), 3, 8,
           rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(y), rows + 3, None)
    yh = g.host(y)
    assert (g.bits(yh[:, :rows]) == g.bits(want)).all()
    assert np.isnan(yh[:, rows:]).all()  # nothing past `rows` written
    # one token at a time, max_cnt 1
    y1 = torch.full((n_tok, rows), float("nan"), device="cuda")
    ones = g.dev(np.ones(n_tok, np.int32))
    tab1 = g.table([wd[m] for m, c in enumerate(counts) for _ in range(c)])
    g.call("q8_group_tok", t, g.a(tab1), g.a(ones), g.a(g.dev(np.arange(n_tok, dtype=np.int32))), g.a(g.dev(xin)),
           n_tok, 1, rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(y1), rows, None)
    assert (g.bits(g.host(y1)) == g.bits(want)).all()


@pytest.mark.parametrize("name", ALL_TYPES)
def test_gate_up(g, name):
    """q8_gate_up: lane_swiglu(gate, up, lim, scale) of the two sums - the oracle's bits; with win (the weights by
    pair) and without (by row); a finite clamp and none"""
    import torch
    t = synth.ID[name]
    rows, cols = 96, 2048 if name != "Q4_0" else 1024
    counts = [2, 1, 4]
    rng = np.random.default_rng(21)
    wg = [synth.random_blocks(t, rows, cols, 300 + m) for m in range(3)]
    wu = [synth.random_blocks(t, rows, cols, 400 + m) for m in range(3)]
    n_tok = sum(counts)
    xrow = np.array([0, 2, 3], np.int32)
    x = rng.normal(0, 1, (4, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    xin = np.array([0, 1, 3, 2, 0, 1, 3], np.int32)
    scale = rng.uniform(0.05, 1, 16).astype(np.float32)
    win = np.array([5, 9, 2, 11, 0, 7, 3], np.int32)
    L = orc.orc()
    for lim, use_win in [(float("inf"), True), (0.75, False)]:
        want = np.zeros((n_tok, rows), np.float32)
        for m, c in enumerate(counts):
            for k in range(c):
                r = xrow[m] + k
                s = xin[r]
                gg = orc.q8_rows(t, wg[m], rows, cols, q[s:s + 1], d[s:s + 1])[0]
                uu = orc.q8_rows(t, wu[m], rows, cols, q[s:s + 1], d[s:s + 1])[0]
                sc = scale[win[r]] if use_win else scale[r]
                want[r] = [L.orc_lane_swiglu(float(a), float(b), lim, float(sc)) for a, b in zip(gg, uu)]
        h = torch.full((n_tok, rows), float("nan"), device="cuda")
        print("gate_up", name, lim, flush=True)
        g.call("q8_gate_up", t, g.a(g.table([g.dev(w) for w in wg])), g.a(g.table([g.dev(w) for w in wu])),
               g.a(g.dev(np.array(counts, np.int32))), g.a(g.dev(xrow)), g.a(g.dev(xin)),
               g.a(g.dev(win)) if use_win else None, 3, 4, rows, cols, g.a(g.dev(q)), g.a(g.dev(d)),
               g.a(g.dev(scale)), lim, g.a(h), rows, None)
        assert (g.bits(g.host(h)) == g.bits(want)).all()


def test_refusals(g):
    """false, nothing queued: a type not the contract's, max_cnt 0 or past 8, n 0, cols not whole blocks, hs short"""
    from libosmos_amd import capi
    L = capi.lib()
    p = capi.addr(g.dev(np.zeros(64, np.int64)))
    assert not L.q8_group_tok(13, p, p, p, None, 1, 1, 16, 512, p, p, p, 16, None)  # Q5_K
    assert not L.q8_group_tok(16, p, p, p, None, 1, 0, 16, 512, p, p, p, 16, None)
    assert not L.q8_group_tok(16, p, p, p, None, 1, 9, 16, 512, p, p, p, 16, None)
    assert not L.q8_group_tok(16, p, p, p, None, 0, 1, 16, 512, p, p, p, 16, None)
    assert not L.q8_group_tok(16, p, p, p, None, 1, 1, 16, 500, p, p, p, 16, None)
    assert not L.q8_gate_up(16, p, p, p, p, None, None, 1, 1, 16, 512, p, p, p, 1.0, p, 8, None)
    assert not L.q8_round(p, 1, 48, 48, p, p, None) and not L.q8_round(p, 1, 64, 32, p, p, None)


@pytest.mark.parametrize("name", ["Q4_0", "Q4_K", "Q3_K", "IQ3_XXS"])
@pytest.mark.parametrize("cols", [2048, 4096])
def test_group_tok_one_token_unaligned_matrix(g, name, cols):
    """one token (max_cnt 1: rows a group of 2L lanes, Q4_0 / Q4_K / Q3_K staged through LDS where the matrix is
    16-aligned): a matrix 8 bytes past a 16-byte boundary (the direct form) and the same matrix aligned give the
    oracle's bits; two matrices of one launch, one of each"""
    import torch
    t = synth.ID[name]
    rows = 70
    w = synth.random_blocks(t, rows, cols, 31)
    n = w.size
    buf = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
    buf[8:8 + n] = torch.from_numpy(np.ascontiguousarray(w).reshape(-1)).cuda()
    wa = g.dev(w)
    assert buf[8:8 + n].data_ptr() % 16 == 8 and wa.data_ptr() % 16 == 0
    x = np.random.default_rng(6).normal(0, 1, (2, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    want = orc.q8_rows(t, w, rows, cols, q, d)
    y = torch.full((2, rows), float("nan"), device="cuda")
    print("group_tok one token", name, cols, flush=True)
    g.call("q8_group_tok", t, g.a(g.table([buf[8:8 + n], wa])), g.a(g.dev(np.array([1, 1], np.int32))),
           g.a(g.dev(np.array([0, 1], np.int32))), None, 2, 1, rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(y), rows,
           None)
    assert (g.bits(g.host(y)) == g.bits(want)).all()


@pytest.mark.parametrize("name", ALL_TYPES)
@pytest.mark.parametrize("cols", [512, 1024, 2048, 4096, 8192])
def test_group_tok_one_token_wide(g, name, cols):
    """one token over 512 - 8192 columns, 16 and 32 logical lanes - for Q4_0, Q4_K, Q3_K, IQ1_S, IQ1_M from 1024 on
    the runs of 8 contract blocks a lane (Q4_0's 8 blocks and Q4_K's super-block: 144 bytes; the others' super-blocks,
    50 - 110 bytes, shifted into place in registers), for the rest group_tok_kernel: three matrices in one launch -
    ragged rows, tokens picked through xin, one matrix with no token (nothing written) - each the oracle's bits"""
    import torch
    t = synth.ID[name]
    rows = 37
    ws = [synth.random_blocks(t, rows, cols, 50 + m) for m in range(3)]
    x = np.random.default_rng(cols).normal(0, 1, (4, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    xin = np.array([3, 0, 2], np.int32)  # matrix m's token: input row xin[xrow[m]]
    y = torch.full((3, rows), float("nan"), device="cuda")
    print("group_tok one token wide", name, cols, flush=True)
    g.call("q8_group_tok", t, g.a(g.table([g.dev(w) for w in ws])), g.a(g.dev(np.array([1, 0, 1], np.int32))),
           g.a(g.dev(np.array([0, 1, 2], np.int32))), g.a(g.dev(xin)), 3, 1, rows, cols, g.a(g.dev(q)), g.a(g.dev(d)),
           g.a(y), rows, None)
    got = g.host(y)
    for m in (0, 2):
        r = xin[m]
        want = orc.q8_rows(t, ws[m], rows, cols, q[r:r + 1], d[r:r + 1])
        assert (g.bits(got[m]) == g.bits(want[0])).all(), (name, cols, m)
    assert np.isnan(got[1]).all()


@pytest.mark.parametrize("name", ALL_TYPES)
@pytest.mark.parametrize("cols", [2048, 4096])
def test_gate_up_one_token(g, name, cols):
    """q8_gate_up at one token a matrix (the reference engine's decode step; on the fused layer's gate/up tile where
    rows come in whole tiles of 4): four matrices - one with no token (nothing written), one 8 bytes past a 16-byte
    boundary - tokens picked through xin, scales through win, a finite clamp: the oracle's bits; and 70 rows (not whole
    tiles) the same"""
    import torch
    t = synth.ID[name]
    if cols % synth.TYPES[t][1]:
        pytest.skip("the type's blocks do not divide the width")
    L = orc.orc()
    rng = np.random.default_rng(cols + t)
    x = rng.normal(0, 1, (5, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    scale = rng.uniform(0.05, 1, 8).astype(np.float32)
    for rows in (96, 70):
        wg = [synth.random_blocks(t, rows, cols, 500 + m) for m in range(4)]
        wu = [synth.random_blocks(t, rows, cols, 600 + m) for m in range(4)]
        counts = np.array([1, 0, 1, 1], np.int32)
        xrow = np.array([3, 0, 1, 2], np.int32)  # matrix m's h row
        xin = np.array([4, 0, 2, 1], np.int32)   # h row r's input row
        win = np.array([6, 1, 3, 0], np.int32)   # h row r's scale
        lim = 1.5
        # matrix 2's gate and up 8 bytes past a 16-byte boundary
        n = wg[2].size
        bufs = []
        for w in (wg[2], wu[2]):
            b = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
            b[8:8 + n] = torch.from_numpy(np.ascontiguousarray(w).reshape(-1)).cuda()
            bufs.append(b)
        tg = [g.dev(w) for w in wg]
        tu = [g.dev(w) for w in wu]
        tg[2], tu[2] = bufs[0][8:8 + n], bufs[1][8:8 + n]
        h = torch.full((4, rows), float("nan"), device="cuda")
        print("gate_up one token", name, cols, rows, flush=True)
        g.call("q8_gate_up", t, g.a(g.table(tg)), g.a(g.table(tu)), g.a(g.dev(counts)), g.a(g.dev(xrow)),
               g.a(g.dev(xin)), g.a(g.dev(win)), 4, 1, rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(g.dev(scale)), lim,
               g.a(h), rows, None)
        got = g.host(h)
        for m in (0, 2, 3):
            r = xrow[m]
            s = xin[r]
            gg = orc.q8_rows(t, wg[m], rows, cols, q[s:s + 1], d[s:s + 1])[0]
            uu = orc.q8_rows(t, wu[m], rows, cols, q[s:s + 1], d[s:s + 1])[0]
            want = np.array([L.orc_lane_swiglu(float(a), float(b), lim, float(scale[win[r]])) for a, b in zip(gg, uu)],
                            np.float32)
            assert (g.bits(got[r]) == g.bits(want)).all(), (name, cols, rows, m)
        assert np.isnan(got[xrow[1]]).all()
