"""The fp32 decode matvec on the MI355X through the C ABI (mv_run, mv_strided, mv_group, mv_group_tok) and the exact
decode (quant_dequant): bit for bit against the reference CPU path's golden vectors and the pinned oracle - every
type, 1 .. 8 tokens and a prompt's 11 and 64, strided slices, groups, ragged rows.
(reference tests: tests/gpu/test_mv_gpu.hip:145-232, tests/test_cpu_expert.c, tests/gpu/test_quant_gpu.hip)"""
import os

import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MV_TYPES = ["F32", "BF16", "Q8_0", "Q4_0", "IQ4_NL", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ2_XXS", "IQ2_XS", "IQ2_S",
            "IQ3_XXS", "IQ1_S", "IQ1_M", "IQ4_XS"]


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def weights(name, rows, cols, seed):
    t = synth.ID[name]
    if name == "F32":
        return np.random.default_rng(seed).normal(0, 0.1, (rows, cols)).astype(np.float32).view(np.uint8)
    if name == "BF16":
        f = np.random.default_rng(seed).normal(0, 0.1, (rows, cols)).astype(np.float32)
        return (f.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(rows, -1)
    return synth.random_blocks(t, rows, cols, seed)


def test_mv_golden(g):
    import torch
    lane = np.load(os.path.join(GOLD, "golden_lane.npz"))
    mv = np.load(os.path.join(GOLD, "golden_mv.npz"))
    for name in ["IQ2_XXS", "IQ2_XS", "IQ1_M", "IQ1_S", "IQ2_S", "IQ3_XXS", "Q2_K"]:
        for cols in [512, 768, 2048, 4352, 5120, 7168]:
            w = g.dev(lane["w_%s_%d" % (name, cols)])
            x = g.dev(lane["x_%d" % cols])
            y = torch.full((3, 6), float("nan"), device="cuda")
            print("mv golden", name, cols, flush=True)
            g.call("mv_run", synth.ID[name], g.a(w), 6, cols, g.a(x), 3, g.a(y), None)
            assert (g.bits(g.host(y)) == g.bits(mv["ym_%s_%d" % (name, cols)])).all()


@pytest.mark.parametrize("name", MV_TYPES)
def test_mv_strided_tokens(g, name):
    """1 .. 4, 8, 11 and 64 tokens, x and y slices of wider rows: the oracle's bits, each token's alone"""
    import torch
    t = synth.ID[name]
    rows, cols = 45, 2048
    w = weights(name, rows, cols, 5)
    wd = g.dev(w)
    rng = np.random.default_rng(1)
    for n_tok in (1, 2, 3, 4, 8, 11, 64):
        xs, ys = cols + 16, rows + 5
        x = rng.normal(0, 1, (n_tok, xs)).astype(np.float32)
        want = orc.mv_rows(t, w, rows, cols, x[:, :cols])
        y = torch.full((n_tok, ys), float("nan"), device="cuda")
        print("mv_strided", name, n_tok, flush=True)
        g.call("mv_strided", t, g.a(wd), rows, cols, g.a(g.dev(x)), xs, n_tok, g.a(y), ys, None)
        yh = g.host(y)
        assert (g.bits(yh[:, :rows]) == g.bits(want)).all(), n_tok
        assert np.isnan(yh[:, rows:]).all()


@pytest.mark.parametrize("name", ["Q4_0", "Q4_K", "Q3_K", "IQ3_XXS", "IQ1_S", "Q8_0"])
def test_mv_group_and_group_tok(g, name):
    import torch
    t = synth.ID[name]
    rows, cols, n = 40, 1024, 5
    ws = [weights(name, rows, cols, 50 + m) for m in range(n)]
    tab = g.table([g.dev(w) for w in ws])
    rng = np.random.default_rng(2)
    # mv_group: x_div 2 (two matrices a vector), x_mat cols
    x = rng.normal(0, 1, (3, cols)).astype(np.float32)
    y = torch.full((n, rows), float("nan"), device="cuda")
    print("mv_group", name, flush=True)
    g.call("mv_group", t, g.a(tab), n, rows, cols, g.a(g.dev(x)), cols, 2, g.a(y), None)
    want = np.stack([orc.mv_rows(t, ws[m], rows, cols, x[m // 2:m // 2 + 1])[0] for m in range(n)])
    assert (g.bits(g.host(y)) == g.bits(want)).all()
    # mv_group_tok: counts 2, 0 (skipped), 3, 1, 2 at max_cnt 3
    cnt = np.array([2, 0, 3, 1, 2], np.int32)
    xrow = np.array([0, 2, 2, 5, 6], np.int32)
    xt = rng.normal(0, 1, (8 + 3, cols)).astype(np.float32)
    y = torch.full((11, rows), float("nan"), device="cuda")
    g.call("mv_group_tok", t, g.a(tab), g.a(g.dev(cnt)), g.a(g.dev(xrow)), n, 3, rows, cols, g.a(g.dev(xt)), cols,
           g.a(y), rows, None)
    yh = g.host(y)
    for m in range(n):
        for k in range(cnt[m]):
            r = xrow[m] + k
            assert (g.bits(yh[r]) == g.bits(orc.mv_rows(t, ws[m], rows, cols, xt[r:r + 1])[0])).all()
    assert np.isnan(yh[8:]).all()


@pytest.mark.parametrize("name", [n for n in MV_TYPES if n != "F32"])
def test_dequant(g, name):
    import torch
    t = synth.ID[name]
    w = weights(name, 8, 512, 77)
    values = 8 * 512
    out = torch.full((values,), float("nan"), device="cuda")
    g.call("quant_dequant", t, g.a(g.dev(w)), values, g.a(out), None)
    assert (g.bits(g.host(out)) == g.bits(orc.dequant(t, w.reshape(-1), values))).all()


def test_refusals(g):
    from libosmos_amd import capi
    L = capi.lib()
    p = capi.addr(g.dev(np.zeros(64, np.int64)))
    assert not L.mv_run(99, p, 16, 512, p, 1, p, None)
    assert not L.mv_run(2, p, 16, 512, p, 9, p, None)  # past MV_MAX_TOKENS
    assert not L.mv_run(12, p, 16, 500, p, 1, p, None)
    assert not L.mv_strided(2, p, 16, 512, p, 500, 2, p, 16, None)  # a stride shorter than the row
    assert not L.mv_group(2, p, 0, 16, 512, p, 0, 1, p, None) and not L.mv_group(2, p, 2, 16, 512, p, 0, 0, p, None)
    assert not L.mv_group_tok(2, p, p, p, 1, 9, 16, 512, p, 512, p, 16, None)
    assert not L.quant_known(99) and L.quant_known(18)


@pytest.mark.parametrize("name", ["Q4_K", "IQ1_M", "IQ2_S", "IQ4_NL"])
def test_mv_one_token_unaligned_matrix(g, name):
    """one token, a matrix whose start is 8- but not 16-byte aligned: the launch keeps the direct path (the staged
    path copies rows with 16-byte loads and takes only 16-aligned matrices) - the oracle's bits, the same as the
    aligned copy's"""
    import torch
    t = synth.ID[name]
    rows, cols = 70, 2048
    w = weights(name, rows, cols, 9)
    n = w.size
    buf = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
    buf[8:8 + n] = torch.from_numpy(np.ascontiguousarray(w).reshape(-1)).cuda()
    wa = g.dev(w)
    x = np.random.default_rng(4).normal(0, 1, (1, cols)).astype(np.float32)
    want = orc.mv_rows(t, w, rows, cols, x)
    xd = g.dev(x)
    for wt, what in ((buf[8:8 + n], "offset 8"), (wa, "aligned")):
        assert wt.data_ptr() % 16 == (8 if what == "offset 8" else 0)
        y = torch.full((1, rows), float("nan"), device="cuda")
        print("mv_run one token", name, what, flush=True)
        g.call("mv_run", t, g.a(wt), rows, cols, g.a(xd), 1, g.a(y), None)
        assert (g.bits(g.host(y)) == g.bits(want)).all(), what


@pytest.mark.parametrize("name", ["Q2_K", "Q4_K", "Q5_K", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ1_M", "IQ1_S",
                                  "IQ4_XS", "IQ4_NL"])
def test_mv_group_mixed_alignment(g, name):
    """mv_group over the types whose rows the launch stages through LDS, at cols 2048 (a row a whole number of 16-byte
    words): a table mixing 16-aligned matrices with ones that start 8 bytes past a 16-byte boundary, so one launch
    takes the staged path for some matrices and the direct path for others - the oracle's bits for every matrix"""
    import torch
    t = synth.ID[name]
    rows, cols, n = 70, 2048, 6
    ws = [weights(name, rows, cols, 90 + m) for m in range(n)]
    keep = []
    for m, w in enumerate(ws):
        b = w.size
        buf = torch.zeros(b + 64, dtype=torch.uint8, device="cuda")
        off = 8 if m % 2 else 0
        buf[off:off + b] = torch.from_numpy(np.ascontiguousarray(w).reshape(-1)).cuda()
        keep.append(buf[off:off + b])
        assert keep[-1].data_ptr() % 16 == off
    tab = g.table(keep)
    x = np.random.default_rng(6).normal(0, 1, (n, cols)).astype(np.float32)
    y = torch.full((n, rows), float("nan"), device="cuda")
    print("mv_group mixed alignment", name, flush=True)
    g.call("mv_group", t, g.a(tab), n, rows, cols, g.a(g.dev(x)), cols, 1, g.a(y), None)
    yh = g.host(y)
    for m in range(n):
        assert (g.bits(yh[m]) == g.bits(orc.mv_rows(t, ws[m], rows, cols, x[m:m + 1])[0])).all(), m
