"""The MoE plumbing and the whole routed lane layer on the MI355X through the C ABI: q4x_route, q4x_expert_tiles,
q4x_moe_sum, ops_* and osmos_lane_tables against independent restatements of their documented contracts, and
osmos_lane_layer bit for bit against the reference CPU lane's golden layer and the oracle at batches 1 / 4 / 32.
(reference: include/osmos/gpu/q4x_ops.h:356-384, tests/gpu/test_q4x_moe_gpu.hip, tests/test_cpu_lane.c)"""
import ctypes
import math
import os

import numpy as np
import pytest

from libosmos_amd import capi, synth
from oracle import orc

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def test_route(g):
    """ids: the k greatest softmax probabilities (lowest id among equals) - exact; weights p / sum within 1e-6 (the
    device's exp and the host's need not agree to the bit); rows[t k + j] = t"""
    import torch
    rng = np.random.default_rng(1)
    for n_exp, k, n_tok in [(512, 10, 7), (256, 8, 33), (64, 4, 3), (1024, 32, 2)]:
        logits = rng.normal(0, 2, (n_tok, n_exp)).astype(np.float32)
        logits[0, 5] = logits[0, 9] = logits[0].max() + 1  # a tie: the lower id first
        ids = torch.zeros(n_tok * k, dtype=torch.int32, device="cuda")
        w = torch.zeros(n_tok * k, dtype=torch.float32, device="cuda")
        rows = torch.zeros(n_tok * k, dtype=torch.int32, device="cuda")
        g.call("q4x_route", g.a(g.dev(logits)), n_tok, n_exp, k, g.a(ids), g.a(w), g.a(rows), None)
        oi = np.zeros(n_tok * k, np.int32)
        ow = np.zeros(n_tok * k, np.float32)
        orc.orc().orc_route(orc.ptr(logits), n_tok, n_exp, k, orc.ptr(oi), orc.ptr(ow))
        assert (g.host(ids) == oi).all()
        assert ids[0].item() == 5 and ids[1].item() == 9
        assert np.allclose(g.host(w), ow, rtol=1e-6, atol=0)
        assert (g.host(rows) == np.repeat(np.arange(n_tok), k)).all()


def test_route_ties_and_zeros(g):
    """all logits equal (every probability the same: the k lowest ids in order), and fewer finite logits than k (the
    rest of the picks are the zero-probability experts, lowest ids first), against the oracle's ids and weights"""
    import torch
    n_exp, k = 64, 8
    logits = np.zeros((3, n_exp), np.float32)
    logits[1, :] = -np.inf
    logits[1, [40, 3, 17, 60, 9]] = [1.0, 0.5, 1.0, -2.0, 0.25]
    logits[2, :] = np.linspace(-3, 3, n_exp).astype(np.float32)[::-1]
    n_tok = logits.shape[0]
    ids = torch.zeros(n_tok * k, dtype=torch.int32, device="cuda")
    w = torch.zeros(n_tok * k, dtype=torch.float32, device="cuda")
    rows = torch.zeros(n_tok * k, dtype=torch.int32, device="cuda")
    g.call("q4x_route", g.a(g.dev(logits)), n_tok, n_exp, k, g.a(ids), g.a(w), g.a(rows), None)
    oi = np.zeros(n_tok * k, np.int32)
    ow = np.zeros(n_tok * k, np.float32)
    orc.orc().orc_route(orc.ptr(logits), n_tok, n_exp, k, orc.ptr(oi), orc.ptr(ow))
    gi = g.host(ids)
    assert (gi == oi).all()
    assert (gi[:k] == np.arange(k)).all()
    assert (gi[k:k + 5] == [17, 40, 3, 9, 60]).all() and (gi[k + 5:2 * k] == [0, 1, 2]).all()
    assert np.allclose(g.host(w), ow, rtol=1e-6, atol=0)


def tiles_ref(ids, k, n_exp, dim, ff, bases, nbytes):
    """q4x_expert_tiles' contract restated on the host (a stable sort by expert)"""
    n = len(ids)
    bd = capi.Q4xExpertBounds()
    capi.lib().q4x_expert_bounds(n, n_exp, ctypes.byref(bd))
    order = np.argsort(ids, kind="stable")
    where = np.empty(n, np.int64)
    where[order] = np.arange(n)
    count = np.bincount(ids, minlength=n_exp)
    place0 = np.concatenate([[0], np.cumsum(count)[:-1]])
    tiles = (count + 15) // 16 * 16
    slot0 = np.concatenate([[0], np.cumsum(tiles)[:-1]])
    gidx = -np.ones(bd.slots, np.int64)
    hidx = -np.ones(bd.slots, np.int64)
    for i in range(n):
        e = ids[i]
        q = where[i]
        gidx[slot0[e] + q - place0[e]] = i // k
        hidx[slot0[e] + q - place0[e]] = q
    entries = {r: [] for r in range(4)}
    for e in range(n_exp):
        c = int(count[e])
        for part in range((c + 127) // 128):
            m = min(128, c - part * 128)
            r = 0 if m <= 16 else 1 if m <= 32 else 2 if m <= 64 else 3
            slot, place = slot0[e] + part * 128, place0[e] + part * 128
            entries[r].append((m, slot * dim, slot * ff, place * ff, place * dim,
                               [bases[j] + e * nbytes[j] for j in range(3)]))
    return bd, where, gidx, hidx, entries


def test_expert_tiles(g):
    """the tables at decode, mid and prefill sizes (the in-workgroup placement up to 1024 picks, the per-expert one
    beyond), experts at a base + stride or through an address table, and the scratch's per-expert figures"""
    import torch
    rng = np.random.default_rng(2)
    cases = [(3, 10, 512, False), (512, 8, 256, False), (40, 4, 64, True), (100, 8, 256, False), (128, 8, 256, True),
             (129, 8, 256, False), (300, 10, 1024, True), (1, 1, 1, False)]
    for _ in range(12):  # random shapes: expert counts off the powers of two, k up to 32, both placement paths
        n_exp = int(rng.integers(1, 1025))
        k = int(rng.integers(1, min(32, n_exp) + 1))
        cases.append((int(rng.integers(1, 2600 // k + 1)), k, n_exp, bool(rng.integers(0, 2))))
    for n_tok, k, n_exp, use_tab in cases:
        if n_tok >= 128 and n_exp >= 8 * k:  # Zipf(1.1) load skew, distinct experts a token
            p = 1.0 / np.arange(1, n_exp + 1) ** 1.1
            p /= p.sum()
            ids = np.concatenate([rng.choice(n_exp, k, replace=False, p=p) for _ in range(n_tok)]).astype(np.int32)
        else:
            ids = np.concatenate([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
        n = len(ids)
        dim, ff = 2048, 512
        if use_tab:  # experts anywhere: a scattered table of addresses per tensor
            tabs = [(rng.integers(1, 1 << 40, n_exp) * 256).astype(np.int64) for _ in range(3)]
            bases, nbytes = [0, 0, 0], [0, 0, 0]
        else:
            tabs = None
            bases, nbytes = [0x10000000, 0x20000000, 0x30000000], [4096, 4096, 8192]
        bd, where, gidx, hidx, entries = tiles_ref(ids, k, n_exp, dim, ff, bases, nbytes)
        if use_tab:
            for r in range(4):
                entries[r] = [(m, a, b, c, d, [int(tabs[j][e]) for j in range(3)])
                              for (m, a, b, c, d, _), e in zip(entries[r], tiles_experts(ids, n_exp, r))]
        E, S = bd.entries, bd.slots
        T = lambda m, dt=torch.int32: torch.full((max(m, 1),), -7, dtype=dt, device="cuda")  # noqa: E731
        cnt, gi, hi, wh, off = T(E), T(S), T(S), T(n), T(3 * n_exp)
        xg, yg, xd, yd = (T(E, torch.int32) for _ in range(4))
        ptrs = [torch.zeros(max(E, 1), dtype=torch.int64, device="cuda") for _ in range(3)]
        dtabs = [torch.from_numpy(tb).cuda() for tb in tabs] if use_tab else None
        t = capi.Q4xExpertTiles()
        for j in range(3):
            t.base[j], t.bytes[j], t.ptr[j] = bases[j], nbytes[j], ptrs[j].data_ptr()
            t.tab[j] = dtabs[j].data_ptr() if use_tab else None
        t.cnt, t.gidx, t.hidx, t.where, t.off = cnt.data_ptr(), gi.data_ptr(), hi.data_ptr(), wh.data_ptr(), off.data_ptr()
        t.xg, t.yg, t.xd, t.yd = xg.data_ptr(), yg.data_ptr(), xd.data_ptr(), yd.data_ptr()
        g.call("q4x_expert_tiles", g.a(g.dev(ids)), n, k, n_exp, dim, ff, ctypes.byref(t), None)
        assert (g.host(wh) == where).all(), n
        assert (g.host(gi)[:S] == gidx).all() and (g.host(hi)[:S] == hidx).all(), n
        count = np.bincount(ids, minlength=n_exp)
        oh = g.host(off)
        assert (oh[2 * n_exp:] == count).all()
        assert (oh[:n_exp] == np.concatenate([[0], np.cumsum(count)[:-1]])).all()
        assert (oh[n_exp:2 * n_exp] == np.concatenate([[0], np.cumsum((count + 15) // 16 * 16)[:-1]])).all()
        ch = g.host(cnt)
        host = {nm: g.host(v).astype(np.int64) for nm, v in [("xg", xg), ("xd", xd), ("yg", yg), ("yd", yd)]}
        ph = [g.host(p_) for p_ in ptrs]
        for r in range(4):
            live = entries[r]
            for i in range(bd.count[r]):
                en = bd.first[r] + i
                if i < len(live):
                    m, a, b, c, d, pp = live[i]
                    assert ch[en] == m and host["xg"][en] == a and host["xd"][en] == b, (n, r, i)
                    assert host["yg"][en] == c and host["yd"][en] == d, (n, r, i)
                    assert [int(ph[j][en]) for j in range(3)] == pp, (n, r, i)
                else:
                    assert ch[en] == 0, (n, r, i)


def tiles_experts(ids, n_exp, r):
    """the expert of each live entry of run r, in entry order"""
    count = np.bincount(ids, minlength=n_exp)
    out = []
    for e in range(n_exp):
        c = int(count[e])
        for part in range((c + 127) // 128):
            m = min(128, c - part * 128)
            if (0 if m <= 16 else 1 if m <= 32 else 2 if m <= 64 else 3) == r:
                out.append(e)
    return out


def test_moe_sum_and_ops(g):
    import torch
    rng = np.random.default_rng(3)
    n_tok, k, dim = 5, 4, 256
    y = rng.normal(0, 1, (n_tok * k, dim)).astype(np.float32)
    where = rng.permutation(n_tok * k).astype(np.int32)
    w = rng.uniform(0, 1, n_tok * k).astype(np.float32)
    sh = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    sl = rng.normal(0, 1, n_tok).astype(np.float32)
    out = torch.zeros((n_tok, dim), device="cuda")
    g.call("q4x_moe_sum", g.a(g.dev(y)), g.a(g.dev(where)), g.a(g.dev(w)), n_tok, k, dim, g.a(g.dev(sh)), g.a(g.dev(sl)),
           g.a(out), None)
    want = np.zeros((n_tok, dim), np.float32)
    orc.orc().orc_moe_sum(orc.ptr(y), orc.ptr(where), orc.ptr(w), n_tok, k, dim, orc.ptr(sh), orc.ptr(sl), orc.ptr(want))
    assert np.allclose(g.host(out), want, rtol=1e-6, atol=1e-6)
    # the weighted sum before the gate is exact to the order: compare with the gate's term removed
    out0 = torch.zeros((n_tok, dim), device="cuda")
    g.call("q4x_moe_sum", g.a(g.dev(y)), g.a(g.dev(where)), g.a(g.dev(w)), n_tok, k, dim,
           g.a(g.dev(np.zeros_like(sh))), g.a(g.dev(sl)), g.a(out0), None)
    want0 = np.zeros((n_tok, dim), np.float32)
    for j in range(k):
        want0 = (want0 + (y[where.reshape(n_tok, k)[:, j]] * w.reshape(n_tok, k)[:, j:j + 1]).astype(np.float32))
    assert (g.bits(g.host(out0)) == g.bits(want0 + np.float32(0))).all()
    # gather_sum_add: the sum in j's order, then add's
    idx = rng.integers(0, n_tok * k, n_tok * k).astype(np.int32)
    add = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    o = torch.zeros((n_tok, dim), device="cuda")
    g.call("ops_gather_sum_add", g.a(o), g.a(g.dev(y)), g.a(g.dev(idx)), k, n_tok, dim, g.a(g.dev(add)), None)
    want = np.zeros((n_tok, dim), np.float32)
    orc.orc().orc_gather_sum_add(orc.ptr(want), orc.ptr(y), orc.ptr(idx), k, n_tok, dim, orc.ptr(add))
    assert (g.bits(g.host(o)) == g.bits(want)).all()
    # swiglu_lane: lane_swiglu's bits
    gg, uu = rng.normal(0, 3, (3, 64)).astype(np.float32), rng.normal(0, 3, (3, 64)).astype(np.float32)
    sc = rng.uniform(0, 1, 3).astype(np.float32)
    h = torch.zeros((3, 64), device="cuda")
    g.call("ops_swiglu_lane", g.a(g.dev(gg)), g.a(g.dev(uu)), 64, 2.5, g.a(g.dev(sc)), 3, g.a(h), None)
    L = orc.orc()
    want = np.array([[L.orc_lane_swiglu(float(a), float(b), 2.5, float(sc[t])) for a, b in zip(gg[t], uu[t])]
                     for t in range(3)], np.float32)
    assert (g.bits(g.host(h)) == g.bits(want)).all()


def _lane_layer_oracle(type_, x, ids, wts, gate, up, down, dim, ff, lim, type_down=None):
    """the reference CPU lane's layer (oracle): pairs sorted by (expert, pick), tokens' rows in ascending expert id"""
    n_tok, k = ids.shape
    pairs = sorted((int(ids[t, j]), t * k + j) for t in range(n_tok) for j in range(k))
    rows_x = np.stack([x[m // k] for _, m in pairs]).astype(np.float32)
    scale = np.array([wts.reshape(-1)[m] for _, m in pairs], np.float32)
    experts = sorted(set(e for e, _ in pairs))
    row0 = np.array([min(r for r, (e, _) in enumerate(pairs) if e == ex) for ex in experts], np.uint32)
    cnt = np.array([sum(1 for e, _ in pairs if e == ex) for ex in experts], np.uint32)
    P = ctypes.c_void_p
    tab = lambda mats: (P * len(experts))(*[mats[e].ctypes.data for e in experts])  # noqa: E731
    ye = np.zeros((len(pairs), dim), np.float32)
    assert orc.orc().orc_lane_layer(type_, type_ if type_down is None else type_down, dim, ff, lim, orc.ptr(rows_x), orc.ptr(scale), len(pairs), tab(gate),
                                    tab(up), tab(down), orc.ptr(row0), orc.ptr(cnt), len(experts), orc.ptr(ye))
    row_of = {m: r for r, (_, m) in enumerate(pairs)}
    order = np.array([sorted(row_of[t * k + j] for j in range(k)) for t in range(n_tok)], np.int32).reshape(-1)
    out = np.zeros((n_tok, dim), np.float32)
    orc.orc().orc_gather_sum_add(orc.ptr(out), orc.ptr(ye), orc.ptr(order), k, n_tok, dim, None)
    return out


def test_lane_layer_golden(g):
    """osmos_lane_layer on the golden layer (the reference CPU lane's bits): dim 512, ff 256, IQ3_XXS, top-2 of 4"""
    import torch
    from libosmos_amd.layer import LaneLayer
    gd = np.load(os.path.join(GOLD, "golden_layer.npz"))
    t3 = synth.ID["IQ3_XXS"]
    gate, up, down = (g.dev(np.ascontiguousarray(gd[k_])) for k_ in ("gate", "up", "down"))
    L = LaneLayer(t3, t3, 512, 256, 4, 2, gate.reshape(4, -1), up.reshape(4, -1), down.reshape(4, -1))
    out = torch.full((3, 512), float("nan"), device="cuda")
    L.forward(g.dev(gd["x"]), g.dev(gd["ids"].astype(np.int32)), g.dev(gd["wts"]), torch.zeros((3, 512), device="cuda"),
              out)
    assert (g.bits(g.host(out)) == g.bits(gd["out"])).all()


@pytest.mark.parametrize("n_tok", [1, 4, 32])
def test_lane_layer_qwen_shape(g, n_tok):
    """the config's MoE layer shape (hidden 2048, expert ff 512, top-10) over 64 experts: the oracle's bits at each
    batch, and each token's bits its own (the batch of 1 row by row)"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t3 = synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff = 64, 10, 2048, 512
    rng = np.random.default_rng(n_tok)
    gate = [synth.iq_blocks(t3, ff, dim, 1000 + e) for e in range(n_exp)]
    up = [synth.iq_blocks(t3, ff, dim, 2000 + e) for e in range(n_exp)]
    down = [synth.iq_blocks(t3, dim, ff, 3000 + e) for e in range(n_exp)]
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    wts = rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32)
    want = _lane_layer_oracle(t3, x, ids, wts, gate, up, down, dim, ff, math.inf)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(t3, t3, dim, ff, n_exp, k, D(gate), D(up), D(down))
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("lane layer", n_tok, flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()
    if n_tok > 1:
        one = torch.full((1, dim), float("nan"), device="cuda")
        for t in (0, n_tok - 1):
            L.forward(g.dev(x[t:t + 1]), g.dev(ids[t:t + 1]), g.dev(wts[t:t + 1]), torch.zeros((1, dim), device="cuda"), one)
            assert (g.bits(g.host(one)[0]) == g.bits(want[t])).all()


@pytest.mark.parametrize("name", ["IQ1_S", "IQ1_M", "IQ2_XXS"])
@pytest.mark.parametrize("n_tok", [1, 4])
def test_lane_layer_deepseek_shape(g, name, n_tok):
    """the DeepSeek-style expert shape (hidden 7168, expert ff 2048: 32 lanes a gate/up row, 16 a down row), top-9
    (8 routed + the shared one as a ninth pick) over 24 experts: the oracle's bits"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t = synth.ID[name]
    n_exp, k, dim, ff = 24, 9, 7168, 2048
    rng = np.random.default_rng(50 + n_tok)
    gate = [synth.iq_blocks(t, ff, dim, 100 + e) for e in range(n_exp)]
    up = [synth.iq_blocks(t, ff, dim, 200 + e) for e in range(n_exp)]
    down = [synth.iq_blocks(t, dim, ff, 300 + e) for e in range(n_exp)]
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids = np.stack([np.concatenate([rng.choice(n_exp - 1, k - 1, replace=False), [n_exp - 1]]) for _ in range(n_tok)])
    ids = ids.astype(np.int32)
    wts = rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32)
    want = _lane_layer_oracle(t, x, ids, wts, gate, up, down, dim, ff, math.inf)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(t, t, dim, ff, n_exp, k, D(gate), D(up), D(down))
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("deepseek layer", name, n_tok, flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()


@pytest.mark.parametrize("name", ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ1_S", "IQ1_M", "Q2_K", "Q4_0", "Q4_K", "Q3_K"])
def test_lane_layer_one_token_types(g, name):
    """a single token (the decode kernels: one gate/up tile a workgroup) for every lane type, dim 2048 (16 lanes a row)
    and 4096 (32), with a finite clamp: the oracle's bits"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t = synth.ID[name]
    for dim, ff in ((2048, 256), (4096, 512)):
        n_exp, k = 12, 5
        mk = synth.iq_blocks if name.startswith("IQ") else synth.random_blocks
        gate = [mk(t, ff, dim, 400 + e) for e in range(n_exp)]
        up = [mk(t, ff, dim, 500 + e) for e in range(n_exp)]
        down = [mk(t, dim, ff, 600 + e) for e in range(n_exp)]
        rng = np.random.default_rng(dim)
        x = rng.normal(0, 1, (1, dim)).astype(np.float32)
        ids, wts = _route(rng, 1, n_exp, k)
        want = _lane_layer_oracle(t, x, ids, wts, gate, up, down, dim, ff, 1.5)
        D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
        L = LaneLayer(t, t, dim, ff, n_exp, k, D(gate), D(up), D(down), lim=1.5)
        out = torch.full((1, dim), float("nan"), device="cuda")
        print("one-token layer", name, dim, flush=True)
        L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((1, dim), device="cuda"), out)
        assert (g.bits(g.host(out)) == g.bits(want)).all(), (name, dim)


@pytest.mark.parametrize("name", ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ1_S", "IQ1_M", "Q2_K", "Q4_0", "Q4_K", "Q3_K"])
def test_lane_layer_batch_types(g, name):
    """a batch of 7 tokens over 6 experts (each expert picked by several tokens: the batch gate/up kernel's full and
    one-token passes) for every lane type, dim 2048 (16 lanes a row) and 4096 (32), with a finite clamp: the oracle's
    bits"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t = synth.ID[name]
    for dim, ff in ((2048, 256), (4096, 512)):
        n_exp, k, n_tok = 6, 3, 7
        mk = synth.iq_blocks if name.startswith("IQ") else synth.random_blocks
        gate = [mk(t, ff, dim, 700 + e) for e in range(n_exp)]
        up = [mk(t, ff, dim, 800 + e) for e in range(n_exp)]
        down = [mk(t, dim, ff, 900 + e) for e in range(n_exp)]
        rng = np.random.default_rng(dim + 1)
        x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
        ids, wts = _route(rng, n_tok, n_exp, k)
        want = _lane_layer_oracle(t, x, ids, wts, gate, up, down, dim, ff, 1.5)
        D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
        L = LaneLayer(t, t, dim, ff, n_exp, k, D(gate), D(up), D(down), lim=1.5)
        out = torch.full((n_tok, dim), float("nan"), device="cuda")
        print("batch layer", name, dim, flush=True)
        L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
        assert (g.bits(g.host(out)) == g.bits(want)).all(), (name, dim)


@pytest.mark.parametrize("n_tok", [1, 5])
def test_lane_layer_other_dims(g, n_tok):
    """a hidden size outside the one-token / batch tiles' ranges (3072: between 2048 and 4096) - the general gate/up
    kernel: the oracle's bits"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t3 = synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff = 8, 3, 3072, 512
    gate, up, down = _layer_case(t3, t3, n_exp, k, dim, ff, 31)
    rng = np.random.default_rng(31 + n_tok)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids, wts = _route(rng, n_tok, n_exp, k)
    want = _lane_layer_oracle(t3, x, ids, wts, gate, up, down, dim, ff, 1.25)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(t3, t3, dim, ff, n_exp, k, D(gate), D(up), D(down), lim=1.25)
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("other dims layer", n_tok, flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()


def test_lane_layer_largest_batch(g):
    """the largest batch (64 tokens, top-10 of 16 experts: 640 picks, up to 64 tokens an expert): the oracle's bits"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t3 = synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff, n_tok = 16, 10, 1024, 256, 64
    gate, up, down = _layer_case(t3, t3, n_exp, k, dim, ff, 21)
    rng = np.random.default_rng(21)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids, wts = _route(rng, n_tok, n_exp, k)
    want = _lane_layer_oracle(t3, x, ids, wts, gate, up, down, dim, ff, math.inf)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(t3, t3, dim, ff, n_exp, k, D(gate), D(up), D(down))
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("largest batch layer", flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()


def _layer_case(tg, td, n_exp, k, dim, ff, seed):
    gate = [synth.iq_blocks(tg, ff, dim, seed + 1000 + e) for e in range(n_exp)]
    up = [synth.iq_blocks(tg, ff, dim, seed + 2000 + e) for e in range(n_exp)]
    down = [synth.iq_blocks(td, dim, ff, seed + 3000 + e) for e in range(n_exp)]
    return gate, up, down


def _route(rng, n_tok, n_exp, k):
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    return ids, rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32)


def test_lane_layer_mixed_types(g):
    """gate/up and down of different types (the two-launch path): the oracle's bits, with a finite clamp"""
    import torch
    from libosmos_amd.layer import LaneLayer
    tg, td = synth.ID["IQ2_XXS"], synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff, n_tok = 16, 4, 2048, 512, 5
    gate, up, down = _layer_case(tg, td, n_exp, k, dim, ff, 7)
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids, wts = _route(rng, n_tok, n_exp, k)
    want = _lane_layer_oracle(tg, x, ids, wts, gate, up, down, dim, ff, 0.75, type_down=td)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(tg, td, dim, ff, n_exp, k, D(gate), D(up), D(down), lim=0.75)
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("mixed layer", flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()


def test_lane_layer_repeat_and_graph(g):
    """the one-launch layer's control words are left zeroed by every call: calls in a row on one workspace, and a
    captured graph replayed with eager calls between, each the oracle's bits (shared experts across tokens too)"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t3 = synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff, n_tok = 12, 6, 1024, 256, 8
    gate, up, down = _layer_case(t3, t3, n_exp, k, dim, ff, 11)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(t3, t3, dim, ff, n_exp, k, D(gate), D(up), D(down), lim=2.0)
    rng = np.random.default_rng(11)
    cases = []
    for _ in range(3):
        x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
        ids, wts = _route(rng, n_tok, n_exp, k)
        add = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
        want = _lane_layer_oracle(t3, x, ids, wts, gate, up, down, dim, ff, 2.0) + add
        cases.append(([g.dev(a) for a in (x, ids, wts, add)], want))
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("repeat layer", flush=True)
    for _ in range(2):
        for (x, ids, wts, add), want in cases:
            out.fill_(float("nan"))
            L.forward(x, ids, wts, add, out)
            assert (g.bits(g.host(out)) == g.bits(want)).all()
    # a graph of the first case, replayed between eager calls of the others
    (x, ids, wts, add), want = cases[0]
    L.workspace(n_tok)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            L.forward(x, ids, wts, add, out, stream=ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    for r in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert (g.bits(g.host(out)) == g.bits(want)).all(), r
        (x1, ids1, wts1, add1), want1 = cases[1 + r % 2]
        o1 = torch.full((n_tok, dim), float("nan"), device="cuda")
        L.forward(x1, ids1, wts1, add1, o1)
        assert (g.bits(g.host(o1)) == g.bits(want1)).all()


def test_lane_layer_halves(g):
    """osmos_lane_gate_up then osmos_lane_down (h kept by the caller): the same bits as osmos_lane_layer, and as the
    oracle"""
    import torch
    from libosmos_amd.layer import LaneLayer
    t3 = synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff, n_tok = 12, 6, 1024, 256, 3
    gate, up, down = _layer_case(t3, t3, n_exp, k, dim, ff, 23)
    D = lambda ms: g.dev(np.stack(ms)).reshape(n_exp, -1)  # noqa: E731
    L = LaneLayer(t3, t3, dim, ff, n_exp, k, D(gate), D(up), D(down))
    rng = np.random.default_rng(23)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids, wts = _route(rng, n_tok, n_exp, k)
    want = _lane_layer_oracle(t3, x, ids, wts, gate, up, down, dim, ff, math.inf)
    xd, idd, wd, add = g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda")
    h = torch.full((n_tok * k, ff), float("nan"), device="cuda")
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    lib = capi.lib()
    print("layer halves", flush=True)
    assert lib.osmos_lane_gate_up(ctypes.byref(L.desc), capi.addr(xd), n_tok, capi.addr(idd), capi.addr(wd),
                                  capi.addr(h), None)
    assert lib.osmos_lane_down(ctypes.byref(L.desc), capi.addr(h), n_tok, capi.addr(idd), capi.addr(add),
                               capi.addr(out), None)
    torch.cuda.synchronize()
    assert (g.bits(g.host(out)) == g.bits(want)).all()
    one = torch.full((n_tok, dim), float("nan"), device="cuda")
    L.forward(xd, idd, wd, add, one)
    assert (g.bits(g.host(one)) == g.bits(want)).all()
    # refusals: nothing queued
    assert not lib.osmos_lane_gate_up(ctypes.byref(L.desc), capi.addr(xd), 0, capi.addr(idd), capi.addr(wd),
                                      capi.addr(h), None)
    assert not lib.osmos_lane_down(ctypes.byref(L.desc), capi.addr(h), 65, capi.addr(idd), capi.addr(add),
                                   capi.addr(out), None)
