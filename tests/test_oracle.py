"""The CPU oracle pinned (CPU only): against the reference's own compiled CPU path's golden vectors
(tests/golden/make_golden.py), the reference codebooks' checksums, independent float64 dequantisation and the
contracts' closed forms and bounds. Every oracle function the GPU tests lean on is pinned here by something that would
catch a dropped term, a swapped index or a wrong rounding.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc
from tests import refdecode

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LANE_TYPES = ["IQ2_XXS", "IQ2_XS", "IQ1_M", "IQ1_S", "IQ2_S", "IQ3_XXS", "Q2_K"]
COLS = [512, 768, 2048, 4352, 5120, 7168]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def lane_gold():
    return np.load(os.path.join(GOLD, "golden_lane.npz"))


def test_grids_match_reference_checksums():
    """each expanded codebook's bytes hash to the reference's quant_grids.h table's (gen_grids.py recorded them)"""
    sums = json.load(open(os.path.join(GOLD, "grids.json")))["sha256"]
    L = orc.orc()
    for i, name in enumerate(["iq2xxs", "iq2xs", "iq2s", "iq1s", "iq3xxs", "ksigns"]):
        n = orc.U32()
        p = L.orc_table(i, orc._c.byref(n))
        raw = orc._c.string_at(p, n.value)
        assert hashlib.sha256(raw).hexdigest() == sums[name], name


def test_grid_invariants():
    """the structural facts of the codebooks (gguf-py's maps): IQ2 magnitudes {8, 25, 43}, IQ1 {-1, 0, 1}, IQ3 {4 .. 62};
    the sign table an index with its parity in bit 7; no two entries alike"""
    L = orc.orc()
    for i, vals, n in [(0, {8, 25, 43}, 256), (1, {8, 25, 43}, 512), (2, {8, 25, 43}, 1024), (3, {255, 0, 1}, 2048)]:
        size = orc.U32()
        t = np.frombuffer(orc._c.string_at(L.orc_table(i, orc._c.byref(size)), size.value), np.uint64)
        assert len(t) == n and len(set(t.tolist())) == n
        assert set(np.unique(t.view(np.uint8)).tolist()) == vals
    size = orc.U32()
    t3 = np.frombuffer(orc._c.string_at(L.orc_table(4, orc._c.byref(size)), size.value), np.uint32)
    assert set(np.unique(t3.view(np.uint8)).tolist()) == {4, 12, 20, 28, 36, 44, 52, 62} and len(set(t3.tolist())) == 256
    ks = np.frombuffer(orc._c.string_at(L.orc_table(5, orc._c.byref(size)), size.value), np.uint8)
    for i in range(128):
        assert ks[i] == i | ((bin(i).count("1") & 1) << 7)
        assert bin(int(ks[i])).count("1") % 2 == 0  # an even count of negatives


def test_q8_round_golden(lane_gold):
    """the oracle's rounding gives the reference cpu_q8_round's bytes and scales (round-half-even, d = amax / 127,
    a zero block -> d 0, a lone -2.5 -> -127)"""
    for cols in COLS:
        q, d = orc.q8_round(lane_gold["x_%d" % cols])
        assert (q == lane_gold["q_%d" % cols]).all() and (bits(d) == bits(lane_gold["d_%d" % cols])).all()
        assert d[0, 0] == 0.0 and (q[0, :32] == 0).all() and q[1, 37] == -127


def test_q8_round_closed_form():
    """rint(x * (127 / amax)) against float64 on random and tie-making inputs"""
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (64, 256)).astype(np.float32)
    x[5, :32] = np.arange(32, dtype=np.float32) - 16  # ties at .5 after scaling
    q, d = orc.q8_round(x)
    g = x.reshape(64, 8, 32)
    amax = np.abs(g).max(axis=2)
    inv = np.where(amax > 0, np.float32(127.0) / amax, 0).astype(np.float32)
    want = np.rint((g * inv[:, :, None]).astype(np.float32)).astype(np.int8).reshape(64, 256)
    assert (q == want).all()
    assert (bits(d) == bits((amax / np.float32(127.0)).astype(np.float32))).all()


@pytest.mark.parametrize("name", LANE_TYPES)
def test_lane_rows_golden(lane_gold, name):
    """the oracle's lane contract gives the reference cpu_q8_rows's bits: every type, 16 and 32 lanes, half-vector tails"""
    t = synth.ID[name]
    for cols in COLS:
        w = lane_gold["w_%s_%d" % (name, cols)]
        y = orc.q8_rows(t, w, w.shape[0], cols, lane_gold["q_%d" % cols], lane_gold["d_%d" % cols])
        assert (bits(y) == bits(lane_gold["y_%s_%d" % (name, cols)])).all(), cols


@pytest.mark.parametrize("name", LANE_TYPES)
def test_mv_rows_golden(lane_gold, name):
    """the oracle's fp32 matvec gives the reference cpu_mv_rows's bits (mv.h rows_of's order over quant.h's values)"""
    mv = np.load(os.path.join(GOLD, "golden_mv.npz"))
    t = synth.ID[name]
    for cols in COLS:
        w = lane_gold["w_%s_%d" % (name, cols)]
        y = orc.mv_rows(t, w, w.shape[0], cols, lane_gold["x_%d" % cols])
        assert (bits(y) == bits(mv["ym_%s_%d" % (name, cols)])).all(), cols


def test_lane_exp_swiglu_golden():
    """lane_exp and lane_swiglu: the reference kernels/lane.h's bits, compiled by the reference's own flags"""
    g = np.load(os.path.join(GOLD, "golden_exp.npz"))
    L = orc.orc()
    y = np.array([L.orc_lane_exp(float(v)) for v in g["x"]], np.float32)
    assert (bits(y) == bits(g["y"])).all()
    h = np.array([L.orc_lane_swiglu(float(a), float(b), float(c), float(e))
                  for a, b, c, e in zip(g["g"], g["u"], g["lim"], g["scale"])], np.float32)
    assert (bits(h) == bits(g["h"])).all()
    # and within 2 ulp of e^x where it is normal (its documented bound)
    x = g["x"][(g["x"] > -80) & (g["x"] < 88)]
    e = np.array([L.orc_lane_exp(float(v)) for v in x], np.float64)
    assert np.all(np.abs(e - np.exp(x.astype(np.float64))) <= 2.5 * np.spacing(np.exp(x).astype(np.float32)))


def test_lane_layer_golden():
    """the oracle's layer (src/cpu/lane.c's phases) and ascending-expert token sums: the reference path's bits"""
    g = np.load(os.path.join(GOLD, "golden_layer.npz"))
    ids, wts, x = g["ids"], g["wts"], g["x"]
    t3 = synth.ID["IQ3_XXS"]
    pairs = sorted(((int(ids[t, j]), t * 2 + j) for t in range(3) for j in range(2)))
    rows_x = np.stack([x[m // 2] for _, m in pairs]).astype(np.float32)
    scale = np.array([wts[m // 2, m % 2] for _, m in pairs], np.float32)
    experts = sorted(set(e for e, _ in pairs))
    row0 = np.array([min(r for r, (e, _) in enumerate(pairs) if e == ex) for ex in experts], np.uint32)
    cnt = np.array([sum(1 for e, _ in pairs if e == ex) for ex in experts], np.uint32)
    P = orc._c.c_void_p
    mats = {k: np.ascontiguousarray(g[k]) for k in ("gate", "up", "down")}  # (an npz loads afresh at each access)
    gate = (P * len(experts))(*[mats["gate"][e].ctypes.data for e in experts])
    up = (P * len(experts))(*[mats["up"][e].ctypes.data for e in experts])
    down = (P * len(experts))(*[mats["down"][e].ctypes.data for e in experts])
    ye = np.zeros((len(pairs), 512), np.float32)
    assert orc.orc().orc_lane_layer(t3, t3, 512, 256, float("inf"), orc.ptr(rows_x), orc.ptr(scale), len(pairs), gate,
                                    up, down, orc.ptr(row0), orc.ptr(cnt), len(experts), orc.ptr(ye))
    assert (bits(ye) == bits(g["ye"])).all()
    row_of = {m: r for r, (_, m) in enumerate(pairs)}
    order = np.array([sorted(row_of[t * 2 + j] for j in range(2)) for t in range(3)], np.int32).reshape(-1)
    out = np.zeros((3, 512), np.float32)
    orc.orc().orc_gather_sum_add(orc.ptr(out), orc.ptr(ye), orc.ptr(order), 2, 3, 512, None)
    assert (bits(out) == bits(g["out"])).all()


# ---- the decoders of the types the reference's CPU path does not cover: independent float64 dequantisation ----
DEQ = {"Q4_0": refdecode.q4_0, "Q8_0": refdecode.q8_0, "Q6_K": refdecode.q6_k, "Q3_K": refdecode.q3_k,
       "IQ4_NL": refdecode.iq4_nl, "IQ4_XS": refdecode.iq4_xs}
DEQ_SUB = {"Q4_K": refdecode.q4_k, "Q5_K": refdecode.q5_k, "Q2_K": refdecode.q2_k}


@pytest.mark.parametrize("name", sorted(DEQ) + sorted(DEQ_SUB) + ["BF16"])
def test_dequant_closed_form(name):
    t = synth.ID[name]
    if name == "BF16":
        raw = np.random.default_rng(1).integers(0, 2**16, 4096, dtype=np.uint16)
        raw = raw[((raw >> 7) & 0xFF) != 0xFF].view(np.uint8)  # no NaN / inf patterns
        vals = raw.size // 2 // 8 * 8
        raw = raw[:vals * 2]
        want = refdecode.bf16(raw)
    else:
        _, v, b = synth.TYPES[t]
        blocks = synth.random_blocks(t, 64, v * 2, 11).reshape(-1, b)
        raw = blocks.reshape(-1)
        vals = blocks.shape[0] * v
        if name in DEQ:
            want = DEQ[name](blocks).reshape(-1)
        else:
            a, c = DEQ_SUB[name](blocks)
            want = (a.astype(np.float32) - c.astype(np.float32)).astype(np.float64).reshape(-1)
    got = orc.dequant(t, raw, vals)
    assert (got.astype(np.float64) == want).all()


def test_mv_bound_and_split_invariance():
    """the fp32 matvec of every mv type within the reference test's bound (terms a lane + tree + 1) u sum |w x| of
    the float64 sum over exactly dequantized values, and rows computed in any split / token grouping give the same bits
    (reference tests/gpu/test_mv_gpu.hip:208-232, tests/test_cpu_expert.c:58-66)"""
    rng = np.random.default_rng(5)
    for name in ["Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "Q3_K", "Q2_K", "IQ4_NL", "IQ4_XS", "IQ3_XXS", "IQ2_XXS", "IQ1_S",
                 "IQ1_M", "IQ2_XS", "IQ2_S"]:
        t = synth.ID[name]
        rows, cols = 9, 2048
        w = synth.random_blocks(t, rows, cols, 21)
        x = rng.normal(0, 1, (5, cols)).astype(np.float32)
        y = orc.mv_rows(t, w, rows, cols, x)
        wd = orc.dequant(t, w.reshape(-1), rows * cols).reshape(rows, cols).astype(np.float64)
        exact = x.astype(np.float64) @ wd.T
        mag = np.abs(x.astype(np.float64)) @ np.abs(wd).T
        u = 2.0 ** -24
        depth = cols // 8 // 32 * 8 + 5 + 1
        assert np.all(np.abs(y - exact) <= depth * u * mag + 1e-30), name
        y1 = np.concatenate([orc.mv_rows(t, w, rows, cols, x[i:i + 1]) for i in range(5)])
        assert (bits(y1) == bits(y)).all()


# ---- the lane contract on the build-defined types (Q4_0, Q4_K, Q3_K): no reference CPU path exists ----
@pytest.mark.parametrize("name", ["Q4_0", "Q4_K", "Q3_K"])
def test_lane_build_defined_block(name):
    """each 32-value block's `sub` from exactly dequantized weights: Q4_0 one part d isum (exact in float64, rounded
    once), Q3_K two halves each rounded then added, Q4_K one part with its minimum - pinned by float64 of the dequantized
    values, which share nothing with the oracle's int8 codes"""
    t = synth.ID[name]
    rng = np.random.default_rng(9)
    cols = 512
    w = synth.random_blocks(t, 1, cols, 31)
    xq = rng.integers(-127, 128, cols).astype(np.int8)
    L = orc.orc()
    blocks = w.reshape(-1, synth.TYPES[t][2])
    for s in range(cols // 32):
        sub = np.float32(L.orc_lane_sub(t, orc.ptr(w.reshape(-1)), s, orc.ptr(xq[32 * s:32 * s + 32])))
        xs = xq[32 * s:32 * s + 32].astype(np.float64)
        if name == "Q4_0":
            wd = refdecode.q4_0(blocks)[s]
            assert sub == np.float32(np.dot(wd, xs))
        elif name == "Q3_K":
            wd = refdecode.q3_k(blocks)[(32 * s) // 256, (32 * s) % 256:(32 * s) % 256 + 32]
            p0, p1 = np.float32(np.dot(wd[:16], xs[:16])), np.float32(np.dot(wd[16:], xs[16:]))
            assert sub == np.float32(p0 + p1)
        else:
            a, c = refdecode.q4_k(blocks)
            j = (32 * s) % 256
            aa, cc = a[(32 * s) // 256, j:j + 32], c[(32 * s) // 256, j:j + 32]
            want = np.float32(np.float32(np.dot(aa, xs)) - np.float32(cc[0] * xs.sum()))
            assert sub == want


@pytest.mark.parametrize("name", ["Q4_0", "Q4_K", "Q3_K"] + LANE_TYPES)
def test_lane_rows_bound_and_invariance(name):
    """a row's lane sum within (blocks a lane + tree + 2) u sum |xd sub| of the float64 sum of the blocks' subs, and the
    same bits for rows split, tokens apart or together (the batch-invariance contract)"""
    t = synth.ID[name]
    rng = np.random.default_rng(13)
    for cols in (512, 4608):
        rows = 7
        w = synth.random_blocks(t, rows, cols, 41)
        x = rng.normal(0, 1, (6, cols)).astype(np.float32)
        q, d = orc.q8_round(x)
        y = orc.q8_rows(t, w, rows, cols, q, d)
        L = orc.orc()
        for r in range(rows):
            for tk in range(6):
                subs = np.array([L.orc_lane_sub(t, orc.ptr(w[r]), s, orc.ptr(q[tk, 32 * s:32 * s + 32]))
                                 for s in range(cols // 32)], np.float64)
                terms = d[tk].astype(np.float64) * subs
                lanes = 32 if cols >= 4096 else 16
                depth = (cols // 32) // lanes + 5 + 2
                assert abs(y[tk, r] - terms.sum()) <= depth * 2.0 ** -24 * np.abs(terms).sum() + 1e-30
        y1 = np.concatenate([orc.q8_rows(t, w, rows, cols, q[i:i + 1], d[i:i + 1]) for i in range(6)])
        assert (bits(y1) == bits(y)).all()


def test_mmq_bound_and_quantization():
    """mmq_x8_rows: |q| <= 127, dx = amax / 127, q = rint(x / dx) (a division), sx = dx sum q, an all-zero group and a
    -1 slot zeros; mmq rows within (groups + 4) u sum |terms| of float64 and slot-independent"""
    rng = np.random.default_rng(17)
    cols, rows = 1024, 16
    x = rng.normal(0, 1, (5, cols)).astype(np.float32)
    x[2, 64:96] = 0
    idx = np.array([0, 1, 2, -1, 4, 3], np.int32)
    x8, dx, sx = orc.mmq_x8_rows(x, idx, cols)
    L = orc.orc()
    for s, r in enumerate(idx):
        for g in range(cols // 32):
            at = L.orc_mmq_dx_at(s, g, cols // 32)
            qv = np.array([x8[L.orc_mmq_x8_at(s, 32 * g + i, cols)] for i in range(32)], np.int64)
            if r < 0 or (r == 2 and g == 2):
                assert dx[at] == 0 and sx[at] == 0 and (qv == 0).all()
                continue
            v = x[r, 32 * g:32 * g + 32]
            a = np.abs(v).max()
            dd = np.float32(a / np.float32(127.0))
            assert dx[at] == dd and np.abs(qv).max() <= 127
            assert (qv == np.clip(np.rint(v / dd), -127, 127)).all()
            assert sx[at] == np.float32(dd * np.float32(qv.sum()))
    w = synth.random_blocks(synth.ID["Q4_K"], rows, cols, 3)
    a, c = refdecode.q4_k(w.reshape(-1, 144))
    for s, r in enumerate(idx):
        y = orc.mmq_rows(w, rows, cols, x8, dx, sx, s)
        qx = np.array([x8[L.orc_mmq_x8_at(s, i, cols)] for i in range(cols)], np.float64)
        dxs = np.repeat([dx[L.orc_mmq_dx_at(s, g, cols // 32)] for g in range(cols // 32)], 32).astype(np.float64)
        wa = a.reshape(rows, cols)
        wc = c.reshape(rows, cols)
        terms = (wa * qx * dxs) - (wc * qx * dxs)
        exact = terms.sum(axis=1)
        assert np.all(np.abs(y - exact) <= (cols // 32 + 8) * 2.0 ** -23 * np.abs(terms).sum(axis=1) + 1e-30)


# ---- the mmq contract's order, bit for bit, from exactly rounded float32 operations ----

def b32(v):
    return int(np.float32(v).view(np.uint32))


def _mmq_exact(blocks, x8s, dxs, sxs, variant=""):
    """one Q4_K row (blocks [nb, 144]) against one slot's codes x8s [cols], scales dxs / sxs [groups], in the order
    reference include/osmos/gpu/mmq.h:37-55 and tests/gpu/test_mmq_gpu.hip:94-115 state: partition p takes blocks
    p, p + 4, ...; per group v = (d sc) dx, acc = fma(v, I, acc), acc = fma(dmin m, -sx, acc); then
    ((p0 + p1) + p2) + p3. Every float step is a correctly rounded binary32 operation (tests/exact32.py).
    variant: "muladd" (a product then a sum in place of each fma), "reverse" (the partitions summed 3 .. 0) or
    "serial" (one chain over all blocks): orders the contract rules out, used to show the test can see them."""
    import exact32 as e
    nb = blocks.shape[0]
    d, dmin = refdecode._h(blocks, 0), refdecode._h(blocks, 2)
    sc, mn = refdecode._k_scales(blocks[:, 4:16].astype(np.int64))
    parts = [np.float32(0.0)] * 4
    order = [(p, b) for p in range(4) for b in range(p, nb, 4)] if variant != "serial" else [(0, b) for b in range(nb)]
    for p, b in order:
        for g in range(8):
            q = ((blocks[b, 16 + 32 * (g // 2):16 + 32 * (g // 2) + 32].astype(np.int64) >> (4 * (g % 2))) & 15)
            gg = 8 * b + g
            isum = int((q * x8s[32 * gg:32 * gg + 32].astype(np.int64)).sum())
            dsc = e.mul(np.float32(d[b]), np.float32(sc[b, g]))
            dm = e.mul(np.float32(dmin[b]), np.float32(mn[b, g]))
            v = e.mul(dsc, dxs[gg])
            if variant == "muladd":
                parts[p] = e.add(e.mul(v, np.float32(isum)), parts[p])
                parts[p] = e.add(e.mul(dm, -sxs[gg]), parts[p])
            else:
                parts[p] = e.fma(v, np.float32(isum), parts[p])
                parts[p] = e.fma(dm, -sxs[gg], parts[p])
    seq = [3, 2, 1, 0] if variant == "reverse" else [0, 1, 2, 3]
    r = parts[seq[0]]
    for p in seq[1:]:
        r = e.add(r, parts[p])
    return r


@pytest.mark.parametrize("cols", [1024, 2048])
def test_mmq_rows_exact_order(cols):
    """orc_mmq_rows equals, bit for bit, the contract's operations replayed in exactly rounded binary32; a product and a
    sum in place of an fma, the partitions summed in reverse, or one serial chain each change some row's bits on the
    same inputs (so the check sees those mistakes)"""
    rng = np.random.default_rng(23 + cols)
    rows = 12
    w = synth.random_blocks(synth.ID["Q4_K"], rows, cols, 5 + cols)
    x = rng.normal(0, 1, (3, cols)).astype(np.float32)
    idx = np.array([2, 0, 1], np.int32)
    x8, dx, sx = orc.mmq_x8_rows(x, idx, cols)
    L = orc.orc()
    blocks = w.reshape(rows, cols // 256, 144)
    differs = {"muladd": 0, "reverse": 0, "serial": 0}
    for s in range(len(idx)):
        y = orc.mmq_rows(w, rows, cols, x8, dx, sx, s)
        x8s = np.array([x8[L.orc_mmq_x8_at(s, i, cols)] for i in range(cols)], np.int8)
        at = [L.orc_mmq_dx_at(s, g, cols // 32) for g in range(cols // 32)]
        dxs, sxs = dx[at], sx[at]
        for r in range(rows):
            want = _mmq_exact(blocks[r], x8s, dxs, sxs)
            assert b32(y[r]) == b32(want), (s, r, y[r], want)
            for v in differs:
                differs[v] += int(b32(_mmq_exact(blocks[r], x8s, dxs, sxs, v)) != b32(want))
    assert all(n > 0 for n in differs.values()), differs


def test_mmq_rows_one_block_closed_form():
    """a row whose only nonzero block is block p (of 4: partition p alone, one block) over one group: the result is
    fma(dmin m, -sx, fma((d sc) dx, I, 0)) exactly, whichever partition holds it"""
    import exact32 as e
    cols = 1024
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (1, cols)).astype(np.float32)
    x8, dx, sx = orc.mmq_x8_rows(x, np.array([0], np.int32), cols)
    L = orc.orc()
    for p in range(4):
        blk = np.zeros((4, 144), np.uint8)
        blk[p, 0:2] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
        blk[p, 2:4] = np.frombuffer(np.float16(0.0071).tobytes(), np.uint8)
        blk[p, 4] = 37  # group 0: sc 37, m 21
        blk[p, 8] = 21
        blk[p, 16:48] = rng.integers(0, 16, 32)
        y = orc.mmq_rows(blk.reshape(-1), 1, cols, x8, dx, sx, 0)
        gg = 8 * p
        at = L.orc_mmq_dx_at(0, gg, cols // 32)
        q = blk[p, 16:48].astype(np.int64) & 15
        xs = np.array([x8[L.orc_mmq_x8_at(0, 32 * gg + i, cols)] for i in range(32)], np.int64)
        dsc = e.mul(np.float16(0.0123).astype(np.float32), np.float32(37))
        dm = e.mul(np.float16(0.0071).astype(np.float32), np.float32(21))
        want = e.fma(dm, -sx[at], e.fma(e.mul(dsc, dx[at]), np.float32((q * xs).sum()), np.float32(0)))
        assert b32(y[0]) == b32(want), p


# ---- the MoE plumbing against float64 ----

def _route64(logits, k):
    """float64 softmax, the k most probable (the greater first, the lower id among equals), weights p / max(sum, floor)
    (reference include/osmos/gpu/q4x_ops.h:356-360)"""
    l = logits.astype(np.float64)
    p = np.exp(l - l.max())
    p /= p.sum()
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))[:k]
    pk = p[order]
    return np.array(order), pk / max(pk.sum(), 6.103515625e-5)


def test_route_float64():
    """orc_route's ids are float64's top-k (ties: the lower id, also among exactly equal logits), its weights within a
    few ulp of float64's; well-separated logits so float32 rounding cannot reorder the picks"""
    rng = np.random.default_rng(31)
    for n_tok, n_exp, k in [(5, 512, 10), (4, 256, 8), (3, 64, 1), (2, 1024, 32)]:
        base = rng.permutation(n_exp).astype(np.float32) * np.float32(0.01)  # distinct, 0.01 apart
        logits = np.stack([np.roll(base, 7 * t) for t in range(n_tok)]).astype(np.float32)
        logits[0, 3] = logits[0, 9] = logits[0].max()  # an exact tie at the top: 3 first, then 9
        ids = np.zeros((n_tok, k), np.int32)
        w = np.zeros((n_tok, k), np.float32)
        orc.orc().orc_route(orc.ptr(logits), n_tok, n_exp, k, orc.ptr(ids), orc.ptr(w))
        for t in range(n_tok):
            i64, w64 = _route64(logits[t], k)
            assert (ids[t] == i64).all(), (n_tok, n_exp, k, t)
            assert np.all(np.abs(w[t] - w64) <= 8 * 2.0 ** -24 * w64), (n_tok, n_exp, k, t)
        if k > 1:
            assert ids[0, 0] == 3 and ids[0, 1] == 9 and w[0, 0] == w[0, 1]


def test_route_sum_floor():
    """the weights' divisor is max(sum of the k probabilities, 6.103515625e-5): with 20000 equal logits and k = 1 the
    sum is 5e-5, under the floor, so w = (1/20000) / 6.103515625e-5 = 0.8192 - and k = 2 (1e-4, over it) gives 0.5"""
    n = 20000
    logits = np.zeros((1, n), np.float32)
    for k, want in [(1, 0.8192), (2, 0.5)]:
        ids = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        orc.orc().orc_route(orc.ptr(logits), 1, n, k, orc.ptr(ids), orc.ptr(w))
        assert list(ids) == list(range(k))
        assert abs(float(w[0]) - want) <= 1e-6 * want, (k, w)


def test_moe_sum_float64():
    """orc_moe_sum: out[t] = sum over j in order of y[where[t k + j]] w[t k + j], plus shared[t] sigmoid(logit[t]):
    exact where every term is (small integers, power-of-two weights; logit 0 gives 1/2, a large logit 1 and a very
    negative one 0); within (k + 2) ulp-sums of float64 on random inputs"""
    rng = np.random.default_rng(41)
    n_tok, k, dim, n_rows = 4, 3, 64, 9
    y = rng.integers(-50, 50, (n_rows, dim)).astype(np.float32)
    where = rng.permutation(n_tok * k).astype(np.int32) % n_rows
    w = np.float32(2.0) ** rng.integers(-3, 3, n_tok * k).astype(np.float32)
    sh = rng.integers(-50, 50, (n_tok, dim)).astype(np.float32)
    sl = np.array([0.0, 100.0, -200.0, 0.0], np.float32)
    out = np.zeros((n_tok, dim), np.float32)
    orc.orc().orc_moe_sum(orc.ptr(y), orc.ptr(where), orc.ptr(w), n_tok, k, dim, orc.ptr(sh), orc.ptr(sl), orc.ptr(out))
    gate = np.array([0.5, 1.0, 0.0, 0.5])
    want = np.stack([sum(y[where[t * k + j]].astype(np.float64) * w[t * k + j] for j in range(k)) + sh[t] * gate[t]
                     for t in range(n_tok)])
    assert (out == want).all()
    # random: the float32 sum against float64
    y = rng.normal(0, 1, (n_rows, dim)).astype(np.float32)
    w = rng.uniform(0, 1, n_tok * k).astype(np.float32)
    sl = rng.normal(0, 2, n_tok).astype(np.float32)
    orc.orc().orc_moe_sum(orc.ptr(y), orc.ptr(where), orc.ptr(w), n_tok, k, dim, orc.ptr(sh), orc.ptr(sl), orc.ptr(out))
    for t in range(n_tok):
        g64 = 1.0 / (1.0 + np.exp(-np.float64(sl[t])))
        terms = [y[where[t * k + j]].astype(np.float64) * w[t * k + j] for j in range(k)] + [sh[t] * g64]
        exact = sum(terms)
        mag = sum(np.abs(a) for a in terms)
        assert np.all(np.abs(out[t] - exact) <= (k + 4) * 2.0 ** -24 * mag + 1e-30), t


# ---- the f16 matmul's K order (orc_mm_rows) ----

MM_ORDER_CASES = [("Q8_0", 2048, False), ("Q8_0", 320, False), ("Q4_K", 2048, False), ("Q5_K", 512, False),
                  ("Q6_K", 1536, False), ("Q6_K", 1536, True), ("Q6_K", 2048, False), ("Q4_0", 512, False),
                  ("IQ4_NL", 512, False), ("Q2_K", 1024, False), ("Q3_K", 1024, False), ("IQ2_XXS", 1024, False),
                  ("IQ2_XS", 1024, True), ("IQ1_S", 1024, False), ("IQ3_XXS", 2048, True), ("IQ4_XS", 512, False)]


@pytest.mark.parametrize("name,cols,group", MM_ORDER_CASES)
def test_mm_rows_partition_order(name, cols, group):
    """orc_mm_rows follows the reference's K split for the type and width (kernels/mm.hip:24-73): partition 0's two
    nearly cancelling products and partition 1's small one give the value worked out by hand from the contract's
    order (partitions first, then their sum in order), not the single K chain's (tests/mmorder.py)"""
    from tests import mmorder
    w, x, ordered, chain = mmorder.case(name, cols, group, 7)
    y = orc.mm_rows(synth.ID[name], w, 16, cols, x, group)
    assert (bits(y) == bits(np.repeat(ordered[:, None], 16, axis=1))).all()
    assert (ordered != chain).all()


def test_mm_rows_bound():
    """on random weights and activations orc_mm_rows is within the reference's bound, (cols/16 + 20) u sum |w x|, of
    the double sum over the f16-rounded values (tests/gpu/test_mm_gpu.hip:321-341)"""
    rng = np.random.default_rng(3)
    for name, cols in (("Q4_K", 1024), ("IQ2_XXS", 2048), ("Q8_0", 320)):
        t = synth.ID[name]
        w = synth.random_blocks(t, 8, cols, 5)
        x = rng.normal(0, 1, (5, cols)).astype(np.float32)
        y = orc.mm_rows(t, w, 8, cols, x)
        wf = orc.dequant(t, w, 8 * cols).reshape(8, cols).astype(np.float16).astype(np.float64)
        xf = x.astype(np.float16).astype(np.float64)
        err = np.abs(y - xf @ wf.T)
        assert (err <= (cols / 16 + 20) * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T)).all(), name
