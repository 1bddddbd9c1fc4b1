"""Parity at the workloads' own shapes (the benchmark configurations), on the MI355X through the C ABI, against the
pinned oracle:

- config 1: Q4_0, 2048 -> 8192 (weights quantized from N(0, 0.02), seed 0), one token: q8_group_tok (the lane's int8
  activations) and mv_run (fp32 activations), every row;
- config 2: Q4_K and Q3_K, 2048 -> 6144 from N(0, 0.02): mv_strided at 1 / 8 / 64 tokens (oracle rows at both ends
  of the matrix), the lane at 1 and 8 tokens (every row), mm_run at 8 and 64 tokens within the reference's f16 bound;
- config 3: the Qwen-style layer at its full expert count (512 experts, hidden 2048, expert ff 512, top-10, IQ3_XXS)
  at batches 1, 4 and 32;
- config 4: the DeepSeek-style layer at its full expert count (256 routed + the shared one, hidden 7168, expert ff
  2048, top-9) in IQ1_S, IQ1_M and IQ2_XXS at batches 1 and 4;
- config 5: the benchmark's own routing (512 tokens top-8 of 256 experts, Zipf 1.1, seed 11): mmq_group over Q4_K
  2048 -> 7168, and osmos_lane_group and mm_group (f16, the kernel form the benchmark times) over IQ2_XXS
  7168 -> 2048, every expert launched; the busiest expert (all of its
  tokens) and two small ones checked on 64-row subsets, and tokens of the busiest expert run alone for batch
  invariance.
(reference checks of the same kind: tests/gpu/test_q8_gpu.hip:232-244, tests/gpu/test_mmq_gpu.hip:207-233,
tests/gpu/test_mv_gpu.hip:208-232)"""
import math

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


def _cfg1_weights():
    return synth.quant_q4_0(synth.normal((8192, 2048), 0, 0.02))


def _lane_tok(g, t, w, rows, cols, q, d):
    import torch
    n = q.shape[0]
    y = torch.full((n, rows), float("nan"), device="cuda")
    g.call("q8_group_tok", t, g.a(g.table([g.dev(w)])), g.a(g.dev(np.array([n], np.int32))),
           g.a(g.dev(np.array([0], np.int32))), None, 1, n, rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(y), rows,
           None)
    return g.host(y)


def _mv(g, t, w, rows, cols, x):
    import torch
    n = x.shape[0]
    y = torch.full((n, rows), float("nan"), device="cuda")
    g.call("mv_strided", t, g.a(g.dev(w)), rows, cols, g.a(g.dev(x)), cols, n, g.a(y), rows, None)
    return g.host(y)


def test_config1_q4_0_lane_and_mv(g):
    rows, cols = 8192, 2048
    t = synth.ID["Q4_0"]
    w = _cfg1_weights()
    x = synth.normal((1, cols), 1)
    q, d = orc.q8_round(x)
    print("config 1 lane", flush=True)
    y = _lane_tok(g, t, w, rows, cols, q, d)
    assert (g.bits(y) == g.bits(orc.q8_rows(t, w, rows, cols, q, d))).all()
    print("config 1 mv", flush=True)
    y = _mv(g, t, w, rows, cols, x)
    assert (g.bits(y) == g.bits(orc.mv_rows(t, w, rows, cols, x))).all()


def _oracle_mv_ends(t, w, rows, cols, x, span):
    """orc_mv_rows on rows [0, span) and [rows - span, rows)"""
    n = x.shape[0]
    y = np.zeros((n, rows), np.float32)
    for r0 in (0, rows - span):
        assert orc.orc().orc_mv_rows(t, orc.ptr(w), cols, r0, r0 + span, orc.ptr(x), cols, n, orc.ptr(y), rows)
    return y


@pytest.mark.parametrize("name", ["Q4_K", "Q3_K"])
def test_config2_mv_and_lane(g, name):
    rows, cols = 6144, 2048
    t = synth.ID[name]
    w = (synth.quant_q4_k if name == "Q4_K" else synth.quant_q3_k)(synth.normal((rows, cols), 2, 0.02))
    x = synth.normal((64, cols), 3)
    for n in (1, 8, 64):
        print("config 2 mv", name, n, flush=True)
        y = _mv(g, t, w, rows, cols, x[:n])
        span = rows if n == 1 else 384
        want = _oracle_mv_ends(t, w, rows, cols, x[:n], span)
        for r0 in (0, rows - span):
            assert (g.bits(y[:, r0:r0 + span]) == g.bits(want[:, r0:r0 + span])).all(), (name, n, r0)
        assert np.isfinite(y).all()
    for n in (1, 8):
        print("config 2 lane", name, n, flush=True)
        q, d = orc.q8_round(x[:n])
        y = _lane_tok(g, t, w, rows, cols, q, d)
        assert (g.bits(y) == g.bits(orc.q8_rows(t, w, rows, cols, q, d))).all(), (name, n)


@pytest.mark.parametrize("name", ["Q4_K", "Q3_K"])
def test_config2_mm_bound(g, name):
    """mm_run at 8 and 64 tokens, 2048 -> 6144: within the reference's bound on a 512-row slice, batch-invariant
    (8 tokens' bits are the first 8 of the 64)"""
    import torch
    from tests.test_mm_gpu import bound_check, mm_x16
    rows, cols = 6144, 2048
    t = synth.ID[name]
    w = (synth.quant_q4_k if name == "Q4_K" else synth.quant_q3_k)(synth.normal((rows, cols), 2, 0.02))
    x = synth.normal((64, cols), 3)
    ys = {}
    for n in (8, 64):
        print("config 2 mm", name, n, flush=True)
        x16, _ = mm_x16(g, x[:n])
        y = torch.full((n, rows), float("nan"), device="cuda")
        g.call("mm_run", t, g.a(g.dev(w)), rows, cols, g.a(x16), n, g.a(y), rows, None)
        ys[n] = g.host(y)
        sl = slice(rows - 512, rows)
        bound_check(name, np.ascontiguousarray(w[sl]), 512, cols, x[:n], ys[n][:, sl])
    assert (g.bits(ys[8]) == g.bits(ys[64][:8])).all()


@pytest.mark.parametrize("n_tok", [1, 4, 32])
def test_config3_qwen_layer_512_experts(g, n_tok):
    """the Qwen-style layer at full size: 512 experts (each its own weights), hidden 2048, ff 512, top-10, IQ3_XXS"""
    import torch
    from libosmos_amd.layer import LaneLayer
    from tests.test_moe_gpu import _lane_layer_oracle
    t3 = synth.ID["IQ3_XXS"]
    n_exp, k, dim, ff = 512, 10, 2048, 512
    G = synth.iq_blocks(t3, n_exp * ff, dim, 71).reshape(n_exp, ff, -1)
    Up = synth.iq_blocks(t3, n_exp * ff, dim, 72).reshape(n_exp, ff, -1)
    Dn = synth.iq_blocks(t3, n_exp * dim, ff, 73).reshape(n_exp, dim, -1)
    rng = np.random.default_rng(74 + n_tok)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    logits = rng.normal(0, 1, (n_tok, n_exp)).astype(np.float32)
    ids = np.zeros((n_tok, k), np.int32)
    wts = np.zeros((n_tok, k), np.float32)
    orc.orc().orc_route(orc.ptr(logits), n_tok, n_exp, k, orc.ptr(ids), orc.ptr(wts))
    want = _lane_layer_oracle(t3, x, ids, wts, G, Up, Dn, dim, ff, math.inf)
    L = LaneLayer(t3, t3, dim, ff, n_exp, k, g.dev(G).reshape(n_exp, -1), g.dev(Up).reshape(n_exp, -1),
                  g.dev(Dn).reshape(n_exp, -1))
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("config 3 layer, 512 experts", n_tok, flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()


def _device_blocks(g, name, n, seed):
    """n blocks of `name` as random bytes made on the device, each scale an f16 in [2^-4, 2^-3) (synth's fill):
    returns uint8 [n, block bytes]"""
    import torch
    _, _, b = synth.TYPES[synth.ID[name]]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    blk = torch.randint(0, 256, (n, b), dtype=torch.uint8, device="cuda", generator=gen)
    h = 0x2C00 | torch.randint(0, 1024, (n,), dtype=torch.int32, device="cuda", generator=gen)
    if name == "IQ1_M":  # the f16's nibble k in the top nibble of scale word k
        for k in range(4):
            at = 48 + 2 * k + 1
            blk[:, at] = (blk[:, at] & 0x0F) | (((h >> (4 * k)) & 0x0F) << 4).to(torch.uint8)
    else:
        blk[:, 0] = (h & 0xFF).to(torch.uint8)
        blk[:, 1] = ((h >> 8) & 0xFF).to(torch.uint8)
    return blk


@pytest.mark.parametrize("name", ["IQ1_S", "IQ1_M", "IQ2_XXS"])
@pytest.mark.parametrize("n_tok", [1, 4])
def test_config4_deepseek_layer_257_experts(g, name, n_tok):
    """the DeepSeek-style layer at its full expert count: 256 routed experts plus the shared one as a ninth pick
    (257 matrices of each kind, hidden 7168, expert ff 2048), IQ1_S and IQ1_M, and IQ2_XXS for comparison, batches 1
    and 4 (the draft/verify batch): the oracle's bits. (weights made on the device; the routed experts' copied back for the oracle)"""
    import torch
    from libosmos_amd.layer import LaneLayer
    from tests.test_moe_gpu import _lane_layer_oracle
    t = synth.ID[name]
    n_exp, k, dim, ff = 257, 9, 7168, 2048
    per = dim // 256 * ff  # blocks a matrix (gate / up: ff rows of dim; down: dim rows of ff)
    mats = [_device_blocks(g, name, n_exp * per, 400 + 10 * n_tok + i).reshape(n_exp, -1) for i in range(3)]
    rng = np.random.default_rng(90 + n_tok)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids = np.stack([np.concatenate([rng.choice(n_exp - 1, k - 1, replace=False), [n_exp - 1]]) for _ in range(n_tok)])
    ids = ids.astype(np.int32)
    wts = rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32)
    used = sorted(set(ids.reshape(-1).tolist()))
    host = [{e: g.host(m[e]).reshape(dim if i == 2 else ff, -1) for e in used} for i, m in enumerate(mats)]
    want = _lane_layer_oracle(t, x, ids, wts, host[0], host[1], host[2], dim, ff, math.inf)
    L = LaneLayer(t, t, dim, ff, n_exp, k, *mats)
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    print("config 4 layer, 257 experts", name, n_tok, flush=True)
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()


def _cfg5_routing():
    """the benchmark's config-5 routing (bench.py prefill_extras): 512 tokens, top-8 of 256, Zipf(1.1), seed 11"""
    n_tok, n_exp, k = 512, 256, 8
    rng = np.random.default_rng(11)
    p = 1.0 / np.arange(1, n_exp + 1) ** 1.1
    p /= p.sum()
    ids = np.stack([rng.choice(n_exp, k, replace=False, p=p) for _ in range(n_tok)])
    pairs = [[] for _ in range(n_exp)]
    for t in range(n_tok):
        for e in ids[t]:
            pairs[e].append(t)
    return pairs


N_MATS = 6  # distinct weight matrices, expert e reads matrix e % N_MATS (the kernels see 256 table entries)


def _checked_experts(pairs):
    cnt = np.array([len(p) for p in pairs])
    busiest = int(cnt.argmax())
    small = [int(e) for e in np.argsort(cnt, kind="stable") if cnt[e] > 0][:2]
    return busiest, small


def test_config5_mmq_group(g):
    import torch
    pairs = _cfg5_routing()
    n_exp, n_tok, rows, cols = 256, 512, 7168, 2048
    t = synth.ID["Q4_K"]
    cnt = np.array([len(p) for p in pairs], np.int32)
    assert cnt.max() == 441
    mats = [synth.quant_q4_k(synth.normal((rows, cols), 500 + m, 0.02)) for m in range(N_MATS)]
    dm = [g.dev(m) for m in mats]
    idx, soff = [], np.zeros(n_exp, np.uint32)
    for e in range(n_exp):
        soff[e] = len(idx)
        idx += pairs[e] + [-1] * ((-len(pairs[e])) % 16)
    slots = len(idx)
    x = synth.normal((n_tok, cols), 13)
    x8 = torch.zeros(slots * cols, dtype=torch.int8, device="cuda")
    dx = torch.zeros(slots * cols // 32, device="cuda")
    sx = torch.zeros(slots * cols // 32, device="cuda")
    g.call("mmq_x8_rows", g.a(g.dev(x)), cols, g.a(g.dev(np.array(idx, np.int32))), slots, cols, g.a(x8), g.a(dx),
           g.a(sx), None)
    o8, odx, osx = orc.mmq_x8_rows(x, np.array(idx, np.int32), cols)
    assert (g.host(x8) == o8).all()
    yoff = (soff.astype(np.int64) * rows).astype(np.uint32)
    y = torch.full((slots * rows,), float("nan"), device="cuda")
    print("config 5 mmq_group", flush=True)
    g.call("mmq_group", t, g.a(g.table([dm[e % N_MATS] for e in range(n_exp)])), g.a(g.dev(cnt)), n_exp,
           int(cnt.max()), rows, cols, g.a(x8), g.a(dx), g.a(sx), g.a(g.dev(soff)), g.a(y), g.a(g.dev(yoff)), rows,
           None)
    yh = g.host(y).reshape(slots, rows)
    live = np.array([i >= 0 for i in idx])
    assert np.isfinite(yh[live]).all() and np.isnan(yh[~live]).all()
    busiest, small = _checked_experts(pairs)
    r0, r1 = 3520, 3584  # a 64-row subset in the middle of the matrix
    for e in [busiest] + small:
        w = mats[e % N_MATS]
        for j in range(len(pairs[e])):
            s = int(soff[e]) + j
            want = np.zeros(rows, np.float32)
            assert orc.orc().orc_mmq_rows(orc.ptr(w), cols, r0, r1, orc.ptr(o8), orc.ptr(odx), orc.ptr(osx), s,
                                          orc.ptr(want))
            assert (g.bits(yh[s, r0:r1]) == g.bits(want[r0:r1])).all(), (e, j)
    # batch invariance: three of the busiest expert's tokens alone (a one-token launch of the same matrix)
    for j in (0, 200, 440):
        s = int(soff[busiest]) + j
        tok = pairs[busiest][j]
        a8 = torch.zeros(16 * cols, dtype=torch.int8, device="cuda")
        adx = torch.zeros(16 * cols // 32, device="cuda")
        asx = torch.zeros(16 * cols // 32, device="cuda")
        g.call("mmq_x8_rows", g.a(g.dev(x)), cols, g.a(g.dev(np.array([tok], np.int32))), 1, cols, g.a(a8), g.a(adx),
               g.a(asx), None)
        y1 = torch.full((rows,), float("nan"), device="cuda")
        g.call("mmq_group", t, g.a(g.table([dm[busiest % N_MATS]])), g.a(g.dev(np.array([1], np.int32))), 1, 1, rows,
               cols, g.a(a8), g.a(adx), g.a(asx), g.a(g.dev(np.zeros(1, np.uint32))), g.a(y1),
               g.a(g.dev(np.zeros(1, np.uint32))), rows, None)
        assert (g.bits(g.host(y1)) == g.bits(yh[s])).all(), j


def test_config5_lane_group(g):
    import torch
    pairs = _cfg5_routing()
    n_exp, n_tok, rows, cols = 256, 512, 2048, 7168
    t = synth.ID["IQ2_XXS"]
    cnt = np.array([len(p) for p in pairs], np.int32)
    mats = [synth.iq_blocks(t, rows, cols, 600 + m) for m in range(N_MATS)]
    dm = [g.dev(m) for m in mats]
    order = [tok for e in range(n_exp) for tok in pairs[e]]
    xrow = np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.int32)
    x = synth.normal((n_tok, cols), 14)
    q, d = orc.q8_round(x[order])
    n = len(order)
    y = torch.full((n + 1, rows), float("nan"), device="cuda")
    print("config 5 osmos_lane_group", flush=True)
    g.call("osmos_lane_group", t, g.a(g.table([dm[e % N_MATS] for e in range(n_exp)])), g.a(g.dev(cnt)),
           g.a(g.dev(xrow)), n_exp, int(cnt.max()), rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(y), rows, None)
    yh = g.host(y)
    assert np.isfinite(yh[:n]).all() and np.isnan(yh[n]).all()
    busiest, small = _checked_experts(pairs)
    r0, r1 = 1000, 1064
    for e in [busiest] + small:
        a, c = int(xrow[e]), int(cnt[e])
        want = np.zeros((c, rows), np.float32)
        assert orc.orc().orc_q8_rows(t, orc.ptr(mats[e % N_MATS]), cols, r0, r1, orc.ptr(q[a:a + c]),
                                     orc.ptr(d[a:a + c]), c, orc.ptr(want), rows)
        assert (g.bits(yh[a:a + c, r0:r1]) == g.bits(want[:, r0:r1])).all(), e
    # batch invariance: tokens of the busiest expert alone
    a = int(xrow[busiest])
    for j in (0, 100, 440):
        y1 = torch.full((1, rows), float("nan"), device="cuda")
        g.call("osmos_lane_group", t, g.a(g.table([dm[busiest % N_MATS]])), g.a(g.dev(np.array([1], np.int32))),
               g.a(g.dev(np.zeros(1, np.int32))), 1, 1, rows, cols, g.a(g.dev(q[a + j:a + j + 1])),
               g.a(g.dev(d[a + j:a + j + 1])), g.a(y1), rows, None)
        assert (g.bits(g.host(y1)[0]) == g.bits(yh[a + j])).all(), j


def test_config5_mm_group_iq2xxs(g):
    """mm_group at the benchmark's config-5 gate: IQ2_XXS 7168 -> 2048, 256 table entries at the Zipf routing (the
    441-token busiest expert, so the tall row-tile form the benchmark times), within the reference's f16 bound on a
    64-row subset for the busiest expert and two small ones, and three tokens of the busiest expert alone the same
    bits (reference tests/gpu/test_mm_gpu.hip:321-341)"""
    import torch
    from tests.test_mm_gpu import bound_check
    pairs = _cfg5_routing()
    n_exp, n_tok, rows, cols = 256, 512, 2048, 7168
    name = "IQ2_XXS"
    t = synth.ID[name]
    cnt = np.array([len(p) for p in pairs], np.int32)
    mats = [synth.iq_blocks(t, rows, cols, 700 + m) for m in range(N_MATS)]
    dm = [g.dev(m) for m in mats]
    idx, soff = [], np.zeros(n_exp, np.uint32)
    for e in range(n_exp):
        soff[e] = len(idx)
        idx += pairs[e] + [-1] * ((-len(pairs[e])) % 16)
    slots = len(idx)
    x = synth.normal((n_tok, cols), 15)
    xd = g.dev(x)
    x16 = torch.zeros(slots * cols, dtype=torch.float16, device="cuda")
    g.call("mm_x16_rows", g.a(xd), cols, g.a(g.dev(np.array(idx, np.int32))), slots, cols, g.a(x16), None, None)
    xoff = (soff.astype(np.int64) * cols).astype(np.uint32)
    yoff = (soff.astype(np.int64) * rows).astype(np.uint32)
    y = torch.full((slots * rows,), float("nan"), device="cuda")
    print("config 5 mm_group IQ2_XXS", flush=True)
    g.call("mm_group", t, g.a(g.table([dm[e % N_MATS] for e in range(n_exp)])), g.a(g.dev(cnt)), n_exp,
           int(cnt.max()), rows, cols, g.a(x16), g.a(g.dev(xoff)), cols, g.a(y), g.a(g.dev(yoff)), rows, None)
    yh = g.host(y).reshape(slots, rows)
    live = np.array([i >= 0 for i in idx])
    assert np.isfinite(yh[live]).all()
    busiest, small = _checked_experts(pairs)
    assert len(pairs[busiest]) == 441
    r0, r1 = 1000, 1064
    for e in [busiest] + small:
        a, c = int(soff[e]), len(pairs[e])
        bound_check(name, np.ascontiguousarray(mats[e % N_MATS][r0:r1]), r1 - r0, cols, x[pairs[e]],
                    yh[a:a + c, r0:r1])
    for j in (0, 200, 440):
        tok = pairs[busiest][j]
        x1 = torch.zeros(16 * cols, dtype=torch.float16, device="cuda")
        g.call("mm_x16_rows", g.a(xd), cols, g.a(g.dev(np.array([tok], np.int32))), 1, cols, g.a(x1), None, None)
        y1 = torch.full((rows,), float("nan"), device="cuda")
        z = g.dev(np.zeros(1, np.uint32))
        g.call("mm_group", t, g.a(g.table([dm[busiest % N_MATS]])), g.a(g.dev(np.array([1], np.int32))), 1, 1, rows,
               cols, g.a(x1), g.a(z), cols, g.a(y1), g.a(z), rows, None)
        assert (g.bits(g.host(y1)) == g.bits(yh[int(soff[busiest]) + j])).all(), j
