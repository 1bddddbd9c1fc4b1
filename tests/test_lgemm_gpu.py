"""The lane contract at prefill scale on the int8 matrix cores (osmos_lane_group): every output row the reference CPU
lane's bits (the pinned oracle, orc_q8_rows = the reference's cpu_q8_rows on the golden vectors) at 1 .. 70 tokens a
matrix, 16 and 32 logical lanes, ragged counts, a token's bits its own (alone = in the batch), and the same bits as
the drop-in q8_group_tok where both apply. (reference: tests/test_cpu_q8.c:139-209, tests/gpu/test_q8_gpu.hip:232-244)
"""
import numpy as np
import pytest

from libosmos_amd import synth
from oracle import orc

pytestmark = pytest.mark.gpu

LG_TYPES = ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ1_S", "IQ1_M"]


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


def run(g, t, ws, counts, rows, cols, q, d):
    import torch
    xrow = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    n = int(np.sum(counts))
    y = torch.full((n + 1, rows), float("nan"), device="cuda")
    g.call("osmos_lane_group", t, g.a(g.table([g.dev(w) for w in ws])), g.a(g.dev(np.array(counts, np.int32))),
           g.a(g.dev(xrow)), len(ws), max(counts), rows, cols, g.a(g.dev(q)), g.a(g.dev(d)), g.a(y), rows, None)
    return g.host(y), xrow


@pytest.mark.parametrize("cols", [512, 768, 4096, 4352])  # (768, 4352: a short last round of blocks)
@pytest.mark.parametrize("name", LG_TYPES)
def test_lane_group_oracle(g, name, cols):
    t = synth.ID[name]
    rows = 80  # a workgroup's 64 rows and a partial one
    counts = [1, 17, 40, 5, 29]  # (last passes of 1, 1, 8, 5 tokens: the 8-token layout; 29: 16 + 13)
    ws = [synth.iq_blocks(t, rows, cols, 70 + m) for m in range(len(counts))]
    rng = np.random.default_rng(cols + t)
    x = rng.normal(0, 1, (int(np.sum(counts)), cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    print("lane_group", name, cols, flush=True)
    y, xrow = run(g, t, ws, counts, rows, cols, q, d)
    for m, c in enumerate(counts):
        want = orc.q8_rows(t, ws[m], rows, cols, q[xrow[m]:xrow[m] + c], d[xrow[m]:xrow[m] + c])
        assert (g.bits(y[xrow[m]:xrow[m] + c]) == g.bits(want)).all(), (name, cols, m)
    assert np.isnan(y[-1]).all()  # nothing written past the rows


def test_lane_group_invariance_and_drop_in(g):
    """one matrix at 70 tokens (9 groups of 8 over 5 passes, the last group of 6) against the same tokens one at a time,
    and q8_group_tok's bits at 8 tokens"""
    import torch
    name, rows, cols = "IQ2_XXS", 64, 2048
    t = synth.ID[name]
    w = synth.iq_blocks(t, rows, cols, 5)
    x = np.random.default_rng(9).normal(0, 1, (70, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    y, _ = run(g, t, [w], [70], rows, cols, q, d)
    for k in (0, 33, 69):
        one, _ = run(g, t, [w], [1], rows, cols, q[k:k + 1], d[k:k + 1])
        assert (g.bits(one[0]) == g.bits(y[k])).all()
    y8 = torch.full((8, rows), float("nan"), device="cuda")
    g.call("q8_group_tok", t, g.a(g.table([g.dev(w)])), g.a(g.dev(np.array([8], np.int32))),
           g.a(g.dev(np.array([0], np.int32))), None, 1, 8, rows, cols, g.a(g.dev(q[:8])), g.a(g.dev(d[:8])), g.a(y8),
           rows, None)
    assert (g.bits(g.host(y8)) == g.bits(y[:8])).all()


@pytest.mark.parametrize("cols", [512, 4096])
def test_lane_group_nonfinite_scale(g, cols):
    """a block whose f16 scale is +inf (no quantizer writes one): the rows of finite blocks keep the oracle's bits; a
    row holding the inf block is NaN for every token (the integer dots come out of the MFMA biased, and the bias's
    correction is inf - inf there), where the contract's own sums are +-inf or NaN"""
    name, rows = "IQ2_XXS", 32
    t = synth.ID[name]
    w = synth.iq_blocks(t, rows, cols, 8)
    w[5, 0:2] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)  # row 5's first block scale
    x = np.random.default_rng(3).normal(0, 1, (9, cols)).astype(np.float32)
    q, d = orc.q8_round(x)
    y, _ = run(g, t, [w], [9], rows, cols, q, d)
    want = orc.q8_rows(t, w, rows, cols, q, d)
    keep = [r for r in range(rows) if r != 5]
    assert (g.bits(y[:9, keep]) == g.bits(want[:, keep])).all()
    assert np.isnan(y[:9, 5]).all() and not np.isfinite(want[:, 5]).any()


def test_lane_group_refusals(g):
    from libosmos_amd import capi
    L = capi.lib()
    p = capi.addr(g.dev(np.zeros(64, np.int64)))
    t = synth.ID["IQ2_XXS"]
    assert not L.osmos_lane_group(synth.ID["Q4_K"], p, p, p, 1, 1, 64, 256, p, p, p, 64, None)  # not a lane GEMM type
    assert not L.osmos_lane_group(t, p, p, p, 1, 1, 60, 256, p, p, p, 64, None)  # rows not whole tiles
    assert not L.osmos_lane_group(t, p, p, p, 1, 1, 64, 200, p, p, p, 64, None)  # cols not whole blocks
    assert not L.osmos_lane_group(t, p, p, p, 1, 4097, 64, 256, p, p, p, 64, None)  # past the most tokens
    assert not L.osmos_lane_group(t, p, p, p, 0, 1, 64, 256, p, p, p, 64, None)
