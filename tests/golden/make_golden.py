"""Writes the golden vectors in tests/golden/ from the reference's own compiled CPU path (oracle/_ref/libref.so, built
by oracle/ref.mk from /root/reference/src/cpu/{q8,expert}.c and kernels/lane.h, in the build container only).

fixtures (inputs and the reference's outputs; the inputs from libosmos_amd.synth with the seeds below):
- golden_lane.npz: for each lane type (IQ2_XXS, IQ2_XS, IQ1_M, IQ1_S, IQ2_S, IQ3_XXS, Q2_K) and cols in COLS:
  w_<type>_<cols> (6 rows of random blocks), shared x_<cols> (3 tokens, the first with a zero block, the second with
  a lone -2.5 - the reference test's specials, tests/test_cpu_q8.c:191-197), the reference's q_<cols>, d_<cols>
  (cpu_q8_round) and y_<type>_<cols> (cpu_q8_rows: 3 tokens x 6 rows);
- golden_mv.npz: the same weights against fp32 x: ym_<type>_<cols> (cpu_mv_rows);
- golden_exp.npz: lane_exp and lane_swiglu over a spread of arguments (kernels/lane.h);
- golden_layer.npz: a small lane layer (dim 512, ff 256, IQ3_XXS gate/up/down, 3 tokens x top-2 over 4 experts)
  composed of the reference's cpu_q8_round, cpu_q8_rows and lane_swiglu in src/cpu/lane.c's phase order.

run: python tests/golden/make_golden.py  (needs oracle/_ref; `make -C oracle ref`)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from libosmos_amd import synth  # noqa: E402
from oracle import orc  # noqa: E402

LANE_TYPES = ["IQ2_XXS", "IQ2_XS", "IQ1_M", "IQ1_S", "IQ2_S", "IQ3_XXS", "Q2_K"]
COLS = [512, 768, 2048, 4352, 5120, 7168]
ROWS, TOK = 6, 3


def x_for(cols, seed):
    x = synth.normal((TOK, cols), seed) * 3.0
    x[0, :32] = 0.0  # a block of zeros
    x[1, 32:64] = 0.0
    x[1, 37] = -2.5  # a block of one value
    return x


def main():
    R = orc.ref()
    assert R is not None and R.ref_q8_ready(), "build oracle/_ref first (make -C oracle ref) on an AVX-512 VNNI host"
    lane, mv = {}, {}
    for ci, cols in enumerate(COLS):
        x = x_for(cols, 100 + ci)
        q, d = orc.q8_round(x, R)
        lane["x_%d" % cols], lane["q_%d" % cols], lane["d_%d" % cols] = x, q, d
        for ti, name in enumerate(LANE_TYPES):
            t = synth.ID[name]
            w = synth.random_blocks(t, ROWS, cols, 1000 * ci + ti)
            lane["w_%s_%d" % (name, cols)] = w
            lane["y_%s_%d" % (name, cols)] = orc.q8_rows(t, w, ROWS, cols, q, d, R)
            mv["ym_%s_%d" % (name, cols)] = orc.mv_rows(t, w, ROWS, cols, x, R)
    np.savez_compressed(os.path.join(HERE, "golden_lane.npz"), **lane)
    np.savez_compressed(os.path.join(HERE, "golden_mv.npz"), **mv)

    rng = np.random.default_rng(7)
    ex = np.concatenate([np.linspace(-87.0, 88.7, 4001, dtype=np.float32), rng.normal(0, 4, 4000).astype(np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 88.72283905, 88.7228393, 89.0, 1e3], np.float32)])
    ey = np.array([R.ref_lane_exp(float(v)) for v in ex], np.float32)
    g = rng.normal(0, 3, 3000).astype(np.float32)
    u = rng.normal(0, 3, 3000).astype(np.float32)
    lim = np.where(np.arange(3000) % 3 == 0, np.float32(np.inf), np.float32(7.0)).astype(np.float32)
    sc = rng.uniform(0, 1, 3000).astype(np.float32)
    h = np.array([R.ref_lane_swiglu(float(a), float(b), float(c), float(e)) for a, b, c, e in zip(g, u, lim, sc)],
                 np.float32)
    np.savez_compressed(os.path.join(HERE, "golden_exp.npz"), x=ex, y=ey, g=g, u=u, lim=lim, scale=sc, h=h)

    # the layer: 3 tokens, top-2 over 4 experts; pair rows sorted by expert (src/run/hip_lane.c:115-177)
    dim, ff, t3 = 512, 256, synth.ID["IQ3_XXS"]
    ids = np.array([[2, 0], [1, 2], [2, 3]], np.int32)
    wts = rng.uniform(0.1, 0.9, ids.shape).astype(np.float32)
    xt = synth.normal((3, dim), 11)
    gate = [synth.iq_blocks(t3, ff, dim, 20 + e) for e in range(4)]
    up = [synth.iq_blocks(t3, ff, dim, 30 + e) for e in range(4)]
    down = [synth.iq_blocks(t3, dim, ff, 40 + e) for e in range(4)]
    pairs = sorted(((int(ids[t, j]), t * 2 + j) for t in range(3) for j in range(2)))
    rows_x = np.stack([xt[m // 2] for _, m in pairs])
    scale = np.array([wts[m // 2, m % 2] for _, m in pairs], np.float32)
    qx, dx = orc.q8_round(rows_x, R)
    h = np.zeros((len(pairs), ff), np.float32)
    for r, (e, _) in enumerate(pairs):
        gg = orc.q8_rows(t3, gate[e], ff, dim, qx[r:r + 1], dx[r:r + 1], R)[0]
        uu = orc.q8_rows(t3, up[e], ff, dim, qx[r:r + 1], dx[r:r + 1], R)[0]
        h[r] = [R.ref_lane_swiglu(float(a), float(b), float("inf"), float(scale[r])) for a, b in zip(gg, uu)]
    qh, dh = orc.q8_round(h, R)
    ye = np.stack([orc.q8_rows(t3, down[e], dim, ff, qh[r:r + 1], dh[r:r + 1], R)[0] for r, (e, _) in enumerate(pairs)])
    row_of = {m: r for r, (_, m) in enumerate(pairs)}
    out = np.zeros((3, dim), np.float32)
    for t in range(3):  # ascending expert id: the pair rows ascend by expert
        for r in sorted(row_of[t * 2 + j] for j in range(2)):
            out[t] += ye[r]
    np.savez_compressed(os.path.join(HERE, "golden_layer.npz"), ids=ids, wts=wts, x=xt, gate=np.stack(gate),
                        up=np.stack(up), down=np.stack(down), h=h, ye=ye, out=out)
    print("ok")


main()
