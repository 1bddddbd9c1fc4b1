"""Test data that exposes the f16 matmul's K order (shared by the CPU oracle test and the GPU test): 16 identical
weight rows and tokens whose activations are zero but for three columns - c0 in slab 0 and c2 in slab W (both
partition 0 of the reference's K split), c1 in slab 1 (partition 1) - chosen so that partition 0's two products
nearly cancel and c1's product is far below c0's: summed as the contract orders it (each partition a chain from zero,
then the partitions added) the result keeps c1's product, summed as one chain in K order it loses it. every step
then has a single product besides the running sum, all of one magnitude where they meet, so a matrix-core step drops
no bit and the oracle's step model is exact."""
import numpy as np

from libosmos_amd import synth
from oracle import orc


def f16(v):
    with np.errstate(over="ignore"):
        return np.float32(np.float16(v))


def case(name, cols, group, seed, n_tok=6):
    t = synth.ID[name]
    mk = synth.iq_blocks if name.startswith("IQ") else synth.random_blocks
    sl, W = orc.mm_shape(t, cols, group)
    assert cols >= (W + 1) * sl
    rng = np.random.default_rng(seed)
    for attempt in range(50):
        row = mk(t, 1, cols, seed + 1000 * attempt)
        wv = np.array([f16(v) for v in orc.dequant(t, row, cols)], np.float32)
        xs, chain, ordered = [], [], []
        for _ in range(n_tok):
            s0 = np.flatnonzero(np.abs(wv[:sl]) > 0)
            s1 = sl + np.flatnonzero(wv[sl:2 * sl] != 0)
            s2 = W * sl + np.flatnonzero(wv[W * sl:(W + 1) * sl] != 0)
            if not len(s0) or not len(s1) or not len(s2):
                break
            c0 = int(rng.choice(s0[np.argsort(-np.abs(wv[s0]))][:8]))
            c1, c2 = int(rng.choice(s1)), int(rng.choice(s2))
            w0, w1, w2 = wv[c0], wv[c1], wv[c2]
            x0 = f16(1024.0)
            x2 = f16(-np.float64(w0) * 1024.0 / np.float64(w2))
            if not np.isfinite(x2) or x2 == 0:
                break
            p0a = np.float32(np.float64(w0) * x0)                       # partition 0 after c0 (exact)
            r = np.float32(np.float64(p0a) + np.float64(w2) * x2)       # after c2: the near cancellation
            if r == 0:
                break
            x1 = f16(np.float64(r) / 64.0 / np.float64(w1))
            if x1 == 0 or not np.isfinite(x1):
                break
            p1 = np.float32(np.float64(w1) * x1)
            ordered.append(np.float32(r + p1))                            # (partitions 2 .. W - 1 zero)
            k = np.float32(np.float64(p0a) + np.float64(p1))              # one chain in K order: c0, c1, c2
            chain.append(np.float32(np.float64(k) + np.float64(w2) * x2))
            x = np.zeros(cols, np.float32)
            x[c0], x[c1], x[c2] = x0, x1, x2
            xs.append(x)
        if len(xs) == n_tok and all(a != b for a, b in zip(ordered, chain)):
            w = np.repeat(row, 16, axis=0)
            return w, np.stack(xs), np.array(ordered, np.float32), np.array(chain, np.float32)
    raise AssertionError("no discriminating case for %s at %d columns" % (name, cols))
