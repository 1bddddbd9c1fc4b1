"""Seeded synthetic GGUF weight blocks and activations (the workloads' inputs; there are no model files offline).

The reference ships no weight quantizer (its requant tools link an external ggml), so these generators are this
package's own. Every generator is deterministic in its seed (numpy's PCG64):

- random_blocks: random bytes in every field, each block's scale a small f16 - the shape of the reference's own test
  fill (tests/test_cpu_q8.c:34-53: bytes from an LCG, d = f16 in [2^-4, 2^-3)); any valid block exercises the kernels.
- iq_blocks: the IQ types as the workload configs describe them - uniform grid indices, random sign bits and 3/4-bit
  scales (random bytes), the block scale f16(|N(0, 0.02)|).
- quant_q4_0 / quant_q4_k / quant_q3_k: N(0, 0.02) weights quantized into valid blocks (Q4_0 as ggml's
  quantize_row_q4_0: d = signed max / -8, q = min(15, int(x / d + 8.5)); Q4_K and Q3_K by a plain per-group scale/min
  fit into 6-bit sub-scales).
"""
import numpy as np

# GGUF type id -> (name, values a block, bytes a block); reference include/osmos/model/qtype.h:28-53
TYPES = {
    0: ("F32", 1, 4),
    2: ("Q4_0", 32, 18),
    8: ("Q8_0", 32, 34),
    10: ("Q2_K", 256, 84),
    11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144),
    13: ("Q5_K", 256, 176),
    14: ("Q6_K", 256, 210),
    16: ("IQ2_XXS", 256, 66),
    17: ("IQ2_XS", 256, 74),
    18: ("IQ3_XXS", 256, 98),
    19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18),
    22: ("IQ2_S", 256, 82),
    23: ("IQ4_XS", 256, 136),
    29: ("IQ1_M", 256, 56),
    30: ("BF16", 1, 2),
}
ID = {v[0]: k for k, v in TYPES.items()}
# where each type's f16 block scale(s) live (byte offsets): the fields a fill overwrites with sane scales
_SCALE_AT = {"Q4_0": [0], "Q8_0": [0], "IQ4_NL": [0], "Q2_K": [80, 82], "Q3_K": [108], "Q4_K": [0, 2], "Q5_K": [0, 2],
             "Q6_K": [208], "IQ2_XXS": [0], "IQ2_XS": [0], "IQ3_XXS": [0], "IQ1_S": [0], "IQ2_S": [0], "IQ4_XS": [0]}


def row_bytes(type_id, cols):
    _, v, b = TYPES[type_id]
    assert cols % v == 0
    return cols // v * b


def _set_f16(blocks, at, h16):
    blocks[:, at] = (h16 & 0xFF).astype(np.uint8)
    blocks[:, at + 1] = (h16 >> 8).astype(np.uint8)


def _set_iq1m_scale(blocks, h16):
    for k in range(4):  # the f16's nibble k in the top nibble of scale word k (reference kernels/quant.h:335-348)
        hi = 48 + 2 * k + 1
        blocks[:, hi] = (blocks[:, hi] & 0x0F) | (((h16 >> (4 * k)) & 0x0F) << 4).astype(np.uint8)


def random_blocks(type_id, rows, cols, seed):
    """random bytes; each scale an f16 in [2^-4, 2^-3) (the reference test fill's range). returns uint8 [rows, rb]"""
    name, v, b = TYPES[type_id]
    rng = np.random.default_rng(seed)
    nblk = rows * (cols // v)
    blocks = rng.integers(0, 256, size=(nblk, b), dtype=np.uint8)
    if name == "IQ1_M":
        _set_iq1m_scale(blocks, (0x2C00 | rng.integers(0, 1024, nblk)).astype(np.uint16))
    elif name in _SCALE_AT:
        for at in _SCALE_AT[name]:
            _set_f16(blocks, at, (0x2C00 | rng.integers(0, 1024, nblk)).astype(np.uint16))
    return blocks.reshape(rows, -1)


def iq_blocks(type_id, rows, cols, seed, sigma=0.02):
    """the IQ configs' weights: uniform indices / signs / sub-scales, block scale f16(|N(0, sigma)|)"""
    name, v, b = TYPES[type_id]
    rng = np.random.default_rng(seed)
    nblk = rows * (cols // v)
    blocks = rng.integers(0, 256, size=(nblk, b), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, sigma, nblk)).astype(np.float16).view(np.uint16)
    if name == "IQ1_M":
        _set_iq1m_scale(blocks, d)
    else:
        _set_f16(blocks, _SCALE_AT[name][0], d)
    return blocks.reshape(rows, -1)


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def quant_q4_0(w):
    """ggml's quantize_row_q4_0 on w [rows, cols] fp32 -> uint8 [rows, cols/32*18]"""
    rows, cols = w.shape
    g = w.reshape(-1, 32).astype(np.float32)
    idx = np.argmax(np.abs(g), axis=1)
    mx = g[np.arange(len(g)), idx]
    d = mx / np.float32(-8.0)
    idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.minimum(15, (g * idv[:, None] + np.float32(8.5)).astype(np.int32)).astype(np.uint8)
    out = np.zeros((len(g), 18), np.uint8)
    _set_f16(out, 0, _f16(d).view(np.uint16))
    out[:, 2:] = (q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)
    return out.reshape(rows, -1)


def _pack_k_scales(sc, m):
    """8 6-bit (sc, m) pairs a block -> the 12 K-quant scale bytes (reference kernels/quant.h:91-103's layout)"""
    n = sc.shape[0]
    s = np.zeros((n, 12), np.uint8)
    for j in range(4):
        s[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (m[:, j] & 63) | ((m[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 15) | ((m[:, j + 4] & 15) << 4)
    return s


def quant_q4_k(w):
    """w [rows, cols] -> Q4_K blocks: per 32-group scale (max-min)/15 and min, 6-bit against the block's d / dmin"""
    rows, cols = w.shape
    g = w.reshape(-1, 8, 32).astype(np.float32)
    lo = np.minimum(g.min(axis=2), 0)
    hi = g.max(axis=2)
    scale = (hi - lo) / 15.0
    mins = -lo
    d = _f16(scale.max(axis=1) / 63.0).astype(np.float32)
    dmin = _f16(mins.max(axis=1) / 63.0).astype(np.float32)
    sc = np.clip(np.rint(scale / np.where(d > 0, d, 1)[:, None]), 0, 63).astype(np.int32)
    m = np.clip(np.rint(mins / np.where(dmin > 0, dmin, 1)[:, None]), 0, 63).astype(np.int32)
    step = d[:, None] * sc
    q = np.clip(np.rint((g + (dmin[:, None] * m)[:, :, None]) / np.where(step > 0, step, 1)[:, :, None]), 0, 15)
    q = q.astype(np.uint8)
    out = np.zeros((g.shape[0], 144), np.uint8)
    _set_f16(out, 0, _f16(d).view(np.uint16))
    _set_f16(out, 2, _f16(dmin).view(np.uint16))
    out[:, 4:16] = _pack_k_scales(sc, m)
    for p in range(4):  # groups 2p (low nibbles) and 2p + 1 (high) share qs[32p .. 32p + 31]
        out[:, 16 + 32 * p:16 + 32 * (p + 1)] = q[:, 2 * p] | (q[:, 2 * p + 1] << 4)
    return out.reshape(rows, -1)


def quant_q3_k(w):
    """w [rows, cols] -> Q3_K blocks: per 16-group a signed 6-bit scale against d, codes -4 .. 3"""
    rows, cols = w.shape
    g = w.reshape(-1, 16, 16).astype(np.float32)
    amax = np.abs(g).max(axis=2)
    scale = amax / 4.0
    d = _f16(scale.max(axis=1) / 31.0).astype(np.float32)
    sc = np.clip(np.rint(scale / np.where(d > 0, d, 1)[:, None]), -32, 31).astype(np.int32)
    step = d[:, None] * sc
    q = np.clip(np.rint(g / np.where(step != 0, step, 1)[:, :, None]), -4, 3).astype(np.int32)
    n = g.shape[0]
    q = q.reshape(n, 256)
    hbit = (q >= 0).astype(np.uint8)
    q2 = np.where(q >= 0, q, q + 4).astype(np.uint8)
    out = np.zeros((n, 110), np.uint8)
    idx = np.arange(256)
    nn, r = idx // 128, idx % 128
    jj, l = r // 32, r % 32
    for i in range(256):  # value i: 2 bits of qs[32 n + l] at 2 jj; its high bit hmask[l] bit 4 n + jj
        out[:, 32 + 32 * nn[i] + l[i]] |= (q2[:, i] << (2 * jj[i])).astype(np.uint8)
        out[:, l[i]] |= (hbit[:, i] << (4 * nn[i] + jj[i])).astype(np.uint8)
    u = (sc + 32).astype(np.uint8)  # 6 bits a 16-group: low 4 a nibble of scales[0..7], high 2 of scales[8..11]
    for gi in range(16):
        grp, wi = gi // 4, gi % 4
        lo_at = 96 + (4 + wi if grp & 1 else wi)
        out[:, lo_at] |= ((u[:, gi] & 15) << (4 if grp & 2 else 0)).astype(np.uint8)
        out[:, 96 + 8 + wi] |= (((u[:, gi] >> 4) & 3) << (2 * grp)).astype(np.uint8)
    _set_f16(out, 108, _f16(d).view(np.uint16))
    return out.reshape(rows, -1)


def normal(shape, seed, sigma=1.0):
    return np.random.default_rng(seed).normal(0.0, sigma, shape).astype(np.float32)
