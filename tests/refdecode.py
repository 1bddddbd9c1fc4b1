"""Independent float64 dequantizers for the non-IQ GGUF types, written from the published GGUF block layouts (ggml's
dequantize_row_* as gguf-py restates them), vectorised in numpy. They share nothing with oracle/mv.c but the layout
and pin its decoders by value: every one of these types' values is an exact product in float32 except the K-quants'
final subtract, which the test compares after rounding the same two float32 operands.
"""
import numpy as np


def f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float64)


def _h(blocks, at):
    return f16(blocks[:, at].astype(np.uint16) | (blocks[:, at + 1].astype(np.uint16) << 8))


def q4_0(blocks):
    d = _h(blocks, 0)
    qs = blocks[:, 2:18]
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float64) - 8
    return d[:, None] * q


def q8_0(blocks):
    d = _h(blocks, 0)
    return d[:, None] * blocks[:, 2:34].view(np.int8).astype(np.float64)


def _k_scales(s):
    sc = np.zeros((s.shape[0], 8), np.int64)
    m = np.zeros((s.shape[0], 8), np.int64)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        m[:, j] = s[:, j + 4] & 63
        sc[:, j + 4] = (s[:, j + 8] & 0xF) | ((s[:, j] >> 6) << 4)
        m[:, j + 4] = (s[:, j + 8] >> 4) | ((s[:, j + 4] >> 6) << 4)
    return sc, m


def q4_k(blocks):
    """returns (a, b) with value = f32(a) - f32(b): a = (d sc) q, b = dmin m (both exact in float32)"""
    d, dmin = _h(blocks, 0), _h(blocks, 2)
    sc, m = _k_scales(blocks[:, 4:16].astype(np.int64))
    a = np.zeros((blocks.shape[0], 256))
    b = np.zeros((blocks.shape[0], 256))
    for g in range(8):
        qs = blocks[:, 16 + 32 * (g // 2):16 + 32 * (g // 2 + 1)]
        q = (qs >> (4 * (g % 2))) & 15
        a[:, 32 * g:32 * g + 32] = (d * sc[:, g])[:, None] * q
        b[:, 32 * g:32 * g + 32] = (dmin * m[:, g])[:, None]
    return a, b


def q5_k(blocks):
    d, dmin = _h(blocks, 0), _h(blocks, 2)
    sc, m = _k_scales(blocks[:, 4:16].astype(np.int64))
    qh = blocks[:, 16:48]
    a = np.zeros((blocks.shape[0], 256))
    b = np.zeros((blocks.shape[0], 256))
    for g in range(8):
        qs = blocks[:, 48 + 32 * (g // 2):48 + 32 * (g // 2 + 1)]
        q = ((qs >> (4 * (g % 2))) & 15) | (((qh >> g) & 1) << 4)
        a[:, 32 * g:32 * g + 32] = (d * sc[:, g])[:, None] * q
        b[:, 32 * g:32 * g + 32] = (dmin * m[:, g])[:, None]
    return a, b


def q6_k(blocks):
    ql, qh = blocks[:, 0:128].astype(np.int64), blocks[:, 128:192].astype(np.int64)
    sc = blocks[:, 192:208].view(np.int8).astype(np.float64)
    d = _h(blocks, 208)
    out = np.zeros((blocks.shape[0], 256))
    for n in range(2):
        for l in range(32):
            q1 = ((ql[:, 64 * n + l] & 15) | (((qh[:, 32 * n + l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[:, 64 * n + l + 32] & 15) | (((qh[:, 32 * n + l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[:, 64 * n + l] >> 4) | (((qh[:, 32 * n + l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[:, 64 * n + l + 32] >> 4) | (((qh[:, 32 * n + l] >> 6) & 3) << 4)) - 32
            for k, q in enumerate((q1, q2, q3, q4)):
                i = 128 * n + l + 32 * k
                out[:, i] = d * sc[:, i // 16] * q
    return out


def q2_k(blocks):
    sc = blocks[:, 0:16].astype(np.int64)
    qs = blocks[:, 16:80].astype(np.int64)
    d, dmin = _h(blocks, 80), _h(blocks, 82)
    a = np.zeros((blocks.shape[0], 256))
    b = np.zeros((blocks.shape[0], 256))
    for i in range(256):
        n, r = i // 128, i % 128
        q = (qs[:, 32 * n + r % 32] >> (2 * (r // 32))) & 3
        g = i // 16
        a[:, i] = d * (sc[:, g] & 15) * q
        b[:, i] = dmin * (sc[:, g] >> 4)
    return a, b


def q3_k(blocks):
    hm = blocks[:, 0:32].astype(np.int64)
    qs = blocks[:, 32:96].astype(np.int64)
    s = blocks[:, 96:108].astype(np.int64)
    d = _h(blocks, 108)
    sc = np.zeros((blocks.shape[0], 16), np.int64)
    for g in range(16):  # ggml's kmask unpacking of 16 6-bit scales
        lo = (s[:, g % 8] >> (4 * (g // 8))) & 15
        hi = (s[:, 8 + g % 4] >> (2 * (g // 4))) & 3
        sc[:, g] = lo | (hi << 4)
    out = np.zeros((blocks.shape[0], 256))
    for i in range(256):
        n, r = i // 128, i % 128
        j, l = r // 32, r % 32
        q = ((qs[:, 32 * n + l] >> (2 * j)) & 3) - np.where((hm[:, l] >> (4 * n + j)) & 1, 0, 4)
        out[:, i] = d * (sc[:, i // 16] - 32) * q
    return out


IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float64)


def iq4_nl(blocks):
    d = _h(blocks, 0)
    qs = blocks[:, 2:18]
    return d[:, None] * IQ4NL[np.concatenate([qs & 15, qs >> 4], axis=1)]


def iq4_xs(blocks):
    d = _h(blocks, 0)
    sh = blocks[:, 2].astype(np.int64) | (blocks[:, 3].astype(np.int64) << 8)
    out = np.zeros((blocks.shape[0], 256))
    for g in range(8):
        ls = ((blocks[:, 4 + g // 2].astype(np.int64) >> (4 * (g % 2))) & 15) | (((sh >> (2 * g)) & 3) << 4)
        qs = blocks[:, 8 + 16 * g:24 + 16 * g]
        v = IQ4NL[np.concatenate([qs & 15, qs >> 4], axis=1)]
        out[:, 32 * g:32 * g + 32] = (d * (ls - 32))[:, None] * v
    return out


def bf16(raw):
    u = raw.view(np.uint16).astype(np.uint32) << 16
    return u.view(np.float32).astype(np.float64)
