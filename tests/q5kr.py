"""numpy restatement of the Q5_KR layout (Q5_K repacked in tiles of 16 rows), test infrastructure: the repack and its
inverse. the layout, from the reference's description (kernels/quant.h:117-123, include/osmos/gpu/quant.h:17-19,42-47):
a tile's block of 256 columns is 2880 bytes - the 16 rows' f16 d and dmin (4 bytes a row) - then for each 32-column
group g a 352-byte segment: 32 slots of 16 values (slot h*16 + r holds row r's chunks 4g + h and 4g + 2 + h, value v
from chunk 4g + 2(v//8) + h's value v%8) as 8 bytes of nibbles (value v at nibble v), their fifth bits as 2 bytes at
256 + slot*2 (bit v), then row r's 6-bit scale and minimum as 2 bytes at 320 + r*2."""
import numpy as np

KB, KR = 176, 180  # a Q5_K block; a row's share of a Q5_KR tile's block


def _fields(blocks):
    """Q5_K blocks (..., 176) -> (d4 (..., 4), sc (..., 8), m (..., 8), q (..., 8, 32)) - the 5-bit values by group"""
    s = blocks[..., 4:16].astype(np.int32)
    sc = np.empty(blocks.shape[:-1] + (8,), np.int32)
    m = np.empty_like(sc)
    sc[..., :4], m[..., :4] = s[..., 0:4] & 63, s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    qh = blocks[..., 16:48].astype(np.int32)
    qs = blocks[..., 48:176].astype(np.int32).reshape(blocks.shape[:-1] + (4, 32))
    q = np.empty(blocks.shape[:-1] + (8, 32), np.int32)
    for g in range(8):
        q[..., g, :] = ((qs[..., g // 2, :] >> (4 * (g % 2))) & 15) | (((qh >> g) & 1) << 4)
    return blocks[..., 0:4], sc, m, q


def repack(w, rows, cols):
    """row-major Q5_K bytes (rows x cols) -> Q5_KR bytes"""
    nb = cols // 256
    blk = np.asarray(w, np.uint8).reshape(rows // 16, 16, nb, KB).transpose(0, 2, 1, 3)  # (tile, block, r, 176)
    d4, sc, m, q = _fields(blk)
    out = np.zeros((rows // 16, nb, 16 * KR), np.uint8)
    out[..., :64] = d4.reshape(rows // 16, nb, 64)
    v = np.arange(16)
    for g in range(8):
        seg = 64 + 352 * g
        out[..., seg + 320:seg + 352:2], out[..., seg + 321:seg + 352:2] = sc[..., g], m[..., g]
        for h in range(2):
            vals = q[..., g, 8 * (2 * (v // 8) + h) + v % 8]  # (tile, block, r, 16)
            lo, hi = vals & 15, vals >> 4
            nib = (lo[..., 0::2] | lo[..., 1::2] << 4).astype(np.uint8)  # (tile, block, r, 8)
            fifth = (hi << v).sum(-1)
            for r in range(16):
                slot = 16 * h + r
                out[..., seg + 8 * slot:seg + 8 * slot + 8] = nib[..., r, :]
                out[..., seg + 256 + 2 * slot] = fifth[..., r] & 255
                out[..., seg + 257 + 2 * slot] = fifth[..., r] >> 8
    return out.reshape(-1)


def unpack(wr, rows, cols):
    """Q5_KR bytes -> (d4, sc, m, q) per (row, block) as _fields gives them for the Q5_K matrix"""
    nb = cols // 256
    t = np.asarray(wr, np.uint8).reshape(rows // 16, nb, 16 * KR).astype(np.int32)
    d4 = t[..., :64].reshape(rows // 16, nb, 16, 4)
    sc = np.empty((rows // 16, nb, 16, 8), np.int32)
    m = np.empty_like(sc)
    q = np.empty((rows // 16, nb, 16, 8, 32), np.int32)
    for g in range(8):
        seg = 64 + 352 * g
        sc[..., g], m[..., g] = t[..., seg + 320:seg + 352:2], t[..., seg + 321:seg + 352:2]
        for slot in range(32):
            h, r = slot // 16, slot % 16
            nib = t[..., seg + 8 * slot:seg + 8 * slot + 8]
            fifth = t[..., seg + 256 + 2 * slot] | t[..., seg + 257 + 2 * slot] << 8
            for vv in range(16):
                val = ((nib[..., vv // 2] >> (4 * (vv % 2))) & 15) | (((fifth >> vv) & 1) << 4)
                q[..., r, g, 8 * (2 * (vv // 8) + h) + vv % 8] = val
    tr = lambda a: np.moveaxis(a, 2, 1).reshape((rows, nb) + a.shape[3:])  # noqa: E731 (tile, block, r) -> (row, block)
    return tr(d4), tr(sc), tr(m), tr(q)
