"""The Q5_KR layout's numpy restatement (tests/q5kr.py) on the CPU: a lone value lands where the reference's
description puts it, the repack carries every Q5_K field unchanged (the 5-bit values, the 6-bit scales and minimums,
d and dmin), and the ABI names the repack. (reference kernels/quant.h:117-123, include/osmos/gpu/quant.h:17-19,42-47;
the reference checks the repack through its products' bits, tests/gpu/test_mm_gpu.hip:290-309 - the GPU tests here)"""
import numpy as np

from libosmos_amd import synth
from tests import q5kr


def test_lone_value_lands_by_the_description():
    # row 19 (tile 1, r 3), column 256 + 77 (block 1, group 2, value 13: chunk 1 -> h 1, v 5): slot 19, nibble 5
    rows, cols = 32, 512
    w = np.zeros((rows, 2, 176), np.uint8)
    w[19, 1, 48 + 32 * 1 + 13] = 0x0B  # group 2 is the low nibbles of qs[32:64]; value 13 = 11
    w[19, 1, 16 + 13] = 1 << 2  # its fifth bit
    out = q5kr.repack(w.reshape(-1), rows, cols).reshape(2, 2, 2880)
    seg = 64 + 2 * 352
    nz = np.flatnonzero(out)
    assert list(nz) == [(1 * 2 + 1) * 2880 + seg + 8 * 19 + 2, (1 * 2 + 1) * 2880 + seg + 256 + 2 * 19]
    assert out[1, 1, seg + 8 * 19 + 2] == 0xB0 and out[1, 1, seg + 256 + 2 * 19] == 1 << 5


def test_scales_and_heads_land_by_the_description():
    rows, cols = 16, 256
    w = np.zeros((rows, 176), np.uint8)
    w[7, 0:4] = [1, 2, 3, 4]
    w[7, 4 + 1] = 45  # group 1's scale (6 bits)
    w[7, 4 + 8 + 2] = 0x9 | 0x5 << 4  # group 6: scale low 4 bits 9, minimum low 4 bits 5
    w[7, 4 + 2] |= 2 << 6  # group 6's scale high bits 2
    out = q5kr.repack(w.reshape(-1), rows, cols)
    assert list(out[28:32]) == [1, 2, 3, 4]
    assert out[64 + 352 * 1 + 320 + 14] == 45
    assert out[64 + 352 * 6 + 320 + 14] == 9 | 2 << 4 and out[64 + 352 * 6 + 321 + 14] == 5
    assert out[64 + 352 * 2 + 320 + 14] == 0  # (group 2's scale is byte 2's low 6 bits: 0)


def test_repack_carries_every_field():
    rows, cols = 48, 768
    w = synth.random_blocks(synth.ID["Q5_K"], rows, cols, 5)
    wr = q5kr.repack(w.reshape(-1), rows, cols)
    assert wr.size == rows * (cols // 256) * 180
    got = q5kr.unpack(wr, rows, cols)
    want = q5kr._fields(np.asarray(w, np.uint8).reshape(rows, cols // 256, 176))
    for a, b in zip(got, want):
        assert (np.asarray(a) == np.asarray(b)).all()
    # a repack is a permutation of the fields: a changed byte anywhere moves the output
    w2 = np.array(w, np.uint8).reshape(-1).copy()
    w2[176 * 7 + 100] ^= 0x10
    assert (q5kr.repack(w2, rows, cols) != wr).sum() == 1


def test_abi_names_the_q5kr_entries():
    from libosmos_amd import capi
    L = capi.lib()
    for name in ("quant_repack_q5k", "quant_dequant_f16"):
        assert hasattr(L, name)
    assert capi.QUANT_Q5_KR == 0x10D and capi.quant_q5kr_bytes(32, 512) == 32 * 2 * 180
