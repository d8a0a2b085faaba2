"""Pins of the oracle's Gemma4 APEX expert formats (oracle/lt_oracle.c:
lto_dequant_q5_0 / lto_dot_q5_0, lto_dequant_q5_1, lto_dequant_iq4_nl /
lto_dot_iq4_nl, lto_dequant_q3_k) and of quantMatvec's dispatch over them
(math.zig:133-171: Q5_0 and IQ4_NL through their fused dots, Q5_1 and Q3_K
through dequant + dotf32).

Decoders below are written from the ggml block layouts, independently of
the oracle's loops; the fused dots' accumulation orders are fixed by
hand-derived cases whose fp32 result depends on that order."""
import numpy as np
import pytest

import pyoracle as orc
from llmtoy_amd import ggml, synth

TABLE = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def f16(b):
    return b[..., 0:2].copy().view(np.float16).astype(np.float32)[..., 0]


def bits(b):  # [..., nbytes] -> [..., nbytes * 8] little-endian bit order
    return np.unpackbits(b, axis=-1, bitorder="little")


def q5_0_np(blocks):
    b = blocks.reshape(-1, 22)
    qs = b[:, 6:22]
    nib = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int32)  # elements 0..15, 16..31
    hb = bits(b[:, 2:6]).astype(np.int32)                               # bit e of the LE u32
    return (f16(b)[:, None] * ((nib | (hb << 4)) - 16).astype(np.float32)).reshape(-1)


def q5_1_np(blocks):
    b = blocks.reshape(-1, 24)
    qs = b[:, 8:24]
    nib = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int32)
    hb = bits(b[:, 4:8]).astype(np.int32)
    d, m = f16(b), f16(b[:, 2:4])
    q = (nib | (hb << 4)).astype(np.float32)
    return ((d[:, None] * q).astype(np.float32) + m[:, None]).reshape(-1)


def iq4_nl_np(blocks):
    b = blocks.reshape(-1, 18)
    qs = b[:, 2:18]
    idx = np.concatenate([qs & 15, qs >> 4], axis=1)
    return (f16(b)[:, None] * TABLE[idx]).reshape(-1)


def q3k_scales_np(s12):
    # scale i: low 4 bits from byte i (i < 8) or the high nibble of byte i - 8,
    # high 2 bits from bits 2 (i // 4) of byte 8 + i % 4
    s12 = s12.astype(np.int32)
    out = np.empty(s12.shape[:-1] + (16,), np.int32)
    for i in range(16):
        lo = s12[..., i] & 15 if i < 8 else s12[..., i - 8] >> 4
        hi = (s12[..., 8 + i % 4] >> (2 * (i // 4))) & 3
        out[..., i] = lo | (hi << 4)
    return out


def q3k_np(blocks):
    b = blocks.reshape(-1, 110)
    hmask, qs = b[:, 0:32].astype(np.int32), b[:, 32:96].astype(np.int32)
    sc = q3k_scales_np(b[:, 96:108])
    d = f16(b[:, 108:110])
    out = np.empty((b.shape[0], 256), np.float32)
    for n in range(256):
        h, j, g, l = n // 128, (n % 128) // 32, (n % 32) // 16, n % 16
        q2 = (qs[:, 32 * h + 16 * g + l] >> (2 * j)) & 3
        hi = (hmask[:, 16 * g + l] >> (j + 4 * h)) & 1
        dl = (d * (sc[:, 8 * h + 2 * j + g] - 32).astype(np.float32)).astype(np.float32)
        out[:, n] = (q2 - 4 * (1 - hi)).astype(np.float32) * dl
    return out.reshape(-1)


DECODERS = {ggml.Q5_0: q5_0_np, ggml.Q5_1: q5_1_np, ggml.IQ4_NL: iq4_nl_np, ggml.Q3_K: q3k_np}


@pytest.mark.parametrize("gtype", list(DECODERS))
def test_dequant_matches_independent_decoder(gtype):
    g = np.random.default_rng(gtype)
    m = synth.quant_matrix(g, gtype, 7, 512)
    m.reshape(-1, ggml.BLOCK_BYTES[gtype])  # whole blocks
    want = DECODERS[gtype](m)
    got = orc.dequant(gtype, m, 7 * 512)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q3k_scale_unpacking_extremes():
    for fill in (0x00, 0xFF, 0x55, 0xAA):
        s = np.full(12, fill, np.uint8)
        assert orc.q3k_scales(s).tolist() == q3k_scales_np(s).tolist()
    s = np.random.default_rng(3).integers(0, 256, 12, dtype=np.uint8)
    assert orc.q3k_scales(s).tolist() == q3k_scales_np(s).tolist()
    assert max(orc.q3k_scales(np.full(12, 0xFF, np.uint8))) == 63


def test_dot_q5_0_reference_kat():
    # dequant.zig:716-735
    data = np.zeros(44, np.uint8)
    data[0:2] = [0x00, 0x38]  # 0.5
    data[2:6] = 0xAA
    for j in range(16):
        data[6 + j] = (j & 15) | (((j + 3) & 15) << 4)
    data[22:24] = [0x00, 0x30]  # 0.125
    data[28:44] = 0x55
    vec = (np.arange(64, dtype=np.float32) * np.float32(0.1) - np.float32(3.0)).astype(np.float32)
    expected = np.float32(0)
    for d, v in zip(orc.dequant(ggml.Q5_0, data, 64), vec):
        expected = np.float32(expected + d * v)
    assert abs(orc.dot_q5_0(data, vec) - expected) <= 1e-3


def test_dot_iq4_nl_reference_kat():
    # dequant.zig:737-758
    data = np.zeros(36, np.uint8)
    data[0:2] = [0x00, 0x3C]
    data[18:20] = [0x00, 0x40]
    for i in range(16):
        data[2 + i] = (i & 15) | ((15 - i) << 4)
        data[20 + i] = ((i + 3) & 15) | (((i + 5) & 15) << 4)
    vec = (((np.arange(64) % 7) + 1) * 0.25).astype(np.float32)
    expected = np.float32(0)
    for w, x in zip(orc.dequant(ggml.IQ4_NL, data, 64), vec):
        expected = np.float32(expected + w * x)
    assert abs(orc.dot_iq4_nl(data, vec) - expected) <= 1e-3


def test_dot_q5_0_uses_eight_lane_accumulators():
    # q5 = 1 on elements 0, 1, 8, 9 (nib 1, high bit 1); 0 elsewhere (nib 0,
    # high bit 1).  x: 2^24, 1, -2^24, 1.  Lanes: acc0 = 2^24 - 2^24 = 0,
    # acc1 = 1 + 1 = 2 -> 2.  Index order would give ((2^24 + 1) - 2^24) + 1 = 1.
    blk = np.zeros(22, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:6] = 0xFF
    for e in (0, 1, 8, 9):
        blk[6 + e] |= 1
    v = np.zeros(32, np.float32)
    v[[0, 1, 8, 9]] = [2.0 ** 24, 1, -2.0 ** 24, 1]
    assert orc.dot_q5_0(blk, v) == 2.0


def test_dot_iq4_nl_interleaves_low_and_high_nibbles():
    # table[8] = 1.  Elements 0, 16, 1, 17 in that accumulation order:
    # ((2^24 + 1) - 2^24) + 1 = 1; all low nibbles first would give 2.
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:18] = 0x00  # table[0] = -127 times x = 0 elsewhere
    blk[2] = 0x88
    blk[3] = 0x88
    v = np.zeros(32, np.float32)
    v[[0, 16, 1, 17]] = [2.0 ** 24, 1, -2.0 ** 24, 1]
    assert orc.dot_iq4_nl(blk, v) == 1.0


@pytest.mark.parametrize("gtype", list(DECODERS))
def test_quant_matvec_dispatch_and_float64(gtype):
    g = np.random.default_rng(100 + gtype)
    rows, cols = 9, 768
    m = synth.quant_matrix(g, gtype, rows, cols)
    x = synth.normal(g, (cols,))
    got = orc.quant_matvec(m, gtype, x, rows, cols)
    W = DECODERS[gtype](m).reshape(rows, cols)
    want = W.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5
    for r in range(rows):  # the reference's per-type dispatch (math.zig:133-171)
        if gtype == ggml.Q5_0:
            assert got[r] == orc.dot_q5_0(m[r], x)
        elif gtype == ggml.IQ4_NL:
            assert got[r] == orc.dot_iq4_nl(m[r], x)
        else:
            assert got[r] == orc.dotf32(W[r], x)
