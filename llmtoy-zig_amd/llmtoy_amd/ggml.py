"""GGUF block formats used on the decode path (numpy, byte-exact).

Ids and sizes follow llmtoy-zig's src/gguf/types.zig:23-53, 138-173 and the
block layouts of src/quant/dequant.zig (Q8_0 31-40, Q4_K 136-155,
Q6_K 219-235).
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
Q5_0, Q5_1, Q3_K, IQ4_NL = 6, 7, 11, 20  # the Gemma4 APEX expert formats (dequant.zig:189-659)

BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q5_0: 32, Q5_1: 32, Q3_K: 256, IQ4_NL: 32}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q5_0: 22, Q5_1: 24, Q3_K: 110, IQ4_NL: 18}
NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", Q5_0: "Q5_0", Q5_1: "Q5_1",
         Q3_K: "Q3_K", IQ4_NL: "IQ4_NL"}


def row_bytes(ggml_type: int, cols: int) -> int:
    """Bytes of one row (ops/math.zig:194-208; integer division, as there)."""
    return (cols // BLOCK_ELEMS[ggml_type]) * BLOCK_BYTES[ggml_type]


def f16_bits(values: np.ndarray) -> np.ndarray:
    """fp32 -> IEEE binary16 bit patterns, round to nearest even."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack 6-bit (scale, min) pairs of 8 sub-blocks into the 12-byte field.

    Inverse of get_scale_min_k4 (quant/dequant.zig:291-300).  sc, mn: uint8
    arrays [..., 8] with values < 64.  Returns uint8 [..., 12].
    """
    sc = np.asarray(sc, dtype=np.uint8)
    mn = np.asarray(mn, dtype=np.uint8)
    out = np.empty(sc.shape[:-1] + (12,), dtype=np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
    return out


def unpack_q4k_scales(s: np.ndarray):
    """get_scale_min_k4 for all 8 sub-blocks: uint8 [..., 12] -> (sc, mn) [..., 8]."""
    s = np.asarray(s, dtype=np.uint8)
    sc = np.empty(s.shape[:-1] + (8,), dtype=np.uint8)
    mn = np.empty_like(sc)
    sc[..., 0:4] = s[..., 0:4] & 63
    mn[..., 0:4] = s[..., 4:8] & 63
    sc[..., 4:8] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:8] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, mn
