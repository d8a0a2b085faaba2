"""Pins the CPU oracle (oracle/lt_oracle.c) before it is trusted as the checker.

Each check cites the llmtoy-zig test or fact it restates.  Where the
reference holds no known answer, the oracle is compared with an independent
decoder written from the ggml block layout, with float64 arithmetic, or with
hand-derived results whose value depends on the exact operation order.
"""
import math

import numpy as np
import pytest

import pyoracle as orc
from llmtoy_amd import ggml, synth


# ---------------------------------------------------------------- f16
def test_f16_kat_pm_one():
    # quant/dequant.zig:671-678: 0x3C00 -> 1.0, 0xBC00 -> -1.0
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f16_to_f32(0xBC00) == -1.0
    out = orc.dequant(orc.F16, np.array([0x00, 0x3C, 0x00, 0xBC], dtype=np.uint8), 2)
    assert out.tolist() == [1.0, -1.0]


def test_f16_all_encodings_match_ieee():
    # IEEE-754 binary16 closed form (numpy's float16 -> float32 is exact),
    # subnormals, signed zeros and infinities included.
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = raw.view(np.float16).astype(np.float32)
    got = orc.dequant(orc.F16, raw.view(np.uint8), 65536)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # subnormal spot checks: 0x0001 = 2^-24, 0x03FF = 1023 * 2^-24
    assert orc.f16_to_f32(0x0001) == 2.0 ** -24
    assert orc.f16_to_f32(0x03FF) == 1023 * 2.0 ** -24


# ---------------------------------------------------------------- Q8_0
def test_q8_0_single_block_kat():
    # dequant.zig:702-714: d = 0.5, q = [2, -2, 4, 0, ...] -> [1, -1, 2, 0]
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = [0x00, 0x38]
    blk[2], blk[3], blk[4] = 2, np.uint8(254), 4
    out = orc.dequant(orc.Q8_0, blk, 32)
    assert out[:4].tolist() == [1.0, -1.0, 2.0, 0.0]
    assert not out[4:].any()


def _q8_two_blocks():
    data = np.zeros(68, dtype=np.uint8)
    data[0:2] = [0x00, 0x38]  # 0.5
    data[2:34] = np.arange(1, 33, dtype=np.uint8)
    data[34:36] = [0x00, 0x34]  # 0.25
    data[36:68] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    vec = (np.arange(64, dtype=np.float32) * np.float32(0.1) - np.float32(3.0)).astype(np.float32)
    return data, vec


def test_dot_q8_0_matches_dequant_dot_kat():
    # dequant.zig:680-700: dotQ8_0 == sum(dequant * vec) within 1e-3
    data, vec = _q8_two_blocks()
    dec = orc.dequant(orc.Q8_0, data, 64)
    expected = np.float32(0)
    for d, v in zip(dec, vec):
        expected = np.float32(expected + np.float32(d * v))
    assert abs(orc.dot_q8_0(data, vec) - expected) <= 1e-3
    # float64 brute force
    exact = float(np.dot(dec.astype(np.float64), vec.astype(np.float64)))
    assert abs(orc.dot_q8_0(data, vec) - exact) <= 1e-4 * max(1.0, abs(exact))


def test_dot_q8_0_scale_after_block_sum():
    # dequant.zig:75: total += reduce(acc) * d -- d multiplies the block sum,
    # not each element.  With d = 1.5 (exact) and q*x chosen so the
    # block sum is 2^24 + 2 (representable) but per-element products are not
    # summed the same way, the two orders give different fp32 results.
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3E]  # f16 1.5
    q = np.zeros(32, dtype=np.int8)
    q[0], q[8] = 1, 1
    blk[2:] = q.view(np.uint8)
    x = np.zeros(32, dtype=np.float32)
    x[0], x[8] = np.float32(2.0 ** 24), np.float32(3.0)
    # lane 0 accumulates x[0] then x[8]: 2^24 + 3 -> 16777220 (RNE), * 1.5 = 25165830
    acc = np.float32(np.float32(2.0 ** 24) + np.float32(3.0))
    assert orc.dot_q8_0(blk, x) == np.float32(acc * np.float32(1.5))


def test_q8_0_gpu_kat_identity_rows():
    # gpu/matvec.zig:3728-3767: 32 rows, d = 1, qs[row] = 1, vec = 1..32 -> i+1
    mat = np.zeros((32, 34), dtype=np.uint8)
    mat[:, 1] = 0x3C
    for r in range(32):
        mat[r, 2 + r] = 1
    vec = np.arange(1, 33, dtype=np.float32)
    out = orc.quant_matvec(mat, orc.Q8_0, vec, 32, 32)
    assert out.tolist() == [float(i + 1) for i in range(32)]


# ---------------------------------------------------------------- Q4_K
def q4k_decode_np(blocks: np.ndarray) -> np.ndarray:
    """Independent Q4_K decoder (ggml block_q4_K layout), float32 math:
    value = (d * sc) * q - (dmin * mn)."""
    blocks = blocks.reshape(-1, 144)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = ggml.unpack_q4k_scales(blocks[:, 4:16])
    qs = blocks[:, 16:]
    out = np.empty((blocks.shape[0], 256), dtype=np.float32)
    for p in range(4):
        byte = qs[:, 32 * p:32 * p + 32]
        for half, q in ((0, byte & 15), (1, byte >> 4)):
            j = 2 * p + half
            scale = (d * sc[:, j].astype(np.float32)).astype(np.float32)
            mins = (dmin * mn[:, j].astype(np.float32)).astype(np.float32)
            out[:, 64 * p + 32 * half:64 * p + 32 * half + 32] = (scale[:, None] * q.astype(np.float32)) - mins[:, None]
    return out.reshape(-1)


def test_q4k_zero_block():
    # dequant.zig:760-766
    assert not orc.dequant(orc.Q4_K, np.zeros(144, dtype=np.uint8), 256).any()


def test_q4k_gpu_kat_scale():
    # gpu/matvec.zig:3877-3908: d = 1, sc[0] = 1, qs[0..31] = 0x11, vec = 1 -> 32.0
    blk = np.zeros(144, dtype=np.uint8)
    blk[1] = 0x3C
    blk[4] = 1
    blk[16:48] = 0x11
    assert orc.quant_matvec(blk, orc.Q4_K, np.ones(256, np.float32), 1, 256)[0] == 32.0


def test_q4k_gpu_kat_min():
    # gpu/matvec.zig:3910-3939: dmin = 1, mn[0] = 2, qs = 0, vec = 1 -> -64.0
    blk = np.zeros(144, dtype=np.uint8)
    blk[3] = 0x3C
    blk[8] = 2
    assert orc.quant_matvec(blk, orc.Q4_K, np.ones(256, np.float32), 1, 256)[0] == -64.0


def test_q4k_scale_pack_roundtrip():
    g = np.random.default_rng(5)
    sc = g.integers(0, 64, (500, 8), dtype=np.uint8)
    mn = g.integers(0, 64, (500, 8), dtype=np.uint8)
    s2, m2 = ggml.unpack_q4k_scales(ggml.pack_q4k_scales(sc, mn))
    assert np.array_equal(s2, sc) and np.array_equal(m2, mn)


def test_q4k_matches_independent_decoder():
    g = np.random.default_rng(11)
    blocks = g.integers(0, 256, (64, 144), dtype=np.uint8)
    blocks[:, 0:2] = ggml.f16_bits(np.abs(g.standard_normal(64)) * 0.01).view(np.uint8).reshape(64, 2)
    blocks[:, 2:4] = ggml.f16_bits(np.abs(g.standard_normal(64)) * 0.01).view(np.uint8).reshape(64, 2)
    got = orc.dequant(orc.Q4_K, blocks, 64 * 256)
    assert np.array_equal(got.view(np.uint32), q4k_decode_np(blocks).view(np.uint32))


def test_q4k_single_element_probes():
    # one nonzero nibble at a time lands on the element the ggml layout says
    for j, (p, half, i) in enumerate([(0, 0, 0), (0, 1, 5), (2, 0, 31), (3, 1, 17)]):
        blk = np.zeros(144, dtype=np.uint8)
        blk[1] = 0x3C  # d = 1
        sc = np.zeros(8, np.uint8)
        sc[2 * p + half] = 3
        blk[4:16] = ggml.pack_q4k_scales(sc, np.zeros(8, np.uint8))
        blk[16 + 32 * p + i] = (5 << 4) if half else 5
        out = orc.dequant(orc.Q4_K, blk, 256)
        idx = 64 * p + 32 * half + i
        assert out[idx] == 15.0 and np.count_nonzero(out) == 1, j


# ---------------------------------------------------------------- Q6_K
def q6k_decode_np(blocks: np.ndarray) -> np.ndarray:
    """Independent Q6_K decoder (ggml block_q6_K layout), float32 math:
    value = (d * sc) * (q - 32)."""
    blocks = blocks.reshape(-1, 210)
    ql, qh = blocks[:, 0:128], blocks[:, 128:192]
    sc = blocks[:, 192:208].view(np.int8).astype(np.float32)
    d = blocks[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    out = np.empty((blocks.shape[0], 256), dtype=np.float32)
    for e in range(256):
        hf, r = divmod(e, 128)
        grp, l = divmod(r, 32)
        lo_src = ql[:, 64 * hf + l + (32 if grp in (1, 3) else 0)]
        lo = (lo_src >> 4) if grp >= 2 else (lo_src & 15)
        hi = (qh[:, 32 * hf + l] >> (2 * grp)) & 3
        q = (lo | (hi << 4)).astype(np.int32) - 32
        s = (d * sc[:, 8 * hf + l // 16 + 2 * grp]).astype(np.float32)
        out[:, e] = s * q.astype(np.float32)
    return out.reshape(-1)


def test_q6k_matches_independent_decoder():
    g = np.random.default_rng(13)
    blocks = g.integers(0, 256, (32, 210), dtype=np.uint8)
    blocks[:, 208:210] = ggml.f16_bits(np.abs(g.standard_normal(32)) * 0.01).view(np.uint8).reshape(32, 2)
    got = orc.dequant(orc.Q6_K, blocks, 32 * 256)
    assert np.array_equal(got.view(np.uint32), q6k_decode_np(blocks).view(np.uint32))


def test_q6k_special_values():
    blk = np.zeros(210, dtype=np.uint8)
    blk[208:210] = [0x00, 0x3C]  # d = 1
    blk[192:208] = 1
    # q = 0 everywhere -> value = -32 ; set element 0 to q = 32 (ql lo = 0, qh bits = 2) -> 0
    blk[128] = 0b10
    out = orc.dequant(orc.Q6_K, blk, 256)
    assert out[0] == 0.0 and np.all(out[1:] == -32.0)
    blk[192:208] = 0  # zero scales -> all zero
    assert not orc.dequant(orc.Q6_K, blk, 256).any()


# ---------------------------------------------------------------- dotf32
def test_dotf32_kat_lengths():
    # ops/math.zig:401-413
    for n in (1, 7, 8, 32, 33):
        a = (np.arange(1, n + 1, dtype=np.float32) * np.float32(0.5)).astype(np.float32)
        b = (np.arange(n, 0, -1, dtype=np.float32) * np.float32(0.3)).astype(np.float32)
        exp = np.float32(0)
        for i in range(n):
            exp = np.float32(exp + np.float32(a[i] * b[i]))
        assert abs(orc.dotf32(a, b) - exp) <= 1e-4


def test_dotf32_accumulator_grouping():
    # acc[l] = (acc0[l] + acc1[l]) + (acc2[l] + acc3[l]) (math.zig:109):
    # lane 0 gets 2^24, 1, 1, -2^24 from the four accumulators:
    # (2^24 + 1) + (1 - 2^24) = 2^24 + (-16777215) = 1 in fp32, whereas a
    # sequential sum gives 0 and a different pairing gives 2.
    a = np.zeros(32, np.float32)
    b = np.ones(32, np.float32)
    a[0], a[8], a[16], a[24] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    assert orc.dotf32(a, b) == 1.0


def test_dotf32_ordered_lane_reduce():
    # @reduce(.Add) in strict mode is ordered (math.zig:113):
    # ((2^24 + 1) + 1) - 2^24 = 0, a pairwise tree would give 1.
    a = np.zeros(8, np.float32)
    a[0:4] = [2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)]
    assert orc.dotf32(a, np.ones(8, np.float32)) == 0.0


def test_dotf32_tail_after_reduce():
    # scalar tail (math.zig:114) is added after the lane reduce:
    # lanes sum to 2^24, then + 1 (lost) + 1 (lost) = 2^24
    a = np.zeros(10, np.float32)
    a[0], a[8], a[9] = 2.0 ** 24, 1.0, 1.0
    assert orc.dotf32(a, np.ones(10, np.float32)) == np.float32(2.0 ** 24)


def test_dotf32_vs_float64():
    g = np.random.default_rng(3)
    for n in (5, 64, 100, 2048, 2051):
        a = g.standard_normal(n).astype(np.float32)
        b = g.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert abs(float(orc.dotf32(a, b)) - exact) <= 1e-5 * math.sqrt(n) * np.linalg.norm(a) * np.linalg.norm(b) / n + 1e-6


def test_quant_matvec_f32_matches_matvec():
    # ops/math.zig:173-191
    mat = np.array([[1.0, -2.0, 0.5, 4.0, -1.0], [0.25, 3.0, 2.0, -0.5, 1.5], [-1.0, 0.0, 0.0, 2.0, 3.0]],
                   dtype=np.float32)
    vec = np.array([0.5, -1.0, 2.0, 0.25, -0.75], dtype=np.float32)
    got = orc.quant_matvec(mat, orc.F32, vec, 3, 5)
    assert np.allclose(got, orc.matvec_f32(mat, vec), atol=1e-6)


def test_matvec_kats():
    # ops/math.zig:324-342
    assert orc.matvec_f32(np.eye(3, dtype=np.float32), np.array([1, 2, 3], np.float32)).tolist() == [1, 2, 3]
    assert orc.matvec_f32(np.array([[2, 0], [0, 3]], np.float32), np.array([4, 5], np.float32)).tolist() == [8, 15]


@pytest.mark.parametrize("gtype", [orc.Q8_0, orc.Q4_K, orc.Q6_K])
def test_quant_matvec_par_thread_invariant(gtype):
    # row-split parallelism computes each row identically (math.zig:277-320)
    g = synth.stream(99, gtype)
    rows, cols = 700, 512
    mat = {orc.Q8_0: synth.q8_0_matrix, orc.Q4_K: synth.q4k_matrix, orc.Q6_K: synth.q6k_matrix}[gtype](g, rows, cols)
    x = synth.normal(g, (cols,))
    ref = orc.quant_matvec(mat, gtype, x, rows, cols)
    for nt in (1, 3, 8):
        with orc.Pool(nt) as p:
            got = orc.quant_matvec(mat, gtype, x, rows, cols, pool=p)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), nt


@pytest.mark.parametrize("gtype", [orc.Q8_0, orc.Q4_K, orc.Q6_K])
def test_quant_matvec_vs_float64(gtype):
    g = synth.stream(98, gtype)
    rows, cols = 64, 1024
    mat = {orc.Q8_0: synth.q8_0_matrix, orc.Q4_K: synth.q4k_matrix, orc.Q6_K: synth.q6k_matrix}[gtype](g, rows, cols)
    x = synth.normal(g, (cols,))
    if gtype == orc.Q4_K:
        dense = q4k_decode_np(mat).reshape(rows, cols)
    elif gtype == orc.Q6_K:
        dense = q6k_decode_np(mat).reshape(rows, cols)
    else:
        blk = mat.reshape(rows, -1, 34)
        d = blk[..., 0:2].copy().view(np.float16).astype(np.float64)
        dense = (blk[..., 2:].view(np.int8).astype(np.float64) * d).reshape(rows, cols)
    want = dense.astype(np.float64) @ x.astype(np.float64)
    got = orc.quant_matvec(mat, gtype, x, rows, cols)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


# ---------------------------------------------------------------- softmax / act
def test_softmax_kats():
    # ops/math.zig:378-393
    s = orc.softmax([1.0, 2.0, 3.0])
    assert abs(float(s.sum()) - 1.0) < 1e-6 and s[2] > s[1] > s[0]
    s = orc.softmax([1000.0, 1001.0, 1002.0])
    assert abs(float(s.sum()) - 1.0) < 1e-5
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    assert np.allclose(orc.softmax([1.0, 2.0, 3.0]), e / e.sum(), rtol=1e-6)


def test_silu_gelu_closed_forms():
    # math.zig:395-399 and the closed forms in float64
    assert orc.silu(0.0) == 0.0 and 0.0 < orc.silu(1.0) < 1.0
    for x in np.linspace(-8, 8, 161):
        xf = float(np.float32(x))
        assert abs(orc.silu(xf) - xf / (1 + math.exp(-xf))) <= 1e-6 * max(1, abs(xf))
        gel = 0.5 * xf * (1 + math.tanh(math.sqrt(2 / math.pi) * (xf + 0.044715 * xf ** 3)))
        assert abs(orc.gelu(xf) - gel) <= 2e-6 * max(1, abs(xf))


# ---------------------------------------------------------------- top-k / router
def test_topk_ties_kat():
    # gemma4/forward.zig:823-829 and the same rule in ops/moe.zig:80-91
    scores = [1.0, 4.0, 4.0, -2.0, 3.5, 4.0, 0.0]
    assert orc.topk_softmax_stats(scores, 4)[0].tolist() == [1, 2, 5, 4]
    assert orc.topk(scores, 4).tolist() == [1, 2, 5, 4]


def test_topk_softmax_stats_kat():
    # gemma4/forward.zig:831-845
    scores = np.array([-3.0, 0.5, 7.0, 2.0, 6.5, -1.0], np.float32)
    _, mx, es = orc.topk_softmax_stats(scores, 3)
    assert mx == 7.0
    assert abs(es - float(np.exp(scores.astype(np.float64) - 7.0).sum())) <= 1e-6 * es


def test_softmax_topk_kat():
    # gemma4/forward.zig:847-861
    ref = np.array([0.5, 4.0, -1.0, 2.5, 3.0, -0.25], np.float32)
    sm = orc.softmax(ref)
    ref_idx = orc.topk(sm, 3)
    got_idx, got = orc.softmax_topk(ref, 3)
    assert got_idx.tolist() == ref_idx.tolist()
    for i in got_idx:
        assert abs(got[i] - sm[i]) <= 1e-6


def test_topk_matvec_f32_kat():
    # gemma4/forward.zig:863-891
    w = np.array([[1.0, -2.0, 0.5, 4.0, -1.0], [0.25, 3.0, 2.0, -0.5, 1.5], [-1.0, 0.0, 0.0, 2.0, 3.0],
                  [2.5, -1.5, 0.25, 0.0, 1.0], [0.0, 0.5, -2.0, 1.0, 2.0], [1.25, -0.25, 1.5, -2.0, 0.75]],
                 np.float32)
    vec = np.array([0.5, -1.0, 2.0, 0.25, -0.75], np.float32)
    logits = orc.matvec_f32(w, vec)
    ref_idx, ref = orc.softmax_topk(logits, 3)
    idx, sel, mx, es = orc.topk_matvec_f32(w, vec, 3)
    assert idx.tolist() == ref_idx.tolist()
    for j, r in enumerate(idx):
        assert abs(logits[r] - sel[j]) <= 1e-6
        assert abs(ref[r] - math.exp(sel[j] - mx) / es) <= 1e-6


def test_topk_matvec_f32_par_kat(pool):
    # gemma4/forward.zig:893-922 (37 x 33 integer pattern, k = 8, 4 threads)
    i = np.arange(37 * 33)
    w = (((i * 17 + 11) % 23 - 9) * 0.125).astype(np.float32).reshape(37, 33)
    j = np.arange(33)
    vec = (((j * 13 + 7) % 19 - 8) * 0.2).astype(np.float32)
    ri, rs, rmax, res = orc.topk_matvec_f32(w, vec, 8)
    with orc.Pool(4) as p4:
        gi, gs, gmax, ges = orc.topk_matvec_f32(w, vec, 8, pool=p4)
    assert rmax == gmax and abs(res - ges) <= 1e-6 * res
    assert ri.tolist() == gi.tolist()
    assert np.allclose(rs, gs, atol=1e-6)


def test_router_topk_softmax_kat(pool):
    # gemma4/forward.zig:924-960
    w = np.array([[0.5, -1.0, 1.5, 0.25], [2.0, 0.0, -0.5, 1.0], [-1.0, 2.0, 0.5, -0.25], [1.25, -0.75, 0.0, 2.0],
                  [0.0, 0.25, 1.0, -1.5]], np.float32)
    vec = np.array([1.0, -0.5, 0.75, 2.0], np.float32)
    ref_scores = orc.quant_matvec(w, orc.F32, vec, 5, 4)
    ref_idx, ref = orc.softmax_topk(ref_scores, 2)
    idx, scores = orc.router_topk_softmax(w, orc.F32, 5, 4, vec, 2, pool=pool)
    assert idx.tolist() == ref_idx.tolist()
    for e in idx:
        assert abs(ref[e] - scores[e]) <= 1e-6


def test_router_gpu_kat_ids_and_scales():
    # gpu/matvec.zig:3582-3656 without the norm: router_in = ones(8), rows
    # [0, 1, 0.5, 1] * ones -> logits [0, 8, 4, 8] -> ids [1, 3],
    # p = e^8 / (2 e^8 + e^4 + 1) (the KAT's down_scale factors set to 1)
    w = np.zeros((4, 8), np.float32)
    w[1], w[2], w[3] = 1.0, 0.5, 1.0
    idx, scores = orc.router_topk_softmax(w, orc.F32, 4, 8, np.ones(8, np.float32), 2)
    assert idx.tolist() == [1, 3]
    p = math.exp(8) / (2 * math.exp(8) + math.exp(4) + 1)
    assert abs(scores[1] - p) <= 1e-6 and abs(scores[3] - p) <= 1e-6


# ---------------------------------------------------------------- MoE composition
def _moe_f64(w, x, k, act, norm, bias=None):
    """float64 restatement of moeForward from the independent decoders."""
    E, D, F, Kd = w.n_experts, w.d_model, w.d_expert, w.down_cols
    logits = w.router.astype(np.float64) @ x.astype(np.float64)
    if bias is not None:
        logits = logits + bias
    p = np.exp(logits - logits.max())
    p /= p.sum()
    order = sorted(range(E), key=lambda e: (-p[e], e))[:k]
    wt = np.array([p[e] for e in order])
    if norm:
        wt = wt / wt.sum()
    gu = q4k_decode_np(w.gate_up).reshape(E, 2 * F, D).astype(np.float64)
    dn = q4k_decode_np(w.down).reshape(E, D, Kd).astype(np.float64)
    out = np.zeros(D)
    for e, we in zip(order, wt):
        g, u = gu[e, :F] @ x, gu[e, F:] @ x
        a = g / (1 + np.exp(-g)) if act == orc.ACT_SILU else \
            0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
        h = np.zeros(Kd)
        h[:F] = a * u
        out += we * (dn[e] @ h)
    return out, order, wt


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("act", [orc.ACT_SILU, orc.ACT_GELU_TANH])
def test_moe_forward_vs_float64(norm, act, pool):
    w = synth.moe_weights(90, 256, 12, 192, down_cols=256)
    x = synth.normal(synth.stream(90, 7), (256,))
    bias = synth.zipf_bias(synth.stream(90, 8), 12)
    got, ids, wt, agree = orc.moe_forward(w, x, 3, act=act, norm_topk=norm, bias=bias, pool=pool)
    want, order, wwant = _moe_f64(w, x, 3, act, norm, bias)
    assert agree
    assert ids.tolist() == order
    assert np.allclose(wt, wwant, rtol=1e-5)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-5
    if norm:
        assert abs(float(wt.astype(np.float64).sum()) - 1.0) < 1e-6


def test_moe_f64_check_has_teeth(pool):
    # A plausible mistake (gate and up halves swapped) must fail the check.
    w = synth.moe_weights(91, 256, 8, 256)
    x = synth.normal(synth.stream(91, 7), (256,))
    want, _, _ = _moe_f64(w, x, 2, orc.ACT_SILU, False)
    F = w.d_expert
    bad = synth.MoEWeights(**{**w.__dict__})
    gu = w.gate_up.reshape(w.n_experts, 2 * F, -1)
    bad.gate_up = np.concatenate([gu[:, F:], gu[:, :F]], axis=1).reshape(w.gate_up.shape)
    got, *_ = orc.moe_forward(bad, x, 2, pool=pool)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) > 1e-2


def test_moe_forward_thread_invariant():
    w = synth.moe_weights(92, 512, 16, 256)
    x = synth.normal(synth.stream(92, 7), (512,))
    ref = orc.moe_forward(w, x, 4)[0]
    for nt in (2, 7):
        with orc.Pool(nt) as p:
            assert np.array_equal(orc.moe_forward(w, x, 4, pool=p)[0], ref)


def q8_0_decode_np(mat: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Independent Q8_0 decoder (ggml block layout: f16 d, then 32 int8 q;
    value = d * q), float64, [rows, cols]."""
    blk = mat.reshape(rows, cols // 32, 34)
    d = blk[..., 0:2].copy().view(np.float16).astype(np.float64)
    return (blk[..., 2:].view(np.int8).astype(np.float64) * d).reshape(rows, cols)


def _act_f64(act, g):
    if act == orc.ACT_SILU:
        return g / (1 + np.exp(-g))
    return 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))


def _ffn_dense_f64(wg, wu, wd, x, d_model, d_ffn, act, act_on_up=False):
    """float64 restatement of the dense gated FFN: h = act(Wg x) * (Wu x),
    out = Wd h (model/forward.zig:304-307 with SiLU; gemma4/forward.zig:
    392-397 with GELU-tanh).  act_on_up plants a mistake for the teeth test."""
    g = q8_0_decode_np(wg, d_ffn, d_model) @ x.astype(np.float64)
    u = q8_0_decode_np(wu, d_ffn, d_model) @ x.astype(np.float64)
    h = g * _act_f64(act, u) if act_on_up else _act_f64(act, g) * u
    return q8_0_decode_np(wd, d_model, d_ffn) @ h


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("act", [orc.ACT_SILU, orc.ACT_GELU_TANH])
@pytest.mark.parametrize("shape", [(896, 4864), (512, 320)])
def test_ffn_dense_vs_float64(act, shape, pool):
    # lto_ffn_dense against the float64 restatement on the independent Q8_0
    # decoder; (896, 4864) is config 1's Qwen2.5-0.5B shape.
    d_model, d_ffn = shape
    g = synth.stream(95, d_ffn)
    wg, wu = synth.q8_0_matrix(g, d_ffn, d_model), synth.q8_0_matrix(g, d_ffn, d_model)
    wd = synth.q8_0_matrix(g, d_model, d_ffn)
    x = synth.normal(g, (d_model,))
    got = orc.ffn_dense(wg, wu, wd, orc.Q8_0, x, d_model, d_ffn, act=act, pool=pool)
    assert _rel(got, _ffn_dense_f64(wg, wu, wd, x, d_model, d_ffn, act)) < 1e-5


def test_ffn_dense_f64_check_has_teeth(pool):
    # Each plausible misreading of model/forward.zig:304-307 must fail the
    # 1e-5 check above by a wide margin (> 1e-3): gate and up swapped, the
    # activation applied to up, and GELU-tanh where SiLU is asked for (or the
    # reverse; the two differ least, ~5e-3 on these inputs).
    d_model, d_ffn = 512, 320
    g = synth.stream(96, 1)
    wg, wu = synth.q8_0_matrix(g, d_ffn, d_model), synth.q8_0_matrix(g, d_ffn, d_model)
    wd = synth.q8_0_matrix(g, d_model, d_ffn)
    x = synth.normal(g, (d_model,))
    for act, other in ((orc.ACT_SILU, orc.ACT_GELU_TANH), (orc.ACT_GELU_TANH, orc.ACT_SILU)):
        want = _ffn_dense_f64(wg, wu, wd, x, d_model, d_ffn, act)
        swapped = orc.ffn_dense(wu, wg, wd, orc.Q8_0, x, d_model, d_ffn, act=act, pool=pool)
        assert _rel(swapped, want) > 1e-3
        right = orc.ffn_dense(wg, wu, wd, orc.Q8_0, x, d_model, d_ffn, act=act, pool=pool)
        act_on_up = _ffn_dense_f64(wg, wu, wd, x, d_model, d_ffn, act, act_on_up=True)
        assert _rel(right, act_on_up) > 1e-3
        wrong_act = orc.ffn_dense(wg, wu, wd, orc.Q8_0, x, d_model, d_ffn, act=other, pool=pool)
        assert _rel(wrong_act, want) > 1e-3


def test_moe_layer_shared_composition(pool):
    # Config-4 layer = shared dense FFN + routerTopKSoftmax(Q8_0) + expert loop
    # (gemma4/forward.zig:392-398, 417, 463-479), every term from float64
    # restatements on the independent decoders.
    w = synth.moe_weights(93, 512, 8, 192, down_cols=256, router_type=ggml.Q8_0)
    x = synth.normal(synth.stream(93, 7), (512,))
    shg = synth.q8_0_matrix(synth.stream(93, 20), 320, 512)
    shu = synth.q8_0_matrix(synth.stream(93, 21), 320, 512)
    shd = synth.q8_0_matrix(synth.stream(93, 22), 512, 320)
    out, ids, wt = orc.moe_layer_shared(w, x, 2, shg, shu, shd, 320, pool=pool)
    shared = _ffn_dense_f64(shg, shu, shd, x, 512, 320, orc.ACT_GELU_TANH)
    logits = q8_0_decode_np(w.router, 8, 512) @ x.astype(np.float64)
    p = np.exp(logits - logits.max())
    p /= p.sum()
    order = sorted(range(8), key=lambda e: (-p[e], e))[:2]
    assert ids.tolist() == order
    assert np.allclose(wt, p[order], rtol=1e-5)
    gu = q4k_decode_np(w.gate_up).reshape(8, 384, 512).astype(np.float64)
    dn = q4k_decode_np(w.down).reshape(8, 512, 256).astype(np.float64)
    moe = np.zeros(512)
    for e, we in zip(order, p[order]):
        g, u = gu[e, :192] @ x, gu[e, 192:] @ x
        h = np.zeros(256)
        h[:192] = _act_f64(orc.ACT_GELU_TANH, g) * u
        moe += we * (dn[e] @ h)
    want = shared + moe
    assert _rel(out, want) < 1e-5


def test_moe_prefill_is_per_token(pool):
    w = synth.moe_weights(94, 256, 8, 256)
    X = synth.normal(synth.stream(94, 7), (5, 256))
    out, ids, wt = orc.moe_prefill(w, X, 2, norm_topk=True, pool=pool)
    for t in range(5):
        o, i, ww, _ = orc.moe_forward(w, X[t], 2, norm_topk=True, pool=pool)
        assert np.array_equal(out[t], o) and np.array_equal(ids[t], i) and np.array_equal(wt[t], ww)
