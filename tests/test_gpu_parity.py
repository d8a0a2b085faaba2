"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars: expert ids bit-exact; outputs within 1e-3
relative L2 of the oracle (fp32 accumulation); router logits bit-exact.
Matvec fuzz cases also hold the reference's own fuzz bound,
max|d| / max|ref| < 1e-4 for fp32 activations (gpu/matvec.zig:4618).
"""
import dataclasses
import os
import sys

import numpy as np
import pytest

import llmtoy_amd as lt
import pyoracle as orc
from llmtoy_amd import ggml, synth
from llmtoy_amd.lib import DeviceError, InvalidError, UnsupportedError

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

REL_L2 = 1e-3
FUZZ_MAX_REL = 1e-4


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / (np.max(np.abs(b)) + 1e-6))


def gpu_matvec(ctx, w, gtype, rows, cols, x, n_experts=1):
    t = ctx.upload(w, gtype, rows, cols, n_experts)
    y = np.zeros(rows * n_experts, np.float32)
    ctx.quant_matvec(y, t, x)
    t.free()
    return y


# ------------------------------------------------------------------ KATs
def test_gpu_matvec_q8_0_identity_rows(ctx):
    # gpu/matvec.zig:3728-3767
    mat = np.zeros((32, 34), np.uint8)
    mat[:, 1] = 0x3C
    for r in range(32):
        mat[r, 2 + r] = 1
    y = gpu_matvec(ctx, mat, ggml.Q8_0, 32, 32, np.arange(1, 33, dtype=np.float32))
    assert y.tolist() == [float(i + 1) for i in range(32)]


def test_gpu_matvec_q4k_scale(ctx):
    # gpu/matvec.zig:3877-3908
    blk = np.zeros(144, np.uint8)
    blk[1], blk[4] = 0x3C, 1
    blk[16:48] = 0x11
    assert gpu_matvec(ctx, blk, ggml.Q4_K, 1, 256, np.ones(256, np.float32))[0] == pytest.approx(32.0, abs=1e-4)


def test_gpu_matvec_q4k_min(ctx):
    # gpu/matvec.zig:3910-3939
    blk = np.zeros(144, np.uint8)
    blk[3], blk[8] = 0x3C, 2
    assert gpu_matvec(ctx, blk, ggml.Q4_K, 1, 256, np.ones(256, np.float32))[0] == pytest.approx(-64.0, abs=1e-4)


def test_gpu_f16_subnormal_scales(ctx):
    # f16 subnormals are kept (quant/dequant.zig:302-305); a flush-to-zero
    # conversion would return 0 here.
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x01, 0x00]  # d = 2^-24
    blk[2:4] = [0xFF, 0x03]  # dmin = 1023 * 2^-24
    blk[4:16] = ggml.pack_q4k_scales(np.full(8, 63, np.uint8), np.full(8, 1, np.uint8))
    blk[16:] = 0xFF
    x = np.ones(256, np.float32)
    y = gpu_matvec(ctx, blk, ggml.Q4_K, 1, 256, x)[0]
    ref = orc.quant_matvec(blk, orc.Q4_K, x, 1, 256)[0]
    assert ref != 0 and abs(y - ref) <= 1e-6 * abs(ref)
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = [0x00, 0x02]  # 512 * 2^-24
    q8[2:] = 100
    y8 = gpu_matvec(ctx, q8, ggml.Q8_0, 1, 32, np.ones(32, np.float32))[0]
    assert y8 == np.float32(orc.quant_matvec(q8, orc.Q8_0, np.ones(32, np.float32), 1, 32)[0]) != 0


def test_gpu_router_kat(ctx):
    # gpu/matvec.zig:3582-3656 (no norm): logits [0, 8, 4, 8] -> ids [1, 3]
    w = np.zeros((4, 8), np.float32)
    w[1], w[2], w[3] = 1.0, 0.5, 1.0
    r = ctx.upload(w, ggml.F32, 4, 8)
    ids = np.zeros(2, np.uint32)
    wt = np.zeros(2, np.float32)
    ctx.router_topk(r, np.ones(8, np.float32), 2, ids, wt)
    assert ids.tolist() == [1, 3]
    p = np.exp(8.0) / (2 * np.exp(8.0) + np.exp(4.0) + 1)
    assert np.allclose(wt, [p, p], atol=1e-6)


def test_gpu_topk_tie_kat(ctx):
    # gemma4/forward.zig:823-829 ties: {1,4,4,-2,3.5,4,0} -> [1,2,5,4]
    logits = np.array([1.0, 4.0, 4.0, -2.0, 3.5, 4.0, 0.0], np.float32)
    r = ctx.upload(np.diag(logits).astype(np.float32), ggml.F32, 7, 7)
    ids = np.zeros(4, np.uint32)
    ctx.router_topk(r, np.ones(7, np.float32), 4, ids, np.zeros(4, np.float32))
    assert ids.tolist() == [1, 2, 5, 4]


# ------------------------------------------------------------------ fuzz (reference style)
@pytest.mark.parametrize("gtype,rows,cols,seed", [
    (ggml.Q8_0, 32, 256, 1), (ggml.Q4_K, 32, 256, 3), (ggml.Q4_K, 64, 2048, 11), (ggml.Q4_K, 19, 4096, 13),
    (ggml.Q6_K, 32, 256, 5), (ggml.Q6_K, 37, 1024, 17), (ggml.Q8_0, 33, 4864, 19), (ggml.Q4_K, 70, 768, 23)])
def test_gpu_matvec_fuzz(ctx, gtype, rows, cols, seed):
    # gpu/matvec.zig:4543-4619: random bytes with every f16 super-scale stamped
    # to 0x21CD (~0.012), x ~ U(-1, 1), max|d|/max|ref| < 1e-4.
    g = np.random.default_rng(seed)
    rb = ggml.row_bytes(gtype, cols)
    mat = g.integers(0, 256, (rows, rb), dtype=np.uint8)
    bb = ggml.BLOCK_BYTES[gtype]
    blk = mat.reshape(rows, -1, bb)
    if gtype == ggml.Q6_K:
        blk[..., 208], blk[..., 209] = 0xCD, 0x21
    else:
        blk[..., 0], blk[..., 1] = 0xCD, 0x21
        if gtype == ggml.Q4_K:
            blk[..., 2], blk[..., 3] = 0xCD, 0x21
    x = ((g.random(cols, dtype=np.float32) - 0.5) * 2).astype(np.float32)
    y = gpu_matvec(ctx, mat, gtype, rows, cols, x)
    ref = orc.quant_matvec(mat, gtype, x, rows, cols)
    assert max_rel(y, ref) < FUZZ_MAX_REL


@pytest.mark.parametrize("rows,cols", [(37, 33), (128, 2048), (5, 4), (200, 2816)])
def test_gpu_matvec_f32_bit_exact(ctx, rows, cols):
    # fp32 rows follow dotf32's order exactly (ops/math.zig:96-116)
    g = np.random.default_rng(rows * cols)
    w = g.standard_normal((rows, cols)).astype(np.float32)
    x = g.standard_normal(cols).astype(np.float32)
    y = gpu_matvec(ctx, w, ggml.F32, rows, cols, x)
    ref = orc.quant_matvec(w, orc.F32, x, rows, cols)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ upload / read-back
# Uploads move GGUF blocks through pinned 4 MiB pieces (several in flight)
# and split them into planes on the device; reading back joins them again.
# Sizes cover one block, ragged workgroup tails, one piece exactly and
# more pieces than in-flight workers.
@pytest.mark.parametrize("gtype,blocks", [
    (ggml.Q8_0, 1), (ggml.Q8_0, 65), (ggml.Q8_0, 123328), (ggml.Q8_0, 8 * 123328 + 777),
    (ggml.Q4_K, 1), (ggml.Q4_K, 63), (ggml.Q4_K, 29120), (ggml.Q4_K, 29121), (ggml.Q4_K, 20 * 29120 + 5),
    (ggml.Q6_K, 3), (ggml.Q6_K, 19968 + 64), (ggml.Q6_K, 17 * 19968 + 1),
    (ggml.F32, 1), (ggml.F32, 1048576 + 3), (ggml.F32, 9 * 1048576)])
def test_gpu_upload_read_round_trip(ctx, gtype, blocks):
    g = np.random.default_rng(blocks * 31 + gtype)
    data = g.integers(0, 256, blocks * ggml.BLOCK_BYTES[gtype], dtype=np.uint8)
    cols = ggml.BLOCK_ELEMS[gtype]
    print(f"upload round trip type {gtype} blocks {blocks}", flush=True)
    t = ctx.upload(data, gtype, blocks, cols)
    back = t.read()
    t.free()
    assert np.array_equal(back, data)


def test_gpu_upload_read_config3_experts(ctx, cfg3):
    # the full 340 MB expert tensors of the headline layer
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    assert np.array_equal(gate_up.read(), w.gate_up.reshape(-1))
    assert np.array_equal(down.read(), w.down.reshape(-1))
    assert np.array_equal(router.read().view(np.float32), w.router.reshape(-1))


def test_gpu_read_rejects_wrong_size(ctx):
    t = ctx.upload(np.zeros(34, np.uint8), ggml.Q8_0, 1, 32)
    buf = np.zeros(33, np.uint8)
    with pytest.raises(InvalidError):
        ctx._check(ctx.lib.lt_tensor_read(ctx.ptr, t.handle, buf.ctypes.data, buf.nbytes))
    t.free()


# ------------------------------------------------------------------ golden fixtures
@pytest.mark.parametrize("name", ["mv_f32", "mv_q8_0", "mv_q4_k", "mv_q4_k_pad", "mv_q6_k_pad"])
def test_gpu_golden_matvec(ctx, name):
    gold = np.load(os.path.join(HERE, "golden", "golden.npz"))
    w, x, y = gold[f"{name}.w"], gold[f"{name}.x"], gold[f"{name}.y"]
    gtype = {"mv_f32": ggml.F32, "mv_q8_0": ggml.Q8_0, "mv_q6_k_pad": ggml.Q6_K}.get(name, ggml.Q4_K)
    rows = w.shape[0]
    cols = x.shape[0]
    got = gpu_matvec(ctx, np.ascontiguousarray(w), gtype, rows, cols, x)
    if gtype == ggml.F32:
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32))
    else:
        assert rel_l2(got, y) <= REL_L2


@pytest.mark.parametrize("name", ["moe_small", "moe_small_norm_bias_gelu"])
def test_gpu_golden_moe(ctx, name):
    gold = np.load(os.path.join(HERE, "golden", "golden.npz"))
    builder, _ = make_golden.cases()[name]
    d = builder()
    w = d["w"]
    k = gold[f"{name}.ids"].size
    act = lt.ACT_GELU_TANH if "gelu" in name else lt.ACT_SILU
    router, gate_up, down = lt.upload_moe(ctx, w)
    out = np.zeros(w.d_model, np.float32)
    ids = np.zeros(k, np.uint32)
    wt = np.zeros(k, np.float32)
    ctx.moe_forward(out, d["x"], router, gate_up, down, k, w.d_expert, act=act, norm_topk="norm" in name,
                    bias=d["bias"], out_ids=ids, out_w=wt)
    assert np.array_equal(ids, gold[f"{name}.ids"])
    assert np.allclose(wt, gold[f"{name}.wt"], rtol=1e-5)
    assert rel_l2(out, gold[f"{name}.out"]) <= REL_L2
    for t in (router, gate_up, down):
        t.free()


# ------------------------------------------------------------------ BASELINE configs
def test_gpu_config2_q4k_4096(ctx):
    c = synth.config2()
    y = gpu_matvec(ctx, c["w"], ggml.Q4_K, 4096, 4096, c["x"])
    with orc.Pool(16) as p:
        ref = orc.quant_matvec(c["w"], orc.Q4_K, c["x"], 4096, 4096, pool=p)
    assert rel_l2(y, ref) <= REL_L2
    assert max_rel(y, ref) < FUZZ_MAX_REL


def test_gpu_config2_q6k_151936(ctx):
    c = synth.config2_q6k()
    y = gpu_matvec(ctx, c["w"], ggml.Q6_K, c["rows"], c["cols"], c["x"])
    with orc.Pool(16) as p:
        ref = orc.quant_matvec(c["w"], orc.Q6_K, c["x"], c["rows"], c["cols"], pool=p)
    assert rel_l2(y, ref) <= REL_L2
    assert max_rel(y, ref) < FUZZ_MAX_REL


def _limb_case_x(kind, cols, g):
    x = g.standard_normal(cols).astype(np.float32)
    if kind == "group_magnitudes":  # each 16-element group at its own scale, 1e-6 .. 1e6
        x *= (10.0 ** np.repeat(np.arange(cols // 16) % 13 - 6, 16)).astype(np.float32)
    elif kind == "spike":  # one large element inside otherwise unit groups
        x[5::37] *= 1e4
    elif kind == "tiny":  # group maxima below 2^-100 (scaled before the division)
        x *= np.float32(2.0 ** -110)
    return x


@pytest.mark.parametrize("gtype,rows,cols", [
    (ggml.Q4_K, 300, 256), (ggml.Q4_K, 257, 2048), (ggml.Q4_K, 4100, 4096),
    (ggml.Q4_K, 33000, 4096),  # past 32768 row slabs: four slabs in flight per wave, ragged tail
    (ggml.Q6_K, 129, 1024), (ggml.Q6_K, 999, 4096),
    (ggml.Q6_K, 99000, 1024)])  # past 24576 row slabs of 4 rows: three slabs in flight per wave
@pytest.mark.parametrize("kind", ["normal", "group_magnitudes", "spike", "tiny"])
def test_gpu_matvec_limb_ranges(ctx, pool, gtype, rows, cols, kind):
    # The streaming Q4_K / Q6_K matvecs carry each group of 16 activations as
    # two int8 limbs scaled by the group's largest magnitude: groups of very
    # different scales, a spike inside a group and groups near 2^-110 stay
    # within the fp32-activation fuzz bound against the oracle's fp32 dot.
    g = np.random.default_rng(rows + cols)
    w = synth.q4k_matrix(g, rows, cols) if gtype == ggml.Q4_K else synth.q6k_matrix(g, rows, cols)
    x = _limb_case_x(kind, cols, g)
    print(f"limb ranges {ggml.NAMES[gtype]} {rows}x{cols} {kind}", flush=True)
    y = gpu_matvec(ctx, w, gtype, rows, cols, x)
    ref = orc.quant_matvec(w, gtype, x, rows, cols, pool=pool)
    assert rel_l2(y, ref) <= REL_L2, rel_l2(y, ref)
    assert max_rel(y, ref) < FUZZ_MAX_REL, max_rel(y, ref)


@pytest.mark.parametrize("gtype,cols", [(ggml.Q4_K, 4096), (ggml.Q6_K, 1024)])
def test_gpu_matvec_limb_nan(ctx, gtype, cols):
    # a NaN activation makes every output NaN, as in the fp32 dot
    g = np.random.default_rng(cols)
    rows = 70
    w = synth.q4k_matrix(g, rows, cols) if gtype == ggml.Q4_K else synth.q6k_matrix(g, rows, cols)
    x = g.standard_normal(cols).astype(np.float32)
    x[cols // 3] = np.nan
    y = gpu_matvec(ctx, w, gtype, rows, cols, x)
    assert np.isnan(y).all()


def test_gpu_config1_dense_ffn_q8_0(ctx):
    c = synth.config1()
    D, F = c["d_model"], c["d_ffn"]
    wg = ctx.upload(c["w_gate"], ggml.Q8_0, F, D)
    wu = ctx.upload(c["w_up"], ggml.Q8_0, F, D)
    wd = ctx.upload(c["w_down"], ggml.Q8_0, D, F)
    with orc.Pool(16) as p:
        ref = orc.ffn_dense(c["w_gate"], c["w_up"], c["w_down"], orc.Q8_0, c["x"], D, F, pool=p)
    for unfused in (False, True):  # single launch, then gate/up + down launches
        out = np.zeros(D, np.float32)
        ctx.ffn_dense(out, wg, wu, wd, c["x"], act=lt.ACT_SILU, unfused=unfused)
        assert rel_l2(out, ref) <= REL_L2, (unfused, rel_l2(out, ref))
        assert rel_l2(out, ref) <= 1e-5, (unfused, rel_l2(out, ref))  # fp32 arithmetic throughout
    for t in (wg, wu, wd):
        t.free()


@pytest.mark.gpu
@pytest.mark.parametrize("D,S,act", [
    (64, 256, 0),       # smallest: one Q8_0 block per h row slice
    (512, 288, 1),      # S / 32 = 9 down-K blocks: slices of 1 and 2 blocks, GELU
    (1024, 2112, 0),    # the Gemma4 shared-FFN width
    (2048, 8192, 1),    # the largest single-launch shape: 2 units per lane, 4 passes
    (2048, 8224, 0),    # past it: two launches
])
def test_gpu_ffn_dense_shapes(ctx, pool, D, S, act):
    # the single-launch dense FFN (one h slice per XCD group, partial rows
    # through float atomics) against the oracle and the two-launch path;
    # several calls in a row (launch epochs) with changing x
    g = synth.stream(120, D + S)
    wg_b = synth.q8_0_matrix(g, S, D)
    wu_b = synth.q8_0_matrix(g, S, D)
    wd_b = synth.q8_0_matrix(g, D, S)
    wg, wu, wd = ctx.upload(wg_b, ggml.Q8_0, S, D), ctx.upload(wu_b, ggml.Q8_0, S, D), ctx.upload(wd_b, ggml.Q8_0, D, S)
    for i in range(3):
        x = synth.normal(synth.stream(121, 10 * D + i), (D,))
        ref = orc.ffn_dense(wg_b, wu_b, wd_b, orc.Q8_0, x, D, S, act=act, pool=pool)
        a = np.zeros(D, np.float32)
        b = np.zeros(D, np.float32)
        ctx.ffn_dense(a, wg, wu, wd, x, act=act)
        ctx.ffn_dense(b, wg, wu, wd, x, act=act, unfused=True)
        assert rel_l2(a, ref) <= 1e-5, (i, rel_l2(a, ref))
        assert rel_l2(b, ref) <= 1e-5, (i, rel_l2(b, ref))
    for t in (wg, wu, wd):
        t.free()


@pytest.fixture(scope="module")
def cfg3(ctx):
    c = synth.config3()
    tens = lt.upload_moe(ctx, c["weights"])
    yield c, tens
    for t in tens:
        t.free()


@pytest.mark.parametrize("norm", [True, False])
def test_gpu_config3_qwen3_moe(ctx, cfg3, pool, norm):
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    for i in range(6):
        x = c["x"] if i == 0 else synth.config3_x(i)
        out = np.zeros(w.d_model, np.float32)
        ids = np.zeros(8, np.uint32)
        wt = np.zeros(8, np.float32)
        ctx.moe_forward(out, x, router, gate_up, down, 8, w.d_expert, norm_topk=norm, out_ids=ids, out_w=wt)
        ref, rids, rw, agree = orc.moe_forward(w, x, 8, norm_topk=norm, pool=pool)
        assert agree, "probability tie changes the reference selection for this input"
        assert np.array_equal(ids, rids), (i, ids, rids)
        assert np.allclose(wt, rw, rtol=1e-5, atol=0), (i, wt, rw)
        assert rel_l2(out, ref) <= REL_L2, i


def test_gpu_config3_router_logits_bit_exact(ctx, cfg3):
    c, (router, _, _) = cfg3
    w = c["weights"]
    for i in range(4):
        x = synth.config3_x(50 + i)
        ids = np.zeros(8, np.uint32)
        scores = np.zeros(w.n_experts, np.float32)
        ctx.router_topk(router, x, 8, ids, np.zeros(8, np.float32), scores=scores)
        logits = orc.quant_matvec(w.router, orc.F32, x, w.n_experts, w.d_model)
        rest = np.setdiff1d(np.arange(w.n_experts), ids)
        assert np.array_equal(scores[rest].view(np.uint32), logits[rest].view(np.uint32))
        assert ids.tolist() == orc.topk_softmax_stats(logits, 8)[0].tolist()


def test_gpu_config3_expert_stages_compose(ctx, cfg3, pool):
    # runExpertBatch-style: caller-provided routing through the two expert stages
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    x = c["x"]
    ids = np.zeros(8, np.uint32)
    wt = np.zeros(8, np.float32)
    ctx.router_topk(router, x, 8, ids, wt, norm_topk=True)
    h = np.zeros((8, w.down_cols), np.float32)
    ctx.expert_gate_up_id(gate_up, x, ids, 8, w.d_expert, w.down_cols, h)
    out = np.full(w.d_model, 0.5, np.float32)
    ctx.expert_down_id(down, h, ids, wt, 8, out, accumulate=True)
    ref, *_ = orc.moe_forward(w, x, 8, norm_topk=True, pool=pool, out=np.full(w.d_model, 0.5, np.float32))
    assert rel_l2(out, ref) <= REL_L2


def test_gpu_config4_gemma_like(ctx, pool):
    c = synth.config4()
    w = c["weights"]
    router, gate_up, down = lt.upload_moe(ctx, w)
    D, S = w.d_model, c["d_shared"]
    sg = ctx.upload(c["sh_gate"], ggml.Q8_0, S, D)
    su = ctx.upload(c["sh_up"], ggml.Q8_0, S, D)
    sd = ctx.upload(c["sh_down"], ggml.Q8_0, D, S)
    for i in range(3):
        x = c["x"] if i == 0 else synth.normal(synth.stream(4, 300 + i), (D,))
        out = np.zeros(D, np.float32)
        ids = np.zeros(8, np.uint32)
        wt = np.zeros(8, np.float32)
        ctx.moe_forward(out, x, router, gate_up, down, 8, w.d_expert, act=lt.ACT_GELU_TANH, shared=(sg, su, sd),
                        out_ids=ids, out_w=wt)
        ref, rids, rw = orc.moe_layer_shared(w, x, 8, c["sh_gate"], c["sh_up"], c["sh_down"], S, pool=pool)
        assert np.array_equal(ids, rids), (i, ids, rids)
        assert np.allclose(wt, rw, rtol=1e-5)
        assert rel_l2(out, ref) <= REL_L2
        # Q8_0 router logits follow dotQ8_0's order bit for bit
        scores = np.zeros(w.n_experts, np.float32)
        ctx.router_topk(router, x, 8, ids, wt, scores=scores)
        logits = orc.quant_matvec(w.router, orc.Q8_0, x, w.n_experts, D)
        rest = np.setdiff1d(np.arange(w.n_experts), ids)
        assert np.array_equal(scores[rest].view(np.uint32), logits[rest].view(np.uint32))
    for t in (router, gate_up, down, sg, su, sd):
        t.free()


def test_gpu_config4_single_launch_vs_unfused(ctx, pool):
    """Config 4 in the single launch (Q8_0 router role, shared FFN roles,
    two positions per gate/up lane) against the separate launches and, with
    LT_MOE_DETERMINISTIC (shared FFN first, then the slot-order kernel), bit
    for bit run to run; accumulate adds onto out."""
    c = synth.config4()
    w = c["weights"]
    router, gate_up, down = lt.upload_moe(ctx, w)
    D, S = w.d_model, c["d_shared"]
    sh = (ctx.upload(c["sh_gate"], ggml.Q8_0, S, D), ctx.upload(c["sh_up"], ggml.Q8_0, S, D),
          ctx.upload(c["sh_down"], ggml.Q8_0, D, S))
    x = synth.normal(synth.stream(4, 411), (D,))
    kw = dict(act=lt.ACT_GELU_TANH, shared=sh)
    ref, rids, rw = orc.moe_layer_shared(w, x, 8, c["sh_gate"], c["sh_up"], c["sh_down"], S, pool=pool)
    outs = {}
    for name, extra in (("fused", {}), ("unfused", {"unfused": True}), ("det", {"deterministic": True}),
                        ("det2", {"deterministic": True})):
        out = np.zeros(D, np.float32)
        ids = np.zeros(8, np.uint32)
        ctx.moe_forward(out, x, router, gate_up, down, 8, w.d_expert, out_ids=ids, **kw, **extra)
        assert np.array_equal(ids, rids), (name, ids, rids)
        assert rel_l2(out, ref) <= REL_L2, name
        outs[name] = out
    assert rel_l2(outs["fused"], outs["unfused"]) <= 1e-5
    assert np.array_equal(outs["det"].view(np.uint32), outs["det2"].view(np.uint32))
    base = synth.normal(synth.stream(4, 412), (D,))
    acc = base.copy()
    ctx.moe_forward(acc, x, router, gate_up, down, 8, w.d_expert, accumulate=True, **kw)
    assert rel_l2(acc - base, ref) <= REL_L2
    for t in (router, gate_up, down) + sh:
        t.free()


@pytest.mark.parametrize("D,E,F,k", [(2304, 8, 256, 2), (4096, 16, 512, 4), (2560, 200, 256, 8)])
def test_gpu_single_launch_wide_rows(ctx, pool, D, E, F, k):
    """d_model above 2048 in the single launch (two positions per gate/up
    lane), with few experts (the start values of out spread over the router
    blocks that publish logits) or many (four logits per lane), with and
    without accumulate, against the oracle and the separate launches."""
    w = synth.moe_weights(70 + E, D, E, F)
    x = synth.normal(synth.stream(70, D + E), (D,))
    router, gate_up, down = lt.upload_moe(ctx, w)
    ref, rids, _, agree = orc.moe_forward(w, x, k, pool=pool)
    assert agree
    for unfused in (False, True):
        out = np.zeros(D, np.float32)
        ids = np.zeros(k, np.uint32)
        ctx.moe_forward(out, x, router, gate_up, down, k, F, out_ids=ids, unfused=unfused)
        assert np.array_equal(ids, rids), (unfused, ids, rids)
        assert rel_l2(out, ref) <= REL_L2, unfused
    base = synth.normal(synth.stream(71, D), (D,))
    acc = base.copy()
    ctx.moe_forward(acc, x, router, gate_up, down, k, F, accumulate=True)
    assert rel_l2(acc - base, ref) <= REL_L2
    for t in (router, gate_up, down):
        t.free()


# ------------------------------------------------------------------ edge cases
@pytest.mark.parametrize("E,k", [(128, 1), (128, 16), (100, 8), (1000, 4), (16, 16)])
def test_gpu_moe_expert_counts_and_k(ctx, pool, E, k):
    w = synth.moe_weights(60 + E % 7, 512, E, 256)
    x = synth.normal(synth.stream(60, E + k), (512,))
    router, gate_up, down = lt.upload_moe(ctx, w)
    out = np.zeros(512, np.float32)
    ids = np.zeros(k, np.uint32)
    ctx.moe_forward(out, x, router, gate_up, down, k, 256, out_ids=ids)
    ref, rids, _, agree = orc.moe_forward(w, x, k, pool=pool)
    assert agree and np.array_equal(ids, rids)
    assert rel_l2(out, ref) <= REL_L2
    for t in (router, gate_up, down):
        t.free()


def test_gpu_probability_tie_selects_on_logits(ctx, pool):
    """Two distinct logits whose probabilities are one float: the reference
    (ops/moe.zig:48-52: softmax, then topK's strict '>' on the probabilities,
    :80-91) keeps the lower index; the GPU selects on the logits and keeps the
    larger logit.  x is one-hot, so each logit is exactly router[e, 0]: expert
    7 at 4 is the maximum; experts 3 and 5 at 1 and the next float above 1
    both give l - 4 = -3 (the odd ulp rounds to even), so both weigh 0.045.
    The GPU returns [7, 5] with weights equal to the reference's [p7, p3]
    (p3 == p5), on every path, and its output equals the reference's on the
    weights with experts 3 and 5 swapped (the same expert data under the
    same weight; with expert 3's data the output differs by far more than
    the tolerance)."""
    D, E, F, k = 512, 16, 256, 2
    w = synth.moe_weights(81, D, E, F)
    router = np.zeros((E, D), np.float32)
    router[:, 0] = -8.0
    router[7, 0] = 4.0
    router[3, 0] = 1.0
    router[5, 0] = np.nextafter(np.float32(1.0), np.float32(2.0))
    w = dataclasses.replace(w, router=router)
    x = np.zeros(D, np.float32)
    x[0] = 1.0
    _, rids, rw, agree = orc.moe_forward(w, x, k, pool=pool)
    assert not agree and rids.tolist() == [7, 3]
    assert np.float32(1.0) - np.float32(4.0) == router[5, 0] - np.float32(4.0) and rw[1] > 0.04
    # the same experts under the reference's rule: 3 and 5 swapped (router rows included)
    sw = w.gate_up.copy().reshape(E, 2 * F, -1)
    sw[[3, 5]] = sw[[5, 3]]
    sd = w.down.copy().reshape(E, D, -1)
    sd[[3, 5]] = sd[[5, 3]]
    rs = router.copy()
    rs[[3, 5]] = rs[[5, 3]]
    ws = dataclasses.replace(w, router=rs, gate_up=sw.reshape(w.gate_up.shape), down=sd.reshape(w.down.shape))
    ref_sw, rids_sw, _, _ = orc.moe_forward(ws, x, k, pool=pool)
    assert rids_sw.tolist() == [7, 3]  # expert 5's data, now at index 3
    assert rel_l2(ref_sw, orc.moe_forward(w, x, k, pool=pool)[0]) > 10 * REL_L2
    router_t, gate_up, down = lt.upload_moe(ctx, w)
    for kw in ({}, {"unfused": True}, {"deterministic": True}):
        out = np.zeros(D, np.float32)
        ids = np.zeros(k, np.uint32)
        wts = np.zeros(k, np.float32)
        ctx.moe_forward(out, x, router_t, gate_up, down, k, F, out_ids=ids, out_w=wts, **kw)
        assert ids.tolist() == [7, 5], (kw, ids)
        assert max_rel(wts, rw) < 1e-6, (kw, wts, rw)
        assert rel_l2(out, ref_sw) <= REL_L2, kw
    for t in (router_t, gate_up, down):
        t.free()


def test_gpu_router_duplicate_rows_lowest_index_wins(ctx):
    g = np.random.default_rng(4)
    w = g.standard_normal((64, 256)).astype(np.float32) * 0.02
    w[40] = w[7]
    w[9] = w[7]
    x = g.standard_normal(256).astype(np.float32)
    w[7] = np.sign(x) * 0.5  # make row 7 (and its copies) the clear maximum
    w[9] = w[7]
    w[40] = w[7]
    r = ctx.upload(w, ggml.F32, 64, 256)
    ids = np.zeros(3, np.uint32)
    ctx.router_topk(r, x, 3, ids, np.zeros(3, np.float32))
    assert ids.tolist() == [7, 9, 40]


def test_gpu_deterministic_repeat(ctx, cfg3):
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    # bit-identical in slot order (LT_MOE_DETERMINISTIC); the default atomic
    # combine may differ in the last bits between calls
    for det in (True, False):
        outs = []
        for _ in range(3):
            out = np.zeros(w.d_model, np.float32)
            ctx.moe_forward(out, c["x"], router, gate_up, down, 8, w.d_expert, norm_topk=True, deterministic=det)
            outs.append(out)
        if det:
            assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
        else:
            assert all(rel_l2(o, outs[0]) <= 1e-6 for o in outs[1:])


def test_gpu_device_pointer_path_matches_host(ctx, cfg3):
    from llmtoy_amd.hip import DeviceArray
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    host = np.zeros(w.d_model, np.float32)
    hids = np.zeros(8, np.uint32)
    ctx.moe_forward(host, c["x"], router, gate_up, down, 8, w.d_expert, norm_topk=True, out_ids=hids,
                    deterministic=True)
    xd = DeviceArray.from_numpy(c["x"])
    od = DeviceArray((w.d_model,), np.float32)
    idd = DeviceArray((8,), np.uint32)
    ctx.moe_forward(od, xd, router, gate_up, down, 8, w.d_expert, norm_topk=True, out_ids=idd, deterministic=True)
    ctx.sync()
    assert np.array_equal(od.numpy().view(np.uint32), host.view(np.uint32))
    assert np.array_equal(idd.numpy(), hids)
    for a in (xd, od, idd):
        a.free()


def test_gpu_graph_replay_matches_eager(ctx, cfg3):
    # the decode step captured into a hipGraph (no allocation, no memset
    # inside) replays to the eager result, with eager work between replays:
    # bit for bit in slot order, to the last few ulps with the atomic combine
    from llmtoy_amd.hip import DeviceArray, Graph
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    xs = [c["x"], synth.config3_x(1)]
    xd = [DeviceArray.from_numpy(x) for x in xs]
    od = DeviceArray((w.d_model,), np.float32)
    for det in (True, False):
        eager = []
        for x in xs:
            o = np.zeros(w.d_model, np.float32)
            ctx.moe_forward(o, x, router, gate_up, down, 8, w.d_expert, norm_topk=True, deterministic=det)
            eager.append(o)
        graphs = [Graph(ctx.stream, lambda d=d: ctx.moe_forward(od, d, router, gate_up, down, 8, w.d_expert,
                                                                norm_topk=True, deterministic=det)) for d in xd]
        for rep in range(3):
            for gi, g in enumerate(graphs):
                g.launch()
                ctx.sync()
                if det:
                    assert np.array_equal(od.numpy().view(np.uint32), eager[gi].view(np.uint32)), (rep, gi)
                else:
                    assert rel_l2(od.numpy(), eager[gi]) <= 1e-6, (rep, gi)
                o = np.zeros(w.d_model, np.float32)  # eager work between replays
                ctx.moe_forward(o, xs[1 - gi], router, gate_up, down, 8, w.d_expert, norm_topk=True,
                                deterministic=det)
        for g in graphs:
            g.destroy()
    for a in xd + [od]:
        a.free()


def test_gpu_graph_survives_scratch_growth():
    # A graph captured with small shapes stays valid after a larger call grows
    # the context's scratch: the old buffers are retired, never freed before
    # lt_destroy (the three-launch path uses the h, logits, ids and weight
    # scratch).  Fresh context, so its scratch starts at the small shapes.
    from llmtoy_amd.hip import DeviceArray, Graph
    small = synth.moe_weights(31, 512, 16, 256)
    big = synth.moe_weights(32, 2048, 32, 768)
    xs = synth.normal(synth.stream(31, 7), (512,))
    xb = synth.normal(synth.stream(32, 7), (2048,))
    with lt.Context(0) as c2:
        ts, tb = lt.upload_moe(c2, small), lt.upload_moe(c2, big)
        eager = np.zeros(512, np.float32)
        c2.moe_forward(eager, xs, *ts, 2, 256, unfused=True)  # sizes the scratch for the small shape
        xd, od = DeviceArray.from_numpy(xs), DeviceArray((512,), np.float32)
        g = Graph(c2.stream, lambda: c2.moe_forward(od, xd, *ts, 2, 256, unfused=True))
        ob = np.zeros(2048, np.float32)
        c2.moe_forward(ob, xb, *tb, 8, 768, unfused=True)  # grows h (2 x 256 -> 8 x 768 floats) and more
        for _ in range(2):
            g.launch()
            c2.sync()
            assert np.array_equal(od.numpy().view(np.uint32), eager.view(np.uint32))
        g.destroy()
        for a in (xd, od):
            a.free()
        for t in ts + tb:
            t.free()


def test_gpu_first_fused_call_not_capturable(cfg3):
    # the single-launch kernel's one-time set-up synchronises the stream, so
    # a context's first such call under capture is refused, not broken
    from llmtoy_amd.hip import DeviceArray, Graph
    c, _ = cfg3
    w = c["weights"]
    with lt.Context(0) as c2:
        tens = lt.upload_moe(c2, w)
        xd, od = DeviceArray.from_numpy(c["x"]), DeviceArray((w.d_model,), np.float32)
        with pytest.raises(InvalidError, match="cannot be captured"):
            Graph(c2.stream, lambda: c2.moe_forward(od, xd, *tens, 8, w.d_expert, norm_topk=True))
        o = np.zeros(w.d_model, np.float32)
        c2.moe_forward(o, c["x"], *tens, 8, w.d_expert, norm_topk=True)  # the context still works
        assert np.isfinite(o).all()
        for a in (xd, od):
            a.free()
        for t in tens:
            t.free()


def test_gpu_profile_timeline(cfg3):
    # LT_PROFILE=timeline (read by lt_init): call spans and the phase stamps
    # of the single-launch kernel; the phases of one launch come in the order
    # the hand-overs impose, and the results are those of an unprofiled context
    c, _ = cfg3
    w = c["weights"]
    os.environ["LT_PROFILE"] = "timeline"
    try:
        cp = lt.Context(0)
    finally:
        del os.environ["LT_PROFILE"]
    try:
        tens = lt.upload_moe(cp, w)
        with lt.Context(0) as c0:
            t0 = lt.upload_moe(c0, w)
            for i in range(6):
                x = synth.config3_x(700 + i)
                a, b = np.zeros(w.d_model, np.float32), np.zeros(w.d_model, np.float32)
                cp.moe_forward(a, x, *tens, 8, w.d_expert, norm_topk=True, deterministic=True)
                c0.moe_forward(b, x, *t0, 8, w.d_expert, norm_topk=True, deterministic=True)
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
            for t in t0:
                t.free()
        rep = cp.profile_report()
        print(rep)
        assert "lt_moe_forward" in rep and "6 launches" in rep

        def med(role, phase):
            line = next(l for l in rep.splitlines() if l.startswith(role) and phase in l)
            return float(line.split()[-2])

        published = med("router", "logit published")
        seen = med("gate/up", "logits seen")
        known = med("gate/up", "expert known")
        hpub = med("gate/up", "h record published")
        adds = med("down", "adds issued")
        assert 0 < published < seen <= known < hpub < adds < 1000, rep
        for t in tens:
            t.free()
    finally:
        cp.close()


def test_gpu_errors(ctx):
    with pytest.raises(UnsupportedError):
        ctx.upload(np.zeros(64, np.uint8), ggml.F16, 1, 32)
    with pytest.raises(UnsupportedError):
        ctx.upload(np.zeros(144, np.uint8), ggml.Q4_K, 1, 200)
    with pytest.raises(InvalidError):
        ctx.upload(np.zeros(100, np.uint8), ggml.Q4_K, 1, 256)
    w = synth.moe_weights(61, 256, 4, 256)
    router, gate_up, down = lt.upload_moe(ctx, w)
    out = np.zeros(256, np.float32)
    with pytest.raises(InvalidError):
        ctx.moe_forward(out, np.zeros(256, np.float32), router, gate_up, down, 0, 256)
    with pytest.raises(InvalidError):
        ctx.moe_forward(out, np.zeros(256, np.float32), router, gate_up, down, 5, 256)
    with pytest.raises(InvalidError):
        ctx.expert_gate_up_id(gate_up, np.zeros(256, np.float32), np.array([0, 9], np.uint32), 2, 256, 256,
                              np.zeros((2, 256), np.float32))
    for t in (router, gate_up, down):
        t.free()


# ------------------------------------------------------------------ prefill (config 5)
PREFILL_REL_L2 = 1e-2  # BASELINE config 5's bound (bf16 named; the tiles are f16, 3 more mantissa bits), fp32 accumulation


def test_gpu_config5_prefill_512(ctx, cfg3, pool):
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    p = synth.config5(512, weights=w)
    out = np.zeros((512, w.d_model), np.float32)
    ids = np.zeros((512, 8), np.uint32)
    wt = np.zeros((512, 8), np.float32)
    ctx.moe_prefill(out, p["X"], router, gate_up, down, 8, w.d_expert, norm_topk=True, bias=p["bias"],
                    out_ids=ids, out_w=wt)
    ref, rids, rw = orc.moe_prefill(w, p["X"], 8, norm_topk=True, bias=p["bias"], pool=pool)
    assert np.array_equal(ids, rids)
    assert np.allclose(wt, rw, rtol=1e-5)
    assert rel_l2(out, ref) <= PREFILL_REL_L2
    # Zipf bias skews the load: the busiest expert gets far more than the mean
    counts = np.bincount(ids.ravel(), minlength=w.n_experts)
    assert counts.max() > 4 * counts.mean()


def test_gpu_prefill_matches_decode_per_token(ctx, cfg3):
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    X = np.stack([synth.config3_x(200 + i) for i in range(7)])
    out = np.zeros((7, w.d_model), np.float32)
    ctx.moe_prefill(out, X, router, gate_up, down, 8, w.d_expert, norm_topk=True)
    for t in range(7):
        o = np.zeros(w.d_model, np.float32)
        ctx.moe_forward(o, X[t], router, gate_up, down, 8, w.d_expert, norm_topk=True)
        assert rel_l2(out[t], o) <= PREFILL_REL_L2


def test_gpu_prefill_gelu_padded_k(ctx, pool):
    # config-4 expert shapes (d_model 2816, d_expert 704 -> down K padded to 768)
    w = synth.moe_weights(44, 2816, 16, 704, down_cols=768)
    X = synth.normal(synth.stream(44, 9), (37, 2816))
    router, gate_up, down = lt.upload_moe(ctx, w)
    out = np.zeros((37, 2816), np.float32)
    ids = np.zeros((37, 4), np.uint32)
    ctx.moe_prefill(out, X, router, gate_up, down, 4, 704, act=lt.ACT_GELU_TANH, out_ids=ids)
    ref, rids, _ = orc.moe_prefill(w, X, 4, act=orc.ACT_GELU_TANH, pool=pool)
    assert np.array_equal(ids, rids)
    assert rel_l2(out, ref) <= PREFILL_REL_L2
    for t in (router, gate_up, down):
        t.free()


def test_gpu_prefill_row_scales_match_decode(ctx, cfg3):
    # X rows of very different magnitudes in one batch: each row is divided
    # by a power of two into f16's range and the activations between the
    # GEMMs by its square, so small rows do not underflow f16 and large ones
    # do not saturate it.  Checked against per-token decode, which selects
    # on the same bit-exact logits (at these scales softmax probabilities
    # underflow and tie, so probability order would not be comparable).
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    scales = np.array([1e-4, 1e5, 1.0, 3e-3, 2e4, 1e-6, 7.0, 5e-2, 1e-4, 1e5], np.float32)
    X = np.stack([synth.config3_x(300 + i) * s for i, s in enumerate(scales)]).astype(np.float32)
    out = np.zeros_like(X)
    ids = np.zeros((len(scales), 8), np.uint32)
    ctx.moe_prefill(out, X, router, gate_up, down, 8, w.d_expert, norm_topk=True, out_ids=ids)
    for t, sc in enumerate(scales):
        o = np.zeros(w.d_model, np.float32)
        dids = np.zeros(8, np.uint32)
        ctx.moe_forward(o, X[t], router, gate_up, down, 8, w.d_expert, norm_topk=True, out_ids=dids)
        assert np.array_equal(ids[t], dids), (t, sc)
        assert np.all(np.isfinite(out[t])), (t, sc)
        assert rel_l2(out[t], o) <= PREFILL_REL_L2, (t, sc, rel_l2(out[t], o))


def test_gpu_prefill_saturation_reported(ctx, pool):
    # gate/up weights with d = 16 in every super-block (|w| up to 15120, still
    # exact in f16): the activations between the GEMMs reach ~1e11 even after
    # the row scaling, saturate at +-65504 and the call reports it; the next
    # call on the context is clean again
    w = synth.moe_weights(45, 1024, 16, 256)
    gu = w.gate_up.reshape(w.gate_up.shape[0], -1, 144).copy()
    gu[:, :, 0:2] = np.frombuffer(np.float16(16.0).tobytes(), np.uint8)
    big = dataclasses.replace(w, gate_up=gu.reshape(w.gate_up.shape))
    X = synth.normal(synth.stream(45, 1), (24, 1024))
    router, gate_up, down = lt.upload_moe(ctx, big)
    out = np.zeros((24, 1024), np.float32)
    with pytest.raises(DeviceError, match="saturated"):
        ctx.moe_prefill(out, X, router, gate_up, down, 4, 256)
    for t in (router, gate_up, down):
        t.free()
    router, gate_up, down = lt.upload_moe(ctx, w)
    ctx.moe_prefill(out, X, router, gate_up, down, 4, 256)
    ref, _, _ = orc.moe_prefill(w, X, 4, pool=pool)
    assert rel_l2(out, ref) <= PREFILL_REL_L2
    for t in (router, gate_up, down):
        t.free()


def test_gpu_prefill_deterministic(ctx, cfg3):
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    p = synth.config5(64, weights=w)
    a = np.zeros((64, w.d_model), np.float32)
    b = np.zeros((64, w.d_model), np.float32)
    ctx.moe_prefill(a, p["X"], router, gate_up, down, 8, w.d_expert, norm_topk=True, bias=p["bias"])
    ctx.moe_prefill(b, p["X"], router, gate_up, down, 8, w.d_expert, norm_topk=True, bias=p["bias"])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("T,E,k", [
    (1100, 128, 8),   # 8,800 assignments: ids read again for the placement
    (300, 600, 4),    # 600 experts: the placement table holds one round at a time
])
def test_gpu_prefill_large_batches(ctx, pool, T, E, k):
    # the dispatch's other placement paths, against the oracle on a sample
    # of the tokens (each token's result is its own)
    w = synth.moe_weights(80 + E % 7, 256, E, 64, down_cols=256)
    router, gate_up, down = lt.upload_moe(ctx, w)
    X = synth.normal(synth.stream(81, T), (T, 256))
    bias = synth.zipf_bias(synth.stream(82, E), E)
    out = np.zeros((T, 256), np.float32)
    ids = np.zeros((T, k), np.uint32)
    for _ in range(2):
        prev = out.copy()
        ctx.moe_prefill(out, X, router, gate_up, down, k, 64, norm_topk=True, bias=bias, out_ids=ids)
    assert np.array_equal(prev.view(np.uint32), out.view(np.uint32))
    sel = np.arange(0, T, 7)
    ref, rids, _ = orc.moe_prefill(w, X[sel], k, norm_topk=True, bias=bias, pool=pool)
    assert np.array_equal(ids[sel], rids)
    assert rel_l2(out[sel], ref) <= PREFILL_REL_L2
    for t in (router, gate_up, down):
        t.free()


@pytest.mark.gpu
def test_gpu_prefill_one_token_chunks(ctx, cfg3, pool):
    # experts that get one token of the batch stream their weights against
    # the token's int8 limbs instead of an f16 tile; LT_PREFILL_NO_TINY
    # (read at each call) sends them through the tile path: both within
    # the prefill bound of the oracle, and close to each other
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    p = synth.config5(512, weights=w)
    ids = np.zeros((512, 8), np.uint32)
    a = np.zeros((512, w.d_model), np.float32)
    b = np.zeros((512, w.d_model), np.float32)
    ctx.moe_prefill(a, p["X"], router, gate_up, down, 8, w.d_expert, norm_topk=True, bias=p["bias"], out_ids=ids)
    os.environ["LT_PREFILL_NO_TINY"] = "1"
    try:
        ctx.moe_prefill(b, p["X"], router, gate_up, down, 8, w.d_expert, norm_topk=True, bias=p["bias"])
    finally:
        del os.environ["LT_PREFILL_NO_TINY"]
    counts = np.bincount(ids.ravel(), minlength=w.n_experts)
    assert ((counts % 128) == 1).sum() >= 10  # the routing has one-token chunks
    ones = np.isin(ids, np.nonzero(counts % 128 == 1)[0]).any(axis=1)  # tokens with a slot in one
    ref, _, _ = orc.moe_prefill(w, p["X"][ones], 8, norm_topk=True, bias=p["bias"], pool=pool)
    assert rel_l2(a[ones], ref) <= PREFILL_REL_L2
    assert rel_l2(b[ones], ref) <= PREFILL_REL_L2
    assert rel_l2(a, b) <= 2e-3
    assert not np.array_equal(a[ones].view(np.uint32), b[ones].view(np.uint32))  # the two paths did run


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 2, 3])
def test_gpu_prefill_few_tokens_gelu_padded_k(ctx, pool, T):
    # a batch of one to three tokens: (nearly) every chunk holds one token,
    # so the streams carry the layer, here with GELU and a down K padded
    # past d_expert (704 -> 768)
    w = synth.moe_weights(45, 2048, 16, 704, down_cols=768)
    X = synth.normal(synth.stream(45, T), (T, 2048))
    router, gate_up, down = lt.upload_moe(ctx, w)
    out = np.zeros((T, 2048), np.float32)
    ids = np.zeros((T, 4), np.uint32)
    ctx.moe_prefill(out, X, router, gate_up, down, 4, 704, act=lt.ACT_GELU_TANH, out_ids=ids)
    ref, rids, _ = orc.moe_prefill(w, X, 4, act=orc.ACT_GELU_TANH, pool=pool)
    assert np.array_equal(ids, rids)
    assert rel_l2(out, ref) <= 2e-3  # int8 limbs; H between the GEMMs is still f16
    for t in (router, gate_up, down):
        t.free()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [512, 37])
def test_gpu_prefill_one_launch_matches_two(ctx, cfg3, T):
    # both grouped GEMMs in one launch (the activations handed over in an
    # XCD's L2, used when blocks with equal index % 8 share an XCD) and in
    # two launches (forced in a second context): every row is computed the
    # same way, so the outputs carry the same bits
    c, _ = cfg3
    w = c["weights"]
    os.environ["LT_FUSED_AGENT_HANDOVER"] = "1"
    try:
        ctx2 = lt.Context(0)
    finally:
        del os.environ["LT_FUSED_AGENT_HANDOVER"]
    try:
        t1 = lt.upload_moe(ctx, w)
        t2 = lt.upload_moe(ctx2, w)
        p = synth.config5(T, weights=w)
        a = np.zeros((T, w.d_model), np.float32)
        b = np.zeros((T, w.d_model), np.float32)
        for _ in range(2):
            ctx.moe_prefill(a, p["X"], *t1, 8, w.d_expert, norm_topk=True, bias=p["bias"])
            ctx2.moe_prefill(b, p["X"], *t2, 8, w.d_expert, norm_topk=True, bias=p["bias"])
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        for t in t1 + t2:
            t.free()
    finally:
        ctx2.close()


# ------------------------------------------------------------------ single-launch kernel
# lt_moe_forward runs the whole layer in one launch when the shape fits
# (F32 router, Q4_K experts, d_model <= 2048); LT_MOE_UNFUSED forces the
# router / gate-up / down launches.  Both must match the oracle; routing is
# bit-exact on both.
@pytest.mark.gpu
@pytest.mark.parametrize("D,E,F,Kd,k,act,norm,bias", [
    (2048, 128, 768, 768, 8, 0, True, False),    # config 3
    (512, 61, 256, 256, 5, 0, False, True),      # E not a multiple of 4, k odd, router bias
    (1024, 200, 288, 512, 16, 1, True, False),   # E > 128, F % 256 != 0, zero-padded down K, GELU
    (256, 8, 64, 256, 1, 0, False, False),       # smallest shapes, one expert
])
def test_gpu_fused_layer_matches_oracle_and_unfused(ctx, pool, D, E, F, Kd, k, act, norm, bias):
    w = synth.moe_weights(70 + E % 11, D, E, F, down_cols=Kd)
    router, gate_up, down = lt.upload_moe(ctx, w)
    b = synth.normal(synth.stream(71, E), (E,), 0.5) if bias else None
    for i in range(3):
        x = synth.normal(synth.stream(72, 100 * E + i), (D,))
        res = {}
        # single launch with the atomic combine (default), single launch in
        # slot order, three launches
        for mode in ("atomic", "deterministic", "unfused"):
            out = np.zeros(D, np.float32)
            ids = np.zeros(k, np.uint32)
            wt = np.zeros(k, np.float32)
            ctx.moe_forward(out, x, router, gate_up, down, k, F, act=act, norm_topk=norm, bias=b, out_ids=ids,
                            out_w=wt, unfused=mode == "unfused", deterministic=mode == "deterministic")
            res[mode] = (out, ids, wt)
        ref, rids, rw, agree = orc.moe_forward(w, x, k, act=act, norm_topk=norm, bias=b, pool=pool)
        assert agree
        for mode, (out, ids, wt) in res.items():
            assert np.array_equal(ids, rids), (mode, i, ids, rids)
            assert np.allclose(wt, rw, rtol=1e-5, atol=0), (mode, i)
            assert rel_l2(out, ref) <= REL_L2, (mode, i, rel_l2(out, ref))
        # the two-limb activations (|error| <= max|x| / 65024 per group of
        # 16) keep the result well inside the bar; the two combines differ
        # only in the order of k adds per row
        for mode in ("atomic", "deterministic"):
            assert rel_l2(res[mode][0], ref) <= 2e-4, (mode, rel_l2(res[mode][0], ref))
        assert rel_l2(res["atomic"][0], res["deterministic"][0]) <= 1e-6
    for t in (router, gate_up, down):
        t.free()


@pytest.mark.gpu
@pytest.mark.parametrize("pattern", ["pairs", "period16", "all_equal"])
def test_gpu_fused_tied_logits(ctx, pool, pattern):
    # Equal router rows give bit-equal logits.  The single-launch kernel
    # selects from the logits at or above a group-maximum threshold (or by
    # serial rounds when more than 64 reach it: all_equal) and must keep the
    # tie rule, the lower index first (ops/moe.zig:87).
    D, E, F, k = 512, 128, 256, 8
    w = synth.moe_weights(91, D, E, F)
    pick = {"pairs": np.arange(E) // 2, "period16": np.arange(E) % 16, "all_equal": None}[pattern]
    router = np.zeros_like(w.router) if pick is None else w.router[pick]
    w = dataclasses.replace(w, router=np.ascontiguousarray(router))
    router_t, gate_up, down = lt.upload_moe(ctx, w)
    for i in range(2):
        x = synth.normal(synth.stream(92, i), (D,))
        ref, rids, rw, agree = orc.moe_forward(w, x, k, norm_topk=True, pool=pool)
        assert agree
        if pattern == "all_equal":
            assert rids.tolist() == list(range(k))
        for mode in ("atomic", "deterministic"):
            out = np.zeros(D, np.float32)
            ids = np.zeros(k, np.uint32)
            wt = np.zeros(k, np.float32)
            ctx.moe_forward(out, x, router_t, gate_up, down, k, F, norm_topk=True, out_ids=ids, out_w=wt,
                            deterministic=mode == "deterministic")
            assert np.array_equal(ids, rids), (pattern, mode, i, ids, rids)
            assert np.allclose(wt, rw, rtol=1e-5, atol=0), (pattern, mode, i)
            assert rel_l2(out, ref) <= 2e-4, (pattern, mode, i, rel_l2(out, ref))
    for t in (router_t, gate_up, down):
        t.free()


@pytest.mark.gpu
def test_gpu_fused_deterministic_is_bit_identical(ctx, cfg3):
    # slot-order combine: repeated calls give the same bits; the atomic
    # combine agrees with it to the last few ulps
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    x = synth.config3_x(400)
    outs = []
    for _ in range(4):
        o = np.zeros(w.d_model, np.float32)
        ctx.moe_forward(o, x, router, gate_up, down, 8, w.d_expert, norm_topk=True, deterministic=True)
        outs.append(o)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    a = np.zeros(w.d_model, np.float32)
    ctx.moe_forward(a, x, router, gate_up, down, 8, w.d_expert, norm_topk=True)
    assert rel_l2(a, outs[0]) <= 1e-6


@pytest.mark.gpu
def test_gpu_fused_agent_handover_matches_local(ctx, cfg3):
    # the h records handed over through the XCD's L2 (workgroup-scope
    # stores, used when blocks with equal index % 8 share an XCD) and
    # through memory (agent scope, forced in a second context) carry the
    # same values: the slot-order combine gives the same bits
    c, _ = cfg3
    w = c["weights"]
    # the knob is read when a context is created
    os.environ["LT_FUSED_AGENT_HANDOVER"] = "1"
    try:
        ctx2 = lt.Context(0)
    finally:
        del os.environ["LT_FUSED_AGENT_HANDOVER"]
    try:
        t1 = lt.upload_moe(ctx, w)
        t2 = lt.upload_moe(ctx2, w)
        for i in range(3):
            x = synth.config3_x(500 + i)
            o1 = np.zeros(w.d_model, np.float32)
            o2 = np.zeros(w.d_model, np.float32)
            ctx.moe_forward(o1, x, *t1, 8, w.d_expert, norm_topk=True, deterministic=True)
            ctx2.moe_forward(o2, x, *t2, 8, w.d_expert, norm_topk=True, deterministic=True)
            assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), i
        for t in t1 + t2:
            t.free()
    finally:
        ctx2.close()


@pytest.mark.gpu
@pytest.mark.parametrize("det", [False, True])
def test_gpu_fused_shared_ffn_base(ctx, pool, det):
    # single-launch kernel with a shared dense FFN added (out = shared(x) +
    # experts), with and without accumulating into out
    D, E, F, S = 1024, 32, 256, 512
    w = synth.moe_weights(76, D, E, F)
    router, gate_up, down = lt.upload_moe(ctx, w)
    gen = synth.stream(77, 0)
    sh = [synth.q8_0_matrix(gen, S, D), synth.q8_0_matrix(gen, S, D), synth.q8_0_matrix(gen, D, S)]
    sg = ctx.upload(sh[0], ggml.Q8_0, S, D)
    su = ctx.upload(sh[1], ggml.Q8_0, S, D)
    sd = ctx.upload(sh[2], ggml.Q8_0, D, S)
    for i, acc in enumerate((False, True)):
        x = synth.normal(synth.stream(78, i), (D,))
        prev = synth.normal(synth.stream(79, i), (D,)) if acc else np.zeros(D, np.float32)
        shared = orc.ffn_dense(sh[0], sh[1], sh[2], orc.Q8_0, x, D, S, act=orc.ACT_SILU, pool=pool)
        ref, *_ = orc.moe_forward(w, x, 4, pool=pool, out=prev + shared)
        out = prev.copy()
        ctx.moe_forward(out, x, router, gate_up, down, 4, F, shared=(sg, su, sd), accumulate=acc, deterministic=det)
        assert rel_l2(out, ref) <= REL_L2, (acc, det, rel_l2(out, ref))
    for t in (router, gate_up, down, sg, su, sd):
        t.free()


@pytest.mark.gpu
def test_gpu_fused_accumulate_and_alternating_shapes(ctx, cfg3, pool):
    # out += layer (moeForward's contract), and calls of another shape in
    # between: the hand-over words of one shape must not satisfy the waits of
    # the next
    c, (router, gate_up, down) = cfg3
    w = c["weights"]
    small = synth.moe_weights(73, 512, 16, 256)
    sr, sg, sd = lt.upload_moe(ctx, small)
    for i in range(4):
        x = synth.config3_x(200 + i)
        base = synth.normal(synth.stream(74, i), (w.d_model,))
        ref, *_ = orc.moe_forward(w, x, 8, norm_topk=True, pool=pool, out=base)
        for det in (False, True):
            out = base.copy()
            ctx.moe_forward(out, x, router, gate_up, down, 8, w.d_expert, norm_topk=True, accumulate=True,
                            deterministic=det)
            assert rel_l2(out, ref) <= REL_L2, (i, det)
        xs = synth.normal(synth.stream(75, i), (512,))
        so = np.zeros(512, np.float32)
        ctx.moe_forward(so, xs, sr, sg, sd, 4, 256)
        sref, *_ = orc.moe_forward(small, xs, 4, pool=pool)
        assert rel_l2(so, sref) <= REL_L2, i
    for t in (sr, sg, sd):
        t.free()


@pytest.mark.gpu
def test_gpu_stream_read(ctx):
    # the read-ceiling probe: enqueues, reads, and rejects what it cannot take
    from llmtoy_amd.hip import DeviceArray
    buf = DeviceArray((1 << 20,), np.uint8)
    for nb in (16, 4096, 1 << 20):
        ctx.stream_read(buf.ptr, nb)
    ctx.sync()
    with pytest.raises(InvalidError):
        ctx.stream_read(buf.ptr, 24)
    with pytest.raises(InvalidError):
        ctx.stream_read(buf.ptr + 8, 16)
    buf.free()
