"""GPU parity of the Gemma4 APEX expert formats (Q5_0, Q5_1, IQ4_NL, Q3_K):
matvec through lt_matvec against the oracle's quantMatvec (the reference's
GPU matvec fuzz bound, max|d| / max|ref| < 1e-4, gpu/matvec.zig:4543-4619),
and the upload / read-back round trip of each planar layout."""
import numpy as np
import pytest

import pyoracle as orc
from llmtoy_amd import ggml, synth

pytestmark = pytest.mark.gpu

FMTS = [ggml.Q5_0, ggml.Q5_1, ggml.IQ4_NL, ggml.Q3_K]


def max_rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / (np.max(np.abs(b)) + 1e-6))


@pytest.mark.parametrize("gtype", FMTS)
@pytest.mark.parametrize("rows,cols", [(37, 256), (64, 2816), (5, 4096), (130, 768), (3, 16384)])
def test_gpu_matvec_formats(ctx, gtype, rows, cols):
    g = np.random.default_rng(rows * 7 + cols + gtype)
    m = synth.quant_matrix(g, gtype, rows, cols)
    x = ((g.random(cols, dtype=np.float32) - 0.5) * 2).astype(np.float32)
    print(f"matvec {ggml.NAMES[gtype]} {rows}x{cols}", flush=True)
    t = ctx.upload(m, gtype, rows, cols)
    y = np.zeros(rows, np.float32)
    ctx.quant_matvec(y, t, x)
    assert np.array_equal(t.read(), m.reshape(-1))
    t.free()
    ref = orc.quant_matvec(m, gtype, x, rows, cols)
    assert max_rel(y, ref) < 1e-4


# The streaming Q3_K kernel (rows of 1, 2, 4, 8 or 16 super-blocks): ragged
# slabs, and a matrix large enough that waves loop over several slab sets.
@pytest.mark.parametrize("rows,cols", [(29, 512), (41, 1024), (19, 2048), (1025, 256), (20000, 4096)])
def test_gpu_matvec_q3k_stream(ctx, rows, cols):
    g = np.random.default_rng(rows + 3 * cols)
    m = synth.quant_matrix(g, ggml.Q3_K, rows, cols)
    x = ((g.random(cols, dtype=np.float32) - 0.5) * 2).astype(np.float32)
    print(f"matvec Q3_K stream {rows}x{cols}", flush=True)
    t = ctx.upload(m, ggml.Q3_K, rows, cols)
    y = np.zeros(rows, np.float32)
    ctx.quant_matvec(y, t, x)
    t.free()
    ref = orc.quant_matvec(m, ggml.Q3_K, x, rows, cols)
    assert max_rel(y, ref) < 1e-4


@pytest.mark.parametrize("gtype", FMTS)
def test_gpu_formats_expert_layout_and_large_upload(ctx, gtype):
    # 3-D expert tensors upload as one flat matrix (gemma4/loader.zig:277-292);
    # more than one 4 MiB staging piece and more pieces than workers
    E, rows, cols = 16, 704, 2816
    g = np.random.default_rng(500 + gtype)
    m = synth.quant_matrix(g, gtype, E * rows, cols)
    t = ctx.upload(m, gtype, rows, cols, E)
    assert np.array_equal(t.read(), m.reshape(-1))
    x = synth.normal(g, (cols,))
    y = np.zeros(E * rows, np.float32)
    ctx.quant_matvec(y, t, x)
    t.free()
    ref = orc.quant_matvec(m, gtype, x, E * rows, cols)
    assert max_rel(y, ref) < 1e-4


# ------------------------------------------------------------------ experts in these formats
def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("gu,dn,F,D", [(ggml.Q3_K, ggml.Q5_0, 704, 2816), (ggml.Q3_K, ggml.Q5_1, 704, 2816),
                                       (ggml.Q3_K, ggml.IQ4_NL, 704, 2816), (ggml.Q5_0, ggml.Q3_K, 768, 2816),
                                       (ggml.IQ4_NL, ggml.Q4_K, 768, 2816), (ggml.Q4_K, ggml.IQ4_NL, 768, 2816),
                                       (ggml.Q3_K, ggml.IQ4_NL, 512, 2048), (ggml.Q3_K, ggml.Q4_K, 256, 4096),
                                       (ggml.Q4_K, ggml.Q5_1, 1024, 1024)])
def test_gpu_moe_forward_apex_formats(ctx, pool, gu, dn, F, D):
    # Q3_K or Q4_K gate/up with IQ4_NL / Q5_0 / Q5_1 / Q4_K down run in the
    # single launch (the format instance), the other mixes in separate
    # launches; unfused forces the separate launches: both against the
    # oracle and against each other (the single launch adds the slots' rows
    # with float atomics and hands h over as int8 limbs, where the Q4_K down
    # kernel of the separate launches reads fp32 h: to about 3e-5)
    import llmtoy_amd as lt
    w = synth.moe_weights(43, D, 32, F, gate_up_type=gu, down_type=dn)
    R, GU, DN = lt.upload_moe(ctx, w)
    x = synth.normal(synth.stream(43, 1), (D,))
    print(f"moe_forward gate_up {ggml.NAMES[gu]} down {ggml.NAMES[dn]} F {F} D {D}", flush=True)
    ref, rids, rw, agree = orc.moe_forward(w, x, 8, act=orc.ACT_GELU_TANH, pool=pool)
    assert agree
    outs = []
    for unfused in (False, True):
        out = np.zeros(D, np.float32)
        ids = np.zeros(8, np.uint32)
        wts = np.zeros(8, np.float32)
        ctx.moe_forward(out, x, R, GU, DN, 8, F, act=lt.ACT_GELU_TANH, out_ids=ids, out_w=wts, unfused=unfused)
        assert ids.tolist() == rids.tolist(), (unfused, ids, rids)
        assert np.max(np.abs(wts - rw)) < 1e-6, unfused
        assert rel_l2(out, ref) < 1e-3, (unfused, rel_l2(out, ref))
        outs.append(out)
    for t in (R, GU, DN):
        t.free()
    assert rel_l2(outs[0], outs[1]) < 1e-4, rel_l2(outs[0], outs[1])


def test_gpu_gemma4_block_apex_formats(ctx, pool):
    # Gemma4 APEX: Q8_0 router, Q3_K gate/up, IQ4_NL down, with every norm step
    import llmtoy_amd as lt
    from llmtoy_amd import lib as ltlib
    w = synth.moe_weights(44, 2816, 32, 704, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K,
                          down_type=ggml.IQ4_NL)
    tens = lt.upload_moe(ctx, w)
    x, dense = synth.normal(synth.stream(44, 1), (2816,)), synth.normal(synth.stream(44, 2), (2816,))
    nm = synth.gemma4_norms(44, 2816, 32)
    ids = np.zeros(8, np.uint32)
    got = ltlib.gemma4_moe_block(ctx, x.copy(), dense, *tens, 8, 704, nm, 0.75, 1e-6, precise=True, out_ids=ids)
    ref, rids, _ = orc.gemma4_moe_block(w, x, dense, 8, nm, 0.75, 1e-6, pool=pool)
    for t in tens:
        t.free()
    assert ids.tolist() == rids.tolist() and rel_l2(got, ref) < 1e-3


def test_gpu_gemma4_block_apex_fused_matches_launches(ctx, pool):
    # the APEX Gemma4 block in one launch (tree-order norms) against its
    # separate launches and the oracle: the same routing bits, the output to
    # the order of the experts' float atomics
    import llmtoy_amd as lt
    from llmtoy_amd import lib as ltlib
    w = synth.moe_weights(45, 2816, 128, 704, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K,
                          down_type=ggml.IQ4_NL)
    tens = lt.upload_moe(ctx, w)
    nm = synth.gemma4_norms(45, 2816, 128)
    for i in range(3):
        x, dense = synth.normal(synth.stream(45, 1 + i), (2816,)), synth.normal(synth.stream(45, 9), (2816,))
        print(f"gemma4 apex block, input {i}", flush=True)
        ref, rids, _ = orc.gemma4_moe_block(w, x, dense, 8, nm, 0.75, 1e-6, pool=pool)
        res = []
        for unfused in (False, True):
            ids, wt = np.zeros(8, np.uint32), np.zeros(8, np.float32)
            got = ltlib.gemma4_moe_block(ctx, x.copy(), dense, *tens, 8, 704, nm, 0.75, 1e-6, out_ids=ids, out_w=wt,
                                         unfused=unfused)
            assert ids.tolist() == rids.tolist() and rel_l2(got, ref) < 1e-3, (i, unfused, rel_l2(got, ref))
            res.append((got, ids, wt))
        (a, ia, wa), (b, ib, wb) = res
        assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
        assert rel_l2(a, b) < 1e-5, (i, rel_l2(a, b))
    for t in tens:
        t.free()


@pytest.mark.parametrize("gtype", FMTS)
def test_gpu_expert_id_entry_points(ctx, gtype):
    # lt_expert_gate_up_id / lt_expert_down_id (GpuWeights.runExpertBatch's two stages)
    import llmtoy_amd as lt
    E, D, F = 12, 1024, 512
    w = synth.moe_weights(45, D, E, F, gate_up_type=gtype, down_type=gtype)
    _, GU, DN = lt.upload_moe(ctx, w)
    x = synth.normal(synth.stream(45, 1), (D,))
    ids = np.array([3, 11, 0, 7, 3], np.uint32)
    wts = np.array([0.4, 0.3, 0.15, 0.1, 0.05], np.float32)
    h = np.zeros((5, F), np.float32)
    ctx.expert_gate_up_id(GU, x, ids, 5, F, F, h, act=lt.ACT_SILU)
    out = np.full(D, 0.5, np.float32)
    ctx.expert_down_id(DN, h, ids, wts, 5, out, accumulate=True)
    GU.free()
    DN.free()
    gu = w.gate_up.reshape(E, 2 * F, -1)
    dn = w.down.reshape(E, D, -1)
    want_out = np.full(D, 0.5, np.float64)
    for s, e in enumerate(ids):
        g = orc.quant_matvec(gu[e, :F], gtype, x, F, D).astype(np.float64)
        u = orc.quant_matvec(gu[e, F:], gtype, x, F, D).astype(np.float64)
        want_h = g / (1 + np.exp(-g)) * u
        assert rel_l2(h[s], want_h) < 1e-4
        want_out += float(wts[s]) * orc.quant_matvec(dn[e], gtype, h[s], D, F).astype(np.float64)
    assert rel_l2(out, want_out) < 1e-4
