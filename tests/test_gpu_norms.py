"""GPU parity of the RMS norms, the MoE tail and the Gemma4 MoE block
(lt_rmsnorm, lt_add_rmsnorm, lt_rmsnorm_weighted_raw_scaled, lt_moe_tail,
lt_gemma4_moe_block) against the CPU oracle.

Bars: with LT_NORM_PRECISE (the reference's sequential sum of squares) the
norms and the tail are bit-exact with the oracle; with the default tree sum
they hold the reference's own GPU norm bound, max|d| / max|ref| < 1e-5
(gpu/matvec.zig:5808-5858, 5930-5978).  The block: expert ids bit-exact,
x within 1e-3 relative L2 (and far tighter in practice).
"""
import numpy as np
import pytest

import llmtoy_amd as lt
import pyoracle as orc
from llmtoy_amd import ggml, lib as ltlib, synth
from llmtoy_amd.lib import InvalidError, UnsupportedError

pytestmark = pytest.mark.gpu

NORM_MAX_REL = 1e-5


def max_rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / (np.max(np.abs(b)) + 1e-6))


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def fuzz_vec(seed, n, scale):
    # the reference's scheme: (U(0,1) - 0.5) * scale
    g = np.random.default_rng(seed)
    return ((g.random(n, dtype=np.float32) - np.float32(0.5)) * np.float32(scale)).astype(np.float32)


def test_gpu_rmsnorm_reference_kat(ctx):
    # ops/math.zig:344-354
    x = np.array([1, 2, 3, 4], np.float32)
    out = ltlib.rmsnorm(ctx, np.zeros(4, np.float32), x, np.ones(4, np.float32), eps=1e-8)
    assert np.allclose(out, x / np.sqrt(7.5), atol=1e-5, rtol=0)


@pytest.mark.parametrize("n,seed", [(512, 71), (2816, 73), (4096, 75), (16384, 77), (1, 78), (1000, 79)])
def test_gpu_rmsnorm_fuzz(ctx, n, seed):
    # gpu/matvec.zig:5808-5858 (fuzzRmsnorm): x ~ (U - 0.5) * 4, w ~ (U - 0.5) * 2
    x, w = fuzz_vec(seed, n, 4.0), fuzz_vec(seed + 1, n, 2.0)
    ref = orc.rmsnorm(x, w, 1e-6)
    tree = ltlib.rmsnorm(ctx, np.zeros(n, np.float32), x, w)
    precise = ltlib.rmsnorm(ctx, np.zeros(n, np.float32), x, w, precise=True)
    assert max_rel(tree, ref) < NORM_MAX_REL
    assert np.array_equal(precise, ref)


def test_gpu_rmsnorm_sequential_sum_kat(ctx):
    # four 1s then twelve 2^-11: only the index-order sum gives rms_inv = 2 exactly
    x = np.array([1] * 4 + [2.0 ** -11] * 12, np.float32)
    w = fuzz_vec(5, 16, 2.0)
    out = ltlib.rmsnorm(ctx, np.zeros(16, np.float32), x, w, eps=0.0, precise=True)
    assert np.array_equal(out, (x * np.float32(2)) * w)


def test_gpu_rmsnorm_raw_one_plus_w_and_rows(ctx):
    n, rows = 2816, 5
    X = np.stack([fuzz_vec(80 + r, n, 4.0) for r in range(rows)])
    w = fuzz_vec(90, n, 2.0)
    raw = ltlib.rmsnorm(ctx, np.zeros_like(X), X, None, precise=True)
    onep = ltlib.rmsnorm(ctx, np.zeros_like(X), X, w, precise=True, one_plus_w=True)
    for r in range(rows):
        assert np.array_equal(raw[r], orc.rmsnorm(X[r], None, 1e-6))
        assert np.array_equal(onep[r], orc.rmsnorm(X[r], w, 1e-6, one_plus_w=True))
    # in place
    Y = X.copy()
    ltlib.rmsnorm(ctx, Y, Y, w, precise=True)
    assert np.array_equal(Y[2], orc.rmsnorm(X[2], w, 1e-6))


def test_gpu_add_rmsnorm_fuzz(ctx):
    # gpu/matvec.zig:5930-5978 (fuzzAddRmsnorm)
    n = 2816
    a, b, w = fuzz_vec(89, n, 4.0), fuzz_vec(90, n, 4.0), fuzz_vec(91, n, 2.0)
    ref = orc.add_rmsnorm(a, b, w, 1e-6)
    assert max_rel(ltlib.add_rmsnorm(ctx, np.zeros(n, np.float32), a, b, w), ref) < NORM_MAX_REL
    assert np.array_equal(ltlib.add_rmsnorm(ctx, np.zeros(n, np.float32), a, b, w, precise=True), ref)


def test_gpu_rmsnorm_weighted_raw_scaled(ctx):
    # ops/math.zig:356-376 shape plus a d_model-sized case
    for n, seed in ((4, 1), (2816, 2)):
        x, w, s = fuzz_vec(seed, n, 4.0), fuzz_vec(seed + 10, n, 2.0), fuzz_vec(seed + 20, n, 2.0)
        gs = np.float32(1) / np.sqrt(np.float32(n))
        rw, rr = orc.rmsnorm_wrs(x, w, s, gs, 1e-6)
        for precise in (False, True):
            wo, ro = np.zeros(n, np.float32), np.zeros(n, np.float32)
            ltlib.rmsnorm_weighted_raw_scaled(ctx, wo, ro, x, w, s, float(gs), precise=precise)
            if precise:
                assert np.array_equal(wo, rw) and np.array_equal(ro, rr)
            else:
                assert max_rel(wo, rw) < NORM_MAX_REL and max_rel(ro, rr) < NORM_MAX_REL


@pytest.mark.parametrize("los", [1.0, 0.75])
def test_gpu_moe_tail(ctx, los):
    n = 2816
    x, dense = fuzz_vec(101, n, 4.0), fuzz_vec(102, n, 4.0)
    moe = fuzz_vec(103, n, 0.2)
    nm = synth.gemma4_norms(4, n, 8)
    ref = orc.moe_tail(x, moe, dense, nm["post_ffw_norm_2"], nm["post_ffw_norm"], los)
    for precise in (False, True):
        got = ltlib.moe_tail(ctx, x.copy(), moe, dense, nm["post_ffw_norm_2"], nm["post_ffw_norm"], los,
                             precise=precise)
        if precise:
            assert np.array_equal(got, ref)
        else:
            assert max_rel(got, ref) < NORM_MAX_REL


def test_gpu_norm_errors(ctx):
    x = np.ones(8, np.float32)
    with pytest.raises(UnsupportedError):
        ctx._check(ctx.lib.lt_rmsnorm(ctx.ptr, x.ctypes.data, x.ctypes.data, None, 1, 16385, 1e-6, ltlib.LT_HOST_IO))
    with pytest.raises(UnsupportedError):
        ctx._check(ctx.lib.lt_rmsnorm(ctx.ptr, x.ctypes.data, x.ctypes.data, None, 1, 0, 1e-6, ltlib.LT_HOST_IO))
    with pytest.raises(InvalidError):
        ltlib.rmsnorm(ctx, np.zeros(8, np.float32), x, eps=-1.0)
    with pytest.raises(InvalidError):
        ctx._check(ctx.lib.lt_rmsnorm(ctx.ptr, x.ctypes.data, x.ctypes.data, None, 1, 8, 1e-6,
                                      ltlib.LT_HOST_IO | (1 << 12)))
    with pytest.raises(InvalidError):
        ctx._check(ctx.lib.lt_moe_tail(ctx.ptr, x.ctypes.data, None, x.ctypes.data, x.ctypes.data, x.ctypes.data,
                                       1.0, 8, 1e-6, ltlib.LT_HOST_IO))


# ------------------------------------------------------------------ the Gemma4 block
@pytest.fixture(scope="module")
def cfg4b(ctx):
    c = synth.config4_block()
    tens = lt.upload_moe(ctx, c["weights"])
    yield c, tens
    for t in tens:
        t.free()


def run_block(ctx, c, tens, x, precise=False, norms=None):
    w = c["weights"]
    ids, wt = np.zeros(c["k"], np.uint32), np.zeros(c["k"], np.float32)
    out = ltlib.gemma4_moe_block(ctx, x.copy(), c["dense_ffn"], *tens, c["k"], w.d_expert, norms or c["norms"],
                                 c["layer_output_scale"], c["eps"], precise=precise, out_ids=ids, out_w=wt)
    return out, ids, wt


@pytest.mark.parametrize("precise", [True, False])
def test_gpu_gemma4_block_config4(ctx, cfg4b, pool, precise):
    c, tens = cfg4b
    w = c["weights"]
    for i in range(4):
        x = c["x"] if i == 0 else synth.normal(synth.stream(4, 60 + i), (w.d_model,))
        print(f"gemma4 block token {i} precise={precise}", flush=True)
        got, ids, wt = run_block(ctx, c, tens, x, precise)
        ref, rids, rwt = orc.gemma4_moe_block(w, x, c["dense_ffn"], c["k"], c["norms"], c["layer_output_scale"],
                                              c["eps"], pool=pool)
        assert ids.tolist() == rids.tolist()
        assert np.allclose(wt, rwt, rtol=1e-5, atol=0)
        assert rel_l2(got, ref) < 1e-3


def test_gpu_gemma4_block_without_down_scale_and_unit_output_scale(ctx, cfg4b, pool):
    c, tens = cfg4b
    w = c["weights"]
    nm = dict(c["norms"], down_exps_scale=None)
    ids = np.zeros(8, np.uint32)
    got = ltlib.gemma4_moe_block(ctx, c["x"].copy(), c["dense_ffn"], *tens, 8, w.d_expert, nm, 1.0, c["eps"],
                                 precise=True, out_ids=ids)
    ref, rids, _ = orc.gemma4_moe_block(w, c["x"], c["dense_ffn"], 8, nm, 1.0, c["eps"], pool=pool)
    assert ids.tolist() == rids.tolist() and rel_l2(got, ref) < 1e-3


def test_gpu_gemma4_block_fused_matches_launches(ctx, cfg4b):
    # the block in one launch of the single-launch kernel (tree-order norms)
    # against its separate launches: the same routing bits, the output to
    # the order of the experts' adds (float atomics in the single launch)
    c, tens = cfg4b
    w = c["weights"]
    for i in range(3):
        x = c["x"] if i == 0 else synth.normal(synth.stream(4, 80 + i), (w.d_model,))
        res = []
        for unfused in (False, True):
            ids, wt = np.zeros(c["k"], np.uint32), np.zeros(c["k"], np.float32)
            got = ltlib.gemma4_moe_block(ctx, x.copy(), c["dense_ffn"], *tens, c["k"], w.d_expert, c["norms"],
                                         c["layer_output_scale"], c["eps"], out_ids=ids, out_w=wt, unfused=unfused)
            res.append((got, ids, wt))
        (a, ia, wa), (b, ib, wb) = res
        assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
        assert rel_l2(a, b) < 1e-6, (i, rel_l2(a, b))


@pytest.mark.parametrize("ds", [True, False])
def test_gpu_gemma4_block_fused_slotless_groups(ctx, pool, ds):
    # k = 4: XCD groups 4-7 hold no slot; without down_exps_scale too
    w = synth.moe_weights(43, 1024, 32, 256, router_type=ggml.Q8_0)
    tens = lt.upload_moe(ctx, w)
    nm = synth.gemma4_norms(43, 1024, 32)
    if not ds:
        nm = dict(nm, down_exps_scale=None)
    for i in range(3):
        x, dense = synth.normal(synth.stream(43, 1 + i), (1024,)), synth.normal(synth.stream(43, 9), (1024,))
        ids = np.zeros(4, np.uint32)
        got = ltlib.gemma4_moe_block(ctx, x.copy(), dense, *tens, 4, 256, nm, 0.5, 1e-6, out_ids=ids)
        ref, rids, _ = orc.gemma4_moe_block(w, x, dense, 4, nm, 0.5, 1e-6, pool=pool)
        assert ids.tolist() == rids.tolist() and rel_l2(got, ref) < 1e-3, (i, rel_l2(got, ref))
    for t in tens:
        t.free()


@pytest.mark.parametrize("E,k", [(300, 8), (16, 4)])
def test_gpu_gemma4_block_expert_counts(ctx, pool, E, k):
    # E > 256 takes the router's own top-k; E <= 256 the gate/up blocks select
    w = synth.moe_weights(41, 1024, E, 256, router_type=ggml.Q8_0)
    tens = lt.upload_moe(ctx, w)
    x, dense = synth.normal(synth.stream(41, 1), (1024,)), synth.normal(synth.stream(41, 2), (1024,))
    nm = synth.gemma4_norms(41, 1024, E)
    ids = np.zeros(k, np.uint32)
    got = ltlib.gemma4_moe_block(ctx, x.copy(), dense, *tens, k, 256, nm, 0.5, 1e-6, precise=True, out_ids=ids)
    ref, rids, _ = orc.gemma4_moe_block(w, x, dense, k, nm, 0.5, 1e-6, pool=pool)
    for t in tens:
        t.free()
    assert ids.tolist() == rids.tolist() and rel_l2(got, ref) < 1e-3


def test_gpu_gemma4_block_f32_router(ctx, pool):
    w = synth.moe_weights(42, 2048, 128, 768)  # config-3 shapes, fp32 router
    tens = lt.upload_moe(ctx, w)
    x, dense = synth.normal(synth.stream(42, 1), (2048,)), synth.normal(synth.stream(42, 2), (2048,))
    nm = synth.gemma4_norms(42, 2048, 128)
    ids = np.zeros(8, np.uint32)
    got = ltlib.gemma4_moe_block(ctx, x.copy(), dense, *tens, 8, 768, nm, 1.0, 1e-6, act=lt.ACT_SILU, precise=True,
                                 out_ids=ids)
    ref, rids, _ = orc.gemma4_moe_block(w, x, dense, 8, nm, 1.0, 1e-6, act=orc.ACT_SILU, pool=pool)
    for t in tens:
        t.free()
    assert ids.tolist() == rids.tolist() and rel_l2(got, ref) < 1e-3


@pytest.mark.parametrize("apex", [False, True])
@pytest.mark.parametrize("det", [True, False])
def test_gpu_gemma4_block_graph_replay_matches_eager(ctx, apex, det):
    # the block captured into a hipGraph (no allocation, no memset inside)
    # replays to the eager result -- bit for bit with the slot-order adds
    # (det), to the order of the float-atomic adds otherwise (the Q4_K block
    # runs as one launch of the single-launch kernel then) -- with eager
    # work between replays; x is updated in place, so each replay starts
    # from a fresh copy
    from llmtoy_amd.hip import D2D, DeviceArray, Graph, check, hip
    if apex:
        w = synth.moe_weights(48, 2816, 16, 704, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K,
                              down_type=ggml.IQ4_NL)
    else:
        w = synth.moe_weights(48, 2816, 16, 704, down_cols=768, router_type=ggml.Q8_0)
    tens = lt.upload_moe(ctx, w)
    nm = synth.gemma4_norms(48, 2816, 16)
    dn = {k: DeviceArray.from_numpy(v) for k, v in nm.items()}
    x0 = synth.normal(synth.stream(48, 1), (2816,))
    dense = synth.normal(synth.stream(48, 2), (2816,))
    eager = ltlib.gemma4_moe_block(ctx, x0.copy(), dense, *tens, 8, 704, nm, 0.75, 1e-6, deterministic=det)
    X0, X, D = DeviceArray.from_numpy(x0), DeviceArray((2816,), np.float32), DeviceArray.from_numpy(dense)
    g = Graph(ctx.stream, lambda: ltlib.gemma4_moe_block(ctx, X, D, *tens, 8, 704, dn, 0.75, 1e-6,
                                                         deterministic=det))
    for rep in range(3):
        check(hip().hipMemcpy(X.ptr, X0.ptr, 2816 * 4, D2D), "hipMemcpy D2D")
        g.launch()
        ctx.sync()
        if det:
            assert np.array_equal(X.numpy().view(np.uint32), eager.view(np.uint32)), rep
        else:
            assert rel_l2(X.numpy(), eager) <= 1e-6, (rep, rel_l2(X.numpy(), eager))
        ltlib.gemma4_moe_block(ctx, x0.copy(), dense, *tens, 8, 704, nm, 1.0, 1e-6)  # eager work between
    g.destroy()
    for a in [X0, X, D] + list(dn.values()):
        a.free()
    for t in tens:
        t.free()
