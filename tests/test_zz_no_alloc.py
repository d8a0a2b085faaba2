"""lt_moe_forward_noalloc: the single-launch MoE layer on the library's
static scratch (no device allocation), through the C ABI, against
lt_moe_forward on the same inputs and against the CPU oracle.  Two calls in
a row, the second on a smaller layer, so the shared scratch is reused."""
import numpy as np
import pytest

import llmtoy_amd as lt
import pyoracle as orc
from llmtoy_amd import ggml, synth
from llmtoy_amd.hip import DeviceArray
from llmtoy_amd.lib import InvalidError, UnsupportedError

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def _run(ctx, fn, tens, x, k, F, det, norm):
    D = x.shape[0]
    xd, od = DeviceArray.from_numpy(x), DeviceArray((D,), np.float32)
    idd, wd = DeviceArray((k,), np.uint32), DeviceArray((k,), np.float32)
    fn(od, xd, *tens, k, F, norm_topk=norm, out_ids=idd, out_w=wd, deterministic=det)
    ctx.sync()
    res = od.numpy(), idd.numpy(), wd.numpy()
    for a in (xd, od, idd, wd):
        a.free()
    return res


@pytest.mark.parametrize("det", [True, False])
def test_noalloc_matches_moe_forward_two_calls(det):
    cases = [  # (seed, D, E, F, k, norm): the config-3 layer, then a smaller one
        (3, 2048, 128, 768, 8, True),
        (41, 1024, 64, 512, 4, False),
    ]
    with lt.Context(0) as ctx, orc.Pool(8) as pool:
        for seed, D, E, F, k, norm in cases:
            w = synth.config3()["weights"] if seed == 3 else synth.moe_weights(seed, D, E, F)
            x = synth.normal(synth.stream(seed, 77), (D,))
            tens = lt.upload_moe(ctx, w)
            got = _run(ctx, ctx.moe_forward_noalloc, tens, x, k, F, det, norm)
            want = _run(ctx, ctx.moe_forward, tens, x, k, F, det, norm)
            ref, rids, rw, agree = orc.moe_forward(w, x, k, norm_topk=norm, pool=pool)
            assert agree
            assert np.array_equal(got[1], want[1]) and np.array_equal(got[1], rids), (seed, got[1], rids)
            assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32))
            if det:  # slot-order combine: the same bits as lt_moe_forward
                assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), seed
            else:    # float-atomic combine: the order of the k adds varies
                assert _rel(got[0], want[0]) <= 1e-6, seed
            assert _rel(got[0], ref) <= 1e-3, seed
            for t in tens:
                t.free()


def _upload_shared(ctx, c):
    D, S = c["weights"].d_model, c["d_shared"]
    return (ctx.upload(c["sh_gate"], ggml.Q8_0, S, D), ctx.upload(c["sh_up"], ggml.Q8_0, S, D),
            ctx.upload(c["sh_down"], ggml.Q8_0, D, S))


def test_noalloc_config4_shared_two_calls():
    """The Gemma4-like layer (Q8_0 router, Q8_0 shared FFN, Q4_K experts,
    d_model 2816) in the single launch, then the config-3 layer, on the same
    static scratch."""
    c = synth.config4()
    w4 = c["weights"]
    with lt.Context(0) as ctx, orc.Pool(8) as pool:
        tens = lt.upload_moe(ctx, w4)
        sh = _upload_shared(ctx, c)
        D = w4.d_model
        for i in range(2):
            x = c["x"] if i == 0 else synth.normal(synth.stream(4, 500), (D,))
            xd, od = DeviceArray.from_numpy(x), DeviceArray((D,), np.float32)
            idd, wd = DeviceArray((8,), np.uint32), DeviceArray((8,), np.float32)
            ctx.moe_forward_noalloc(od, xd, *tens, 8, w4.d_expert, act=lt.ACT_GELU_TANH, shared=sh, out_ids=idd,
                                    out_w=wd)
            ctx.sync()
            want = np.zeros(D, np.float32)
            wids = np.zeros(8, np.uint32)
            ctx.moe_forward(want, x, *tens, 8, w4.d_expert, act=lt.ACT_GELU_TANH, shared=sh, out_ids=wids)
            ref, rids, rw = orc.moe_layer_shared(w4, x, 8, c["sh_gate"], c["sh_up"], c["sh_down"], c["d_shared"],
                                                 pool=pool)
            assert np.array_equal(idd.numpy(), rids) and np.array_equal(wids, rids), (i, idd.numpy(), rids)
            assert np.allclose(wd.numpy(), rw, rtol=1e-5)
            assert _rel(od.numpy(), want) <= 1e-6, i
            assert _rel(od.numpy(), ref) <= 1e-3, i
            for a in (xd, od, idd, wd):
                a.free()
        with pytest.raises(UnsupportedError, match="shared FFN"):
            xd, od = DeviceArray.from_numpy(c["x"]), DeviceArray((D,), np.float32)
            try:
                ctx.moe_forward_noalloc(od, xd, *tens, 8, w4.d_expert, act=lt.ACT_GELU_TANH, shared=sh,
                                        deterministic=True)
            finally:
                xd.free()
                od.free()
        # a smaller layer next on the same scratch
        w = synth.config3()["weights"]
        x = synth.normal(synth.stream(3, 77), (w.d_model,))
        t3 = lt.upload_moe(ctx, w)
        got = _run(ctx, ctx.moe_forward_noalloc, t3, x, 8, w.d_expert, False, True)
        ref, rids, _, agree = orc.moe_forward(w, x, 8, norm_topk=True, pool=pool)
        assert agree and np.array_equal(got[1], rids)
        assert _rel(got[0], ref) <= 1e-3
        for t in list(tens) + list(sh) + list(t3):
            t.free()


def test_noalloc_rejects_what_it_cannot_run():
    w = synth.moe_weights(42, 512, 16, 256)
    x = synth.normal(synth.stream(42, 7), (512,))
    with lt.Context(0) as ctx:
        tens = lt.upload_moe(ctx, w)
        xd, od = DeviceArray.from_numpy(x), DeviceArray((512,), np.float32)
        with pytest.raises(InvalidError, match="device arrays only"):
            ctx.moe_forward_noalloc(np.zeros(512, np.float32), x, *tens, 2, 256)
        big = synth.moe_weights(43, 4352, 8, 256)  # d_model above 4096
        tb = lt.upload_moe(ctx, big)
        xb, ob = DeviceArray((4352,), np.float32), DeviceArray((4352,), np.float32)
        with pytest.raises(UnsupportedError, match="beyond the static scratch"):
            ctx.moe_forward_noalloc(ob, xb, *tb, 2, 256)
        ctx.moe_forward_noalloc(od, xd, *tens, 2, 256)  # still usable
        ctx.sync()
        ref, *_ = orc.moe_forward(w, x, 2)
        assert _rel(od.numpy(), ref) <= 1e-3
        for a in (xd, od, xb, ob):
            a.free()
        for t in tens + tb:
            t.free()
