"""Pins of the oracle's RMS norms, the Gemma4 MoE tail and the Gemma4 MoE
block (oracle/lt_oracle.c: lto_rmsnorm, lto_add_rmsnorm, lto_rmsnorm_wrs,
lto_moe_tail, lto_gemma4_moe_block).

The reference sums the squares sequentially in fp32 (math.zig:19-25,
51-82); a hand-derived case fixes that order.  The block is checked against
a float64 restatement built on independent decoders, and that check is
shown to catch plausible mistakes (a dropped norm, a missing scale, a step
out of order)."""
import math

import numpy as np
import pytest

import pyoracle as orc
from llmtoy_amd import ggml, synth
from test_oracle import q4k_decode_np


def test_rmsnorm_reference_kat():
    # math.zig:344-354
    x = np.array([1, 2, 3, 4], np.float32)
    out = orc.rmsnorm(x, np.ones(4, np.float32), 1e-8)
    rms = math.sqrt((1 + 4 + 9 + 16) / 4)
    assert abs(out[0] - 1 / rms) <= 1e-5 and abs(out[3] - 4 / rms) <= 1e-5


def test_rmsnorm_wrs_reference_kat():
    # math.zig:356-376: equals rmsnorm and rmsnormRaw * (global * scale)
    x = np.array([3, -4, 1, 2], np.float32)
    w = np.array([0.5, 1.25, -0.75, 2.0], np.float32)
    s = np.array([2.0, 0.25, -1.0, 0.5], np.float32)
    weighted, raw = orc.rmsnorm_wrs(x, w, s, 0.125, 1e-6)
    want_w = orc.rmsnorm(x, w, 1e-6)
    want_r = orc.rmsnorm(x, None, 1e-6) * (np.float32(0.125) * s)
    assert np.allclose(weighted, want_w, atol=1e-6, rtol=0) and np.allclose(raw, want_r, atol=1e-6, rtol=0)


def test_rmsnorm_sum_is_sequential():
    # x = four 1s then twelve 2^-11 (n = 16, eps 0).  In index order the sum
    # reaches 4, and each further square (2^-22, half an ulp of 4) rounds away
    # (ties to even): ss = 4, ss/n = 1/4, rms_inv = 2 exactly.  Any wider or
    # pairwise sum keeps the small squares (ss = 4 + 12 * 2^-22) and gives an
    # rms_inv 6 ulps below 2.
    t = np.float32(2.0 ** -11)
    x = np.array([1] * 4 + [t] * 12, np.float32)
    w = synth.normal(synth.stream(95, 0), (16,))
    assert np.array_equal(orc.rmsnorm(x, w, 0.0), (x * np.float32(2)) * w)
    wide = np.float32(4) + np.float32(12) * t * t
    assert np.float32(1) / np.sqrt(wide / np.float32(16)) == np.float32(2) - np.float32(6 * 2.0 ** -23)


@pytest.mark.parametrize("c,n", [(0.25, 64), (-8.0, 4096), (2.0 ** -20, 256)])
def test_rmsnorm_power_of_two_closed_form(c, n):
    # x = c (a power of two), n a power of two, eps 0: ss = n c^2 exactly,
    # rms_inv = 1/|c| exactly, so out = sign(c) * w bit for bit.
    w = synth.normal(synth.stream(95, n), (n,))
    x = np.full(n, c, np.float32)
    assert np.array_equal(orc.rmsnorm(x, w, 0.0), np.float32(math.copysign(1, c)) * w)
    assert np.array_equal(orc.rmsnorm(x, w - np.float32(1), 0.0, one_plus_w=True),
                          np.float32(math.copysign(1, c)) * ((np.float32(1) + (w - np.float32(1)))))


def _rms64(x, eps):
    x = x.astype(np.float64)
    return 1 / math.sqrt(float(np.mean(x * x)) + eps)


def test_rmsnorm_vs_float64_and_eps_matters():
    g = synth.stream(96, 0)
    w = synth.normal(g, (2816,))
    for scale, eps in ((1.0, 1e-6), (1e-3, 1e-6)):
        x = (synth.normal(g, (2816,)) * np.float32(scale)).astype(np.float32)
        got = orc.rmsnorm(x, w, eps)
        want = x.astype(np.float64) * _rms64(x, eps) * w
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-6
        if scale < 1:  # here eps is a visible part of the denominator: leaving it out fails
            no_eps = x.astype(np.float64) * _rms64(x, 0.0) * w
            assert np.max(np.abs(got - no_eps)) / np.max(np.abs(want)) > 1e-3


def test_add_rmsnorm_is_rmsnorm_of_rounded_sum():
    g = synth.stream(97, 0)
    a, b, w = (synth.normal(g, (2816,)) for _ in range(3))
    assert np.array_equal(orc.add_rmsnorm(a, b, w, 1e-6), orc.rmsnorm((a + b).astype(np.float32), w, 1e-6))


def _tail64(x, moe, ffn, w2, w, los, eps):
    moe = moe.astype(np.float64) * _rms64(moe, eps) * w2
    c = ffn.astype(np.float64) + moe
    f = c * (1 / math.sqrt(float(np.mean(c * c)) + eps)) * w
    return (x.astype(np.float64) + f) * los


def test_moe_tail_vs_float64_with_teeth():
    g = synth.stream(98, 0)
    n = 2816
    x, moe, ffn = (synth.normal(g, (n,)) for _ in range(3))
    moe = (moe * np.float32(0.05)).astype(np.float32)  # the expert sum is small next to the dense FFN
    nm = synth.gemma4_norms(98, n, 4)
    w2, w = nm["post_ffw_norm_2"], nm["post_ffw_norm"]
    got = orc.moe_tail(x, moe, ffn, w2, w, 0.75)
    want = _tail64(x, moe, ffn, w2, w, 0.75, 1e-6)
    err = lambda a: float(np.linalg.norm(a - want) / np.linalg.norm(want))  # noqa: E731
    assert err(got) < 1e-6
    # plausible mistakes, each restated in float64, are far from the oracle
    c_raw = ffn.astype(np.float64) + moe  # moe not normalised before the add
    no_norm2 = (x + c_raw * (1 / math.sqrt(float(np.mean(c_raw * c_raw)) + 1e-6)) * w) * 0.75
    scale_first = x * 0.75 + (_tail64(np.zeros(n), moe, ffn, w2, w, 1.0, 1e-6))
    no_scale = _tail64(x, moe, ffn, w2, w, 1.0, 1e-6)
    for bad in (no_norm2, scale_first, no_scale):
        assert err(bad) > 1e-2
    # layer_output_scale 0.5 halves the result exactly; 1.0 skips the multiply
    half = orc.moe_tail(x, moe, ffn, w2, w, 0.5)
    assert np.array_equal(half, orc.moe_tail(x, moe, ffn, w2, w, 1.0) * np.float32(0.5))


def q8_0_decode_np(blocks):
    b = blocks.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d * q).reshape(-1)


def _gemma4_block64(w, x, dense, k, nm, los, eps, down_scale=True, pre_norm=True):
    E, D, F, Kd = w.n_experts, w.d_model, w.d_expert, w.down_cols
    r = _rms64(x, eps)
    x64 = x.astype(np.float64)
    moe_in = x64 * r * nm["pre_ffw_norm_2"] if pre_norm else x64
    router_in = x64 * r / math.sqrt(D) * nm["router_scale"]
    R = q8_0_decode_np(w.router).reshape(E, D).astype(np.float64)
    logits = R @ router_in
    p = np.exp(logits - logits.max())
    p /= p.sum()
    order = sorted(range(E), key=lambda e: (-p[e], e))[:k]
    gu = q4k_decode_np(w.gate_up).reshape(E, 2 * F, D).astype(np.float64)
    dn = q4k_decode_np(w.down).reshape(E, D, Kd).astype(np.float64)
    moe = np.zeros(D)
    for e in order:
        g, u = gu[e, :F] @ moe_in, gu[e, F:] @ moe_in
        a = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
        h = np.zeros(Kd)
        h[:F] = a * u
        s = (nm["down_exps_scale"][e] if down_scale else 1.0) * p[e]
        moe += s * (dn[e] @ h)
    return _tail64(x, moe, dense, nm["post_ffw_norm_2"], nm["post_ffw_norm"], los, eps), order


def test_gemma4_block_vs_float64_with_teeth(pool):
    w = synth.moe_weights(99, 512, 16, 192, down_cols=256, router_type=ggml.Q8_0)
    x = synth.normal(synth.stream(99, 1), (512,))
    dense = synth.normal(synth.stream(99, 2), (512,))
    nm = synth.gemma4_norms(99, 512, 16)
    got, ids, wt = orc.gemma4_moe_block(w, x, dense, 4, nm, layer_output_scale=0.75, pool=pool)
    want, order = _gemma4_block64(w, x, dense, 4, nm, 0.75, 1e-6)
    assert ids.tolist() == order
    err = lambda a: float(np.linalg.norm(a - want) / np.linalg.norm(want))  # noqa: E731
    assert err(got) < 1e-5
    # routing probabilities are the softmax over all logits at the selected ids
    router_in = orc.rmsnorm_wrs(x, nm["pre_ffw_norm_2"], nm["router_scale"],
                                np.float32(1) / np.sqrt(np.float32(512)))[1]
    logits = orc.quant_matvec(w.router, orc.Q8_0, router_in, 16, 512)
    ref_ids, probs = orc.softmax_topk(logits, 4)
    assert ids.tolist() == ref_ids.tolist() and np.allclose(wt, probs[ref_ids], rtol=1e-6)
    # the float64 check separates plausible mistakes: no down_exps_scale, no pre-norm of the expert input
    for bad in (_gemma4_block64(w, x, dense, 4, nm, 0.75, 1e-6, down_scale=False)[0],
                _gemma4_block64(w, x, dense, 4, nm, 0.75, 1e-6, pre_norm=False)[0]):
        assert float(np.linalg.norm(bad - want) / np.linalg.norm(want)) > 1e-4
    # and the oracle itself with down_exps_scale dropped moves by as much
    nm1 = dict(nm, down_exps_scale=None)
    got1 = orc.gemma4_moe_block(w, x, dense, 4, nm1, layer_output_scale=0.75, pool=pool)[0]
    assert err(got1) > 1e-4


def test_gemma4_block_thread_invariant():
    w = synth.moe_weights(100, 512, 16, 256, router_type=ggml.Q8_0)
    x = synth.normal(synth.stream(100, 1), (512,))
    dense = synth.normal(synth.stream(100, 2), (512,))
    nm = synth.gemma4_norms(100, 512, 16)
    ref = orc.gemma4_moe_block(w, x, dense, 4, nm)[0]
    with orc.Pool(5) as p:
        assert np.array_equal(orc.gemma4_moe_block(w, x, dense, 4, nm, pool=p)[0], ref)
