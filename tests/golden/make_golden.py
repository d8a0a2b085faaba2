"""Writes tests/golden/golden.npz: small seeded cases with the CPU oracle's
outputs.

The reference (Zig, no toolchain here) cannot be run, and it ships no golden
vectors or fixture files, so these fixtures are produced by the oracle after
it has been pinned by tests/test_oracle.py (reference KATs, independent
decoders, float64 brute force).  They freeze the oracle's outputs so that a
later change to the oracle or to the generators is caught, and they give the
GPU tests known answers that need no oracle build.

Inputs are regenerated from llmtoy_amd.synth seeds; the SHA-256 of every
input is stored next to the outputs so a generator change is detected.

Run:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "llmtoy-zig_amd"), os.path.join(ROOT, "oracle")]

import pyoracle as orc  # noqa: E402
from llmtoy_amd import ggml, synth  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def cases():
    """name -> (builder, runner).  Builders are deterministic."""
    out = {}

    def mv(gtype, rows, cols, valid=None):
        g = synth.stream(70, 100 + gtype)
        if gtype == ggml.F32:
            w = synth.normal(g, (rows, cols), 0.02)
        elif gtype == ggml.Q8_0:
            w = synth.q8_0_matrix(g, rows, cols)
        elif gtype == ggml.Q4_K:
            w = synth.q4k_matrix(g, rows, cols, valid)
        else:
            w = synth.q6k_matrix(g, rows, cols, valid)
        x = synth.normal(g, (cols,))
        if valid:
            x[valid:] = 0
        return dict(w=w, x=x), (lambda d: dict(y=orc.quant_matvec(d["w"], gtype, d["x"], rows, cols)))

    out["mv_f32"] = mv(ggml.F32, 37, 33)
    out["mv_q8_0"] = mv(ggml.Q8_0, 48, 96)
    out["mv_q4_k"] = mv(ggml.Q4_K, 40, 512)
    out["mv_q4_k_pad"] = mv(ggml.Q4_K, 24, 768, valid=704)
    out["mv_q6_k_pad"] = mv(ggml.Q6_K, 24, 1024, valid=896)

    def moe(config, E, D, F, Kd, k, norm, bias, act):
        def build():
            w = synth.moe_weights(config, D, E, F, down_cols=Kd)
            x = synth.normal(synth.stream(config, 7), (D,))
            b = synth.zipf_bias(synth.stream(config, 8), E) if bias else None
            return dict(w=w, x=x, bias=b)

        def run(d):
            o, ids, wt, agree = orc.moe_forward(d["w"], d["x"], k, act=act, norm_topk=norm, bias=d["bias"])
            assert agree
            return dict(out=o, ids=ids, wt=wt)

        return build, run

    out["moe_small"] = moe(71, 6, 256, 128, 256, 2, False, False, orc.ACT_SILU)
    out["moe_small_norm_bias_gelu"] = moe(72, 10, 512, 256, 256, 4, True, True, orc.ACT_GELU_TANH)
    return out


def build_inputs(name, builder):
    if callable(builder):
        return builder()
    return builder


def main():
    blob = {}
    for name, (builder, runner) in cases().items():
        d = build_inputs(name, builder)
        res = runner(d)
        if "w" in d and isinstance(d["w"], synth.MoEWeights):
            w = d["w"]
            parts = [w.router, w.gate_up, w.down, d["x"]] + ([d["bias"]] if d["bias"] is not None else [])
        else:
            parts = [d["w"], d["x"]]
            blob[f"{name}.x"] = d["x"]
            blob[f"{name}.w"] = d["w"]
        blob[f"{name}.sha256"] = np.frombuffer(sha(*parts).encode(), dtype=np.uint8)
        for k, v in res.items():
            blob[f"{name}.{k}"] = v
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **blob)
    print("wrote", os.path.join(HERE, "golden.npz"), len(blob), "arrays")


if __name__ == "__main__":
    main()
