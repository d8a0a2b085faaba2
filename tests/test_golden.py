"""The committed golden fixtures (tests/golden/golden.npz) against the
generators and the oracle: inputs hash to the stored SHA-256, and the oracle
reproduces the stored outputs bit for bit."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402

GOLD = np.load(os.path.join(HERE, "golden", "golden.npz"))
CASES = make_golden.cases()


def _parts(d):
    from llmtoy_amd import synth
    if isinstance(d.get("w"), synth.MoEWeights):
        w = d["w"]
        return [w.router, w.gate_up, w.down, d["x"]] + ([d["bias"]] if d["bias"] is not None else [])
    return [d["w"], d["x"]]


@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_inputs_and_oracle_outputs(name):
    builder, runner = CASES[name]
    d = make_golden.build_inputs(name, builder)
    assert make_golden.sha(*_parts(d)) == bytes(GOLD[f"{name}.sha256"]).decode()
    res = runner(d)
    for k, v in res.items():
        assert np.array_equal(np.asarray(v), GOLD[f"{name}.{k}"]), (name, k)
