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
