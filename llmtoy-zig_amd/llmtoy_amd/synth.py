"""Seeded synthetic inputs for the five BASELINE configurations.

Every tensor is drawn from its own numpy PCG64 stream seeded with
[0x1A70000 + config, tensor_id], so any tensor can be regenerated alone and
the GPU box and this container produce identical bytes.  Quantised weights
are raw GGUF block bytes (llmtoy-zig src/quant/dequant.zig layouts);
f16 fields are round-to-nearest-even conversions of the fp32 draws.

Value schemes:
  Q8_0 : q ~ U{-127..127}, d = |N(0,1)| * 0.01
  Q4_K : q ~ U{0..15}, 6-bit sc, mn ~ U{0..63}, d = |N|*0.002, dmin = |N|*0.001
  Q6_K : q6 ~ U{0..63} (random ql/qh bytes), int8 sc ~ U{0..63}, d = |N|*0.002
  x ~ N(0,1); fp32 router ~ N(0, 0.02)
Rows whose GGUF length is not a multiple of the block (Q6_K 896, Q4_K 704)
are padded with zero blocks: the padded sub-blocks get zero scales/mins and
zero quants, and the matching x entries are zero.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import ggml

BASE_SEED = 0x1A70000


def stream(config: int, tensor_id: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([BASE_SEED + config, tensor_id]))


def _absn(g, shape, scale):
    return np.abs(g.standard_normal(shape, dtype=np.float32)) * np.float32(scale)


def q8_0_matrix(g: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """uint8 [rows, row_bytes] of Q8_0 blocks."""
    assert cols % 32 == 0
    nb = cols // 32
    d = ggml.f16_bits(_absn(g, (rows, nb), 0.01))
    q = g.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8)
    blk = np.empty((rows, nb, 34), dtype=np.uint8)
    blk[..., 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[..., 2:] = q.view(np.uint8)
    return blk.reshape(rows, nb * 34)


def q4k_matrix(g: np.random.Generator, rows: int, cols: int, valid_cols: int | None = None) -> np.ndarray:
    """uint8 [rows, row_bytes] of Q4_K super-blocks; elements >= valid_cols are zero."""
    assert cols % 256 == 0
    nsb = cols // 256
    d = ggml.f16_bits(_absn(g, (rows, nsb), 0.002))
    dmin = ggml.f16_bits(_absn(g, (rows, nsb), 0.001))
    sc = g.integers(0, 64, size=(rows, nsb, 8), dtype=np.uint8)
    mn = g.integers(0, 64, size=(rows, nsb, 8), dtype=np.uint8)
    qs = g.integers(0, 256, size=(rows, nsb, 128), dtype=np.uint8)
    if valid_cols is not None and valid_cols < cols:
        assert valid_cols % 32 == 0
        for sub in range(valid_cols // 32, cols // 32):
            sb, j = divmod(sub, 8)
            sc[:, sb, j] = 0
            mn[:, sb, j] = 0
            p, hi = divmod(j, 2)
            qs[:, sb, 32 * p:32 * p + 32] &= np.uint8(0x0F if hi else 0xF0)
    blk = np.empty((rows, nsb, 144), dtype=np.uint8)
    blk[..., 0:2] = d.view(np.uint8).reshape(rows, nsb, 2)
    blk[..., 2:4] = dmin.view(np.uint8).reshape(rows, nsb, 2)
    blk[..., 4:16] = ggml.pack_q4k_scales(sc, mn)
    blk[..., 16:] = qs
    return blk.reshape(rows, nsb * 144)


def q6k_matrix(g: np.random.Generator, rows: int, cols: int, valid_cols: int | None = None) -> np.ndarray:
    """uint8 [rows, row_bytes] of Q6_K super-blocks; elements >= valid_cols are zero."""
    assert cols % 256 == 0
    nsb = cols // 256
    ql = g.integers(0, 256, size=(rows, nsb, 128), dtype=np.uint8)
    qh = g.integers(0, 256, size=(rows, nsb, 64), dtype=np.uint8)
    sc = g.integers(0, 64, size=(rows, nsb, 16), dtype=np.int8)
    d = ggml.f16_bits(_absn(g, (rows, nsb), 0.002))
    if valid_cols is not None and valid_cols < cols:
        assert valid_cols % 128 == 0
        for half in range(valid_cols // 128, cols // 128):
            sb, hf = divmod(half, 2)
            ql[:, sb, 64 * hf:64 * hf + 64] = 0
            qh[:, sb, 32 * hf:32 * hf + 32] = 0
            sc[:, sb, 8 * hf:8 * hf + 8] = 0
    blk = np.empty((rows, nsb, 210), dtype=np.uint8)
    blk[..., 0:128] = ql
    blk[..., 128:192] = qh
    blk[..., 192:208] = sc.view(np.uint8)
    blk[..., 208:210] = d.view(np.uint8).reshape(rows, nsb, 2)
    return blk.reshape(rows, nsb * 210)


def small_block_matrix(g: np.random.Generator, gtype: int, rows: int, cols: int) -> np.ndarray:
    """uint8 [rows, row_bytes] of Q5_0 / Q5_1 / IQ4_NL blocks: uniform quant
    bits, d = |N| * 0.01 (Q5_1 also m = N * 0.01)."""
    assert cols % 32 == 0
    nb = cols // 32
    bb = ggml.BLOCK_BYTES[gtype]
    blk = g.integers(0, 256, size=(rows, nb, bb), dtype=np.uint8)
    blk[..., 0:2] = ggml.f16_bits(_absn(g, (rows, nb), 0.01)).view(np.uint8).reshape(rows, nb, 2)
    if gtype == ggml.Q5_1:
        blk[..., 2:4] = ggml.f16_bits(normal(g, (rows, nb), 0.01)).view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * bb)


def q3k_matrix(g: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """uint8 [rows, row_bytes] of Q3_K super-blocks: uniform hmask/quant/scale
    bytes, d = |N| * 0.002."""
    assert cols % 256 == 0
    nsb = cols // 256
    blk = g.integers(0, 256, size=(rows, nsb, 110), dtype=np.uint8)
    blk[..., 108:110] = ggml.f16_bits(_absn(g, (rows, nsb), 0.002)).view(np.uint8).reshape(rows, nsb, 2)
    return blk.reshape(rows, nsb * 110)


def quant_matrix(g: np.random.Generator, gtype: int, rows: int, cols: int) -> np.ndarray:
    """Random rows of any device-path type."""
    if gtype == ggml.Q8_0:
        return q8_0_matrix(g, rows, cols)
    if gtype == ggml.Q4_K:
        return q4k_matrix(g, rows, cols)
    if gtype == ggml.Q6_K:
        return q6k_matrix(g, rows, cols)
    if gtype == ggml.Q3_K:
        return q3k_matrix(g, rows, cols)
    return small_block_matrix(g, gtype, rows, cols)


def normal(g, shape, scale=1.0) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def zipf_bias(g: np.random.Generator, n_experts: int, s: float = 1.1) -> np.ndarray:
    """bias_e = -s * ln(rank_e), rank = a seeded permutation of 1..n_experts."""
    rank = g.permutation(n_experts) + 1
    return (-np.float32(s) * np.log(rank.astype(np.float32))).astype(np.float32)


@dataclass
class MoEWeights:
    d_model: int
    n_experts: int
    d_expert: int
    down_cols: int
    router: np.ndarray          # fp32 [E, D] or Q8_0 bytes [E, row_bytes]
    router_type: int
    gate_up: np.ndarray         # expert bytes [E * 2F, row_bytes(D)]
    down: np.ndarray            # expert bytes [E * D, row_bytes(down_cols)]
    extra: dict = field(default_factory=dict)
    gate_up_type: int = ggml.Q4_K
    down_type: int = ggml.Q4_K


def moe_weights(config: int, d_model: int, n_experts: int, d_expert: int, down_cols: int | None = None,
                router_type: int = ggml.F32, tid0: int = 0, gate_up_type: int = ggml.Q4_K,
                down_type: int = ggml.Q4_K) -> MoEWeights:
    """Router + flattened expert tensors (gate rows then up rows per expert,
    ops/moe.zig:55-73).  Experts are generated one at a time so a subset of
    experts can be regenerated identically.  Down columns past d_expert are
    zero (K padding)."""
    down_cols = down_cols or d_expert
    if router_type == ggml.F32:
        router = normal(stream(config, tid0 + 1), (n_experts, d_model), 0.02)
    else:
        router = q8_0_matrix(stream(config, tid0 + 1), n_experts, d_model)
    gu_rb = ggml.row_bytes(gate_up_type, d_model)
    dn_rb = ggml.row_bytes(down_type, down_cols)
    gate_up = np.empty((n_experts * 2 * d_expert, gu_rb), dtype=np.uint8)
    down = np.empty((n_experts * d_model, dn_rb), dtype=np.uint8)
    for e in range(n_experts):
        g1, g2 = stream(config, tid0 + 1000 + e), stream(config, tid0 + 5000 + e)
        if gate_up_type == ggml.Q4_K:
            gate_up[e * 2 * d_expert:(e + 1) * 2 * d_expert] = q4k_matrix(g1, 2 * d_expert, d_model)
        else:
            gate_up[e * 2 * d_expert:(e + 1) * 2 * d_expert] = quant_matrix(g1, gate_up_type, 2 * d_expert, d_model)
        if down_type == ggml.Q4_K:
            down[e * d_model:(e + 1) * d_model] = q4k_matrix(g2, d_model, down_cols, valid_cols=d_expert)
        else:
            dm = quant_matrix(g2, down_type, d_model, down_cols)
            be, bb = ggml.BLOCK_ELEMS[down_type], ggml.BLOCK_BYTES[down_type]
            assert d_expert % be == 0
            dm[:, (d_expert // be) * bb:] = 0  # zero blocks: every element 0
            down[e * d_model:(e + 1) * d_model] = dm
    return MoEWeights(d_model, n_experts, d_expert, down_cols, router, router_type, gate_up, down,
                      gate_up_type=gate_up_type, down_type=down_type)


# ---------------------------------------------------------------- configs
def config1(rows_ffn: int = 4864, d_model: int = 896) -> dict:
    """Dense FFN, Qwen2.5-0.5B shape, Q8_0."""
    return dict(
        x=normal(stream(1, 0), (d_model,)),
        w_gate=q8_0_matrix(stream(1, 1), rows_ffn, d_model),
        w_up=q8_0_matrix(stream(1, 2), rows_ffn, d_model),
        w_down=q8_0_matrix(stream(1, 3), d_model, rows_ffn),
        d_model=d_model, d_ffn=rows_ffn)


def config2(n: int = 4096) -> dict:
    """Q4_K matvec [n x n]."""
    return dict(x=normal(stream(2, 0), (n,)), w=q4k_matrix(stream(2, 1), n, n), rows=n, cols=n)


def config2_q6k(rows: int = 151936, cols: int = 896) -> dict:
    """Q6_K output-projection companion, K padded to a multiple of 256."""
    kp = (cols + 255) // 256 * 256
    x = np.zeros(kp, dtype=np.float32)
    x[:cols] = normal(stream(2, 10), (cols,))
    return dict(x=x, w=q6k_matrix(stream(2, 11), rows, kp, valid_cols=cols), rows=rows, cols=kp, valid_cols=cols)


def config3(n_experts: int = 128, d_model: int = 2048, d_expert: int = 768) -> dict:
    """Qwen3-style MoE decode layer: fp32 router, Q4_K experts, SiLU, top-8, renormalised."""
    w = moe_weights(3, d_model, n_experts, d_expert)
    return dict(x=normal(stream(3, 0), (d_model,)), weights=w, k=8)


def config3_x(i: int, d_model: int = 2048) -> np.ndarray:
    """The i-th input of a pool of decode inputs for config 3 (bench rotation)."""
    return normal(stream(3, 100000 + i), (d_model,))


def config4(n_experts: int = 128, d_model: int = 2816, d_expert: int = 704, d_shared: int = 2112) -> dict:
    """Gemma4-A4B-like layer: Q8_0 router and shared FFN, Q4_K experts, GELU-tanh, top-8."""
    down_cols = (d_expert + 255) // 256 * 256
    w = moe_weights(4, d_model, n_experts, d_expert, down_cols=down_cols, router_type=ggml.Q8_0)
    return dict(
        x=normal(stream(4, 0), (d_model,)), weights=w, k=8,
        sh_gate=q8_0_matrix(stream(4, 20), d_shared, d_model),
        sh_up=q8_0_matrix(stream(4, 21), d_shared, d_model),
        sh_down=q8_0_matrix(stream(4, 22), d_model, d_shared),
        d_shared=d_shared)


def gemma4_norms(config: int, d_model: int, n_experts: int, tid0: int = 40) -> dict:
    """Norm and scale vectors of one Gemma4 MoE block (gemma4/weights.zig:
    pre_ffw_norm_2, router_scale, down_exps_scale, post_ffw_norm_2,
    post_ffw_norm), drawn around 1 so that no step is an identity."""
    def around1(tid, n, sd):
        return (1.0 + sd * stream(config, tid0 + tid).standard_normal(n)).astype(np.float32)
    return dict(pre_ffw_norm_2=around1(0, d_model, 0.2), router_scale=around1(1, d_model, 0.1),
                down_exps_scale=around1(2, n_experts, 0.25), post_ffw_norm_2=around1(3, d_model, 0.2),
                post_ffw_norm=around1(4, d_model, 0.2))


def config4_block(n_experts: int = 128, d_model: int = 2816, d_expert: int = 704) -> dict:
    """The config-4 layer inside a Gemma4 block: x (residual stream), the
    dense FFN output after post_ffw_norm_1, norm vectors, Q8_0 router, Q4_K
    experts (K padded to 768), GELU, top-8, layer_output_scale 0.75."""
    down_cols = (d_expert + 255) // 256 * 256
    w = moe_weights(4, d_model, n_experts, d_expert, down_cols=down_cols, router_type=ggml.Q8_0)
    return dict(x=normal(stream(4, 50), (d_model,)), dense_ffn=normal(stream(4, 51), (d_model,)), weights=w, k=8,
                norms=gemma4_norms(4, d_model, n_experts), layer_output_scale=0.75, eps=1e-6)


def config5(T: int = 512, weights: MoEWeights | None = None) -> dict:
    """Batched prefill of the config-3 layer with Zipf-biased router logits."""
    w = weights if weights is not None else moe_weights(3, 2048, 128, 768)
    return dict(X=normal(stream(5, 0), (T, w.d_model)), bias=zipf_bias(stream(5, 1), w.n_experts), weights=w, k=8,
                T=T)
