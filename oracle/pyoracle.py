"""ctypes wrapper of the CPU oracle (oracle/build/liblt_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the timed CPU
baseline, never as part of the product path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# LT_ORACLE_LIB selects another build of the same library (the sanitizer
# build, oracle/build/asan/liblt_oracle.so)
LIB_PATH = os.environ.get("LT_ORACLE_LIB") or os.path.join(HERE, "build", "liblt_oracle.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
Q5_0, Q5_1, Q3_K, IQ4_NL = 6, 7, 11, 20
ACT_SILU, ACT_GELU_TANH = 0, 1
NORM_TOPK = 1

_lib = None


class Stats(C.Structure):
    _fields_ = [("max", C.c_float), ("exp_sum", C.c_float)]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} not built: run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        vp, sz, u32, f = C.c_void_p, C.c_size_t, C.c_uint32, C.c_float
        sigs = {
            "lto_f16_to_f32": (f, [C.c_uint16]),
            "lto_dequant_q8_0": (None, [vp, vp, sz]),
            "lto_dequant_q4_k": (None, [vp, vp, sz]),
            "lto_dequant_q6_k": (None, [vp, vp, sz]),
            "lto_dequant_f16": (None, [vp, vp, sz]),
            "lto_dot_q8_0": (f, [vp, vp, sz]),
            "lto_dotf32": (f, [vp, vp, sz]),
            "lto_row_bytes": (sz, [u32, sz]),
            "lto_dequant_row": (C.c_int, [vp, vp, u32, sz]),
            "lto_matvec_f32": (None, [vp, vp, vp, sz, sz]),
            "lto_quant_matvec": (C.c_int, [vp, vp, u32, vp, sz, sz, vp]),
            "lto_quant_matvec_par": (C.c_int, [vp, vp, u32, vp, sz, sz, vp, vp]),
            "lto_softmax": (None, [vp, sz]),
            "lto_silu": (f, [f]),
            "lto_gelu": (f, [f]),
            "lto_pool_create": (vp, [C.c_int]),
            "lto_pool_destroy": (None, [vp]),
            "lto_pool_threads": (C.c_int, [vp]),
            "lto_topk": (None, [vp, sz, vp, sz]),
            "lto_topk_softmax_stats": (Stats, [vp, sz, vp, sz]),
            "lto_softmax_topk": (None, [vp, sz, vp, sz]),
            "lto_topk_matvec_f32": (Stats, [vp, vp, sz, sz, vp, vp, sz]),
            "lto_topk_matvec_f32_par": (Stats, [vp, vp, sz, sz, vp, vp, sz, vp]),
            "lto_router_topk_softmax": (C.c_int, [vp, vp, sz, vp, u32, sz, sz, vp, vp, vp]),
            "lto_moe_forward": (C.c_int, [vp, vp, sz, vp, vp, u32, vp, u32, sz, vp, sz, sz, sz, u32, u32, vp, vp,
                                          vp, vp]),
            "lto_moe_layer_shared": (C.c_int, [vp, vp, sz, vp, u32, sz, vp, u32, vp, u32, sz, sz, sz, vp, vp, vp,
                                               u32, sz, u32, vp, vp, vp]),
            "lto_ffn_dense": (C.c_int, [vp, vp, vp, vp, u32, vp, sz, sz, u32, vp]),
            "lto_moe_prefill": (C.c_int, [vp, vp, sz, vp, sz, vp, vp, u32, vp, u32, sz, sz, sz, sz, u32, u32, vp,
                                          vp, vp]),
            "lto_dot_q5_0": (f, [vp, vp, sz]),
            "lto_dot_iq4_nl": (f, [vp, vp, sz]),
            "lto_q3k_scales": (None, [vp, vp]),
            "lto_rmsnorm": (None, [vp, vp, vp, sz, f, C.c_int]),
            "lto_add_rmsnorm": (None, [vp, vp, vp, vp, sz, f, C.c_int]),
            "lto_rmsnorm_wrs": (None, [vp, vp, vp, vp, vp, f, sz, f]),
            "lto_moe_tail": (None, [vp, vp, vp, vp, vp, f, sz, f]),
            "lto_gemma4_moe_block": (C.c_int, [vp, vp, sz, vp, u32, sz, vp, u32, vp, u32, sz, sz, sz, vp, vp, vp,
                                               vp, vp, f, f, u32, vp, vp, vp]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a).view(np.uint8)


class Pool:
    """The persistent thread pool (thread_pool.zig)."""

    def __init__(self, n_threads: int):
        self.ptr = lib().lto_pool_create(int(n_threads))
        self.n = int(n_threads)

    def close(self):
        if self.ptr:
            lib().lto_pool_destroy(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def _pp(pool):
    return pool.ptr if pool is not None else None


def _gut(w):
    return getattr(w, "gate_up_type", Q4_K)


def _dnt(w):
    return getattr(w, "down_type", Q4_K)


def f16_to_f32(raw: int) -> float:
    return float(np.float32(lib().lto_f16_to_f32(int(raw))))


def dequant(ggml_type: int, data: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    d = _u8(data)
    rc = lib().lto_dequant_row(_p(d), _p(out), ggml_type, n)
    if rc:
        raise ValueError(f"unsupported type {ggml_type}")
    return out


def dot_q8_0(data, vec) -> np.float32:
    vec = _f32(vec)
    d = _u8(data)
    return np.float32(lib().lto_dot_q8_0(_p(d), _p(vec), vec.size))


def dot_q5_0(data, vec) -> np.float32:
    vec = _f32(vec)
    return np.float32(lib().lto_dot_q5_0(_p(_u8(data)), _p(vec), vec.size))


def dot_iq4_nl(data, vec) -> np.float32:
    vec = _f32(vec)
    return np.float32(lib().lto_dot_iq4_nl(_p(_u8(data)), _p(vec), vec.size))


def q3k_scales(scales12) -> np.ndarray:
    out = np.zeros(16, np.uint8)
    lib().lto_q3k_scales(_p(_u8(np.ascontiguousarray(scales12, np.uint8))), _p(out))
    return out


def dotf32(a, b) -> np.float32:
    a, b = _f32(a), _f32(b)
    return np.float32(lib().lto_dotf32(_p(a), _p(b), a.size))


def row_bytes(ggml_type: int, cols: int) -> int:
    return int(lib().lto_row_bytes(ggml_type, cols))


def matvec_f32(mat, vec) -> np.ndarray:
    mat, vec = _f32(mat), _f32(vec)
    rows, cols = mat.shape
    out = np.zeros(rows, dtype=np.float32)
    lib().lto_matvec_f32(_p(out), _p(mat), _p(vec), rows, cols)
    return out


def quant_matvec(data, ggml_type, vec, rows, cols, pool: Pool | None = None) -> np.ndarray:
    vec = _f32(vec)
    d = _u8(data)
    out = np.zeros(rows, dtype=np.float32)
    n = pool.n if pool else 1
    scratch = np.zeros(max(n, 1) * cols, dtype=np.float32)
    if pool is None:
        rc = lib().lto_quant_matvec(_p(out), _p(d), ggml_type, _p(vec), rows, cols, _p(scratch))
    else:
        rc = lib().lto_quant_matvec_par(_p(out), _p(d), ggml_type, _p(vec), rows, cols, _p(scratch), pool.ptr)
    if rc:
        raise ValueError("quant_matvec failed")
    return out


def softmax(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().lto_softmax(_p(x), x.size)
    return x


def silu(x: float) -> np.float32:
    return np.float32(lib().lto_silu(float(x)))


def gelu(x: float) -> np.float32:
    return np.float32(lib().lto_gelu(float(x)))


def topk(scores, k) -> np.ndarray:
    s = _f32(scores)
    out = np.zeros(k, dtype=np.uintp)
    lib().lto_topk(_p(s), s.size, _p(out), k)
    return out.astype(np.int64)


def topk_softmax_stats(scores, k):
    s = _f32(scores)
    out = np.zeros(k, dtype=np.uintp)
    st = lib().lto_topk_softmax_stats(_p(s), s.size, _p(out), k)
    return out.astype(np.int64), np.float32(st.max), np.float32(st.exp_sum)


def softmax_topk(scores, k):
    s = _f32(scores).copy()
    out = np.zeros(k, dtype=np.uintp)
    lib().lto_softmax_topk(_p(s), s.size, _p(out), k)
    return out.astype(np.int64), s


def topk_matvec_f32(w, vec, k, pool: Pool | None = None):
    w, vec = _f32(w), _f32(vec)
    rows, cols = w.shape
    out = np.zeros(k, dtype=np.uintp)
    sel = np.zeros(k, dtype=np.float32)
    if pool is None:
        st = lib().lto_topk_matvec_f32(_p(w), _p(vec), rows, cols, _p(out), _p(sel), k)
    else:
        st = lib().lto_topk_matvec_f32_par(_p(w), _p(vec), rows, cols, _p(out), _p(sel), k, pool.ptr)
    return out.astype(np.int64), sel, np.float32(st.max), np.float32(st.exp_sum)


def router_topk_softmax(router, router_type, rows, cols, x, k, pool: Pool | None = None):
    """routerTopKSoftmax: returns (ids, scores) with the selected probabilities at ids."""
    x = _f32(x)
    r = _u8(router)
    scores = np.zeros(rows, dtype=np.float32)
    out = np.zeros(k, dtype=np.uintp)
    n = pool.n if pool else 1
    scratch = np.zeros(max(n, 1) * cols, dtype=np.float32)
    rc = lib().lto_router_topk_softmax(_p(scores), _p(out), k, _p(r), router_type, rows, cols, _p(x),
                                       _p(scratch), _pp(pool))
    if rc:
        raise ValueError("router_topk_softmax failed")
    return out.astype(np.int64), scores


def moe_forward(w, x, k, act=ACT_SILU, norm_topk=False, bias=None, pool: Pool | None = None, out=None):
    """moeForward on a synth.MoEWeights; returns (out, ids, weights, logit_order_agrees)."""
    x = _f32(x)
    o = np.zeros(w.d_model, dtype=np.float32) if out is None else _f32(out).copy()
    ids = np.zeros(k, dtype=np.uint32)
    wt = np.zeros(k, dtype=np.float32)
    agree = C.c_int(0)
    b = None if bias is None else _f32(bias)
    rc = lib().lto_moe_forward(_p(o), _p(_f32(w.router)), w.n_experts, _p(b), _p(_u8(w.gate_up)), _gut(w),
                               _p(_u8(w.down)), _dnt(w), w.down_cols, _p(x), w.d_model, k, w.d_expert, act,
                               NORM_TOPK if norm_topk else 0, _pp(pool), _p(ids), _p(wt), C.byref(agree))
    if rc:
        raise ValueError(f"moe_forward failed ({rc})")
    return o, ids, wt, bool(agree.value)


def moe_layer_shared(w, x, k, sh_gate, sh_up, sh_down, d_shared, act=ACT_GELU_TANH, pool: Pool | None = None):
    """Config-4 layer (Gemma4 router + experts + shared Q8_0 FFN)."""
    x = _f32(x)
    out = np.zeros(w.d_model, dtype=np.float32)
    ids = np.zeros(k, dtype=np.uint32)
    wt = np.zeros(k, dtype=np.float32)
    rc = lib().lto_moe_layer_shared(_p(out), _p(x), w.d_model, _p(_u8(w.router)), w.router_type, w.n_experts,
                                    _p(_u8(w.gate_up)), _gut(w), _p(_u8(w.down)), _dnt(w), w.down_cols, k,
                                    w.d_expert,
                                    _p(_u8(sh_gate)), _p(_u8(sh_up)), _p(_u8(sh_down)), Q8_0, d_shared, act,
                                    _pp(pool), _p(ids), _p(wt))
    if rc:
        raise ValueError(f"moe_layer_shared failed ({rc})")
    return out, ids, wt


def ffn_dense(wg, wu, wd, ggml_type, x, d_model, d_ffn, act=ACT_SILU, pool: Pool | None = None):
    x = _f32(x)
    out = np.zeros(d_model, dtype=np.float32)
    rc = lib().lto_ffn_dense(_p(out), _p(_u8(wg)), _p(_u8(wu)), _p(_u8(wd)), ggml_type, _p(x), d_model, d_ffn,
                             act, _pp(pool))
    if rc:
        raise ValueError(f"ffn_dense failed ({rc})")
    return out


def moe_prefill(w, X, k, act=ACT_SILU, norm_topk=False, bias=None, pool: Pool | None = None):
    X = _f32(X)
    T = X.shape[0]
    out = np.zeros((T, w.d_model), dtype=np.float32)
    ids = np.zeros((T, k), dtype=np.uint32)
    wt = np.zeros((T, k), dtype=np.float32)
    b = None if bias is None else _f32(bias)
    rc = lib().lto_moe_prefill(_p(out), _p(X), T, _p(_f32(w.router)), w.n_experts, _p(b), _p(_u8(w.gate_up)),
                               Q4_K, _p(_u8(w.down)), Q4_K, w.down_cols, w.d_model, k, w.d_expert, act,
                               NORM_TOPK if norm_topk else 0, _pp(pool), _p(ids), _p(wt))
    if rc:
        raise ValueError(f"moe_prefill failed ({rc})")
    return out, ids, wt


# ---------------------------------------------------------------- norms, Gemma4 block
def rmsnorm(x, w=None, eps=1e-6, one_plus_w=False) -> np.ndarray:
    """math.rmsnorm (w given) / rmsnormRaw (w None)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().lto_rmsnorm(_p(out), _p(x), None if w is None else _p(_f32(w)), x.size, eps, int(one_plus_w))
    return out


def add_rmsnorm(a, b, w, eps=1e-6, one_plus_w=False) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().lto_add_rmsnorm(_p(out), _p(a), _p(b), _p(_f32(w)), a.size, eps, int(one_plus_w))
    return out


def rmsnorm_wrs(x, w, raw_scale, raw_global_scale, eps=1e-6):
    """math.rmsnormWeightedAndRawScaled: returns (weighted, raw_scaled)."""
    x = _f32(x)
    wo, ro = np.empty_like(x), np.empty_like(x)
    lib().lto_rmsnorm_wrs(_p(wo), _p(ro), _p(x), _p(_f32(w)), _p(_f32(raw_scale)), raw_global_scale, x.size, eps)
    return wo, ro


def moe_tail(x, moe, ffn, post_ffw_norm_2, post_ffw_norm, layer_output_scale=1.0, eps=1e-6) -> np.ndarray:
    """gemma4/forward.zig:482-497 on copies; returns the new x."""
    x, moe, ffn = _f32(x).copy(), _f32(moe).copy(), _f32(ffn).copy()
    lib().lto_moe_tail(_p(x), _p(moe), _p(ffn), _p(_f32(post_ffw_norm_2)), _p(_f32(post_ffw_norm)),
                       layer_output_scale, x.size, eps)
    return x


def gemma4_moe_block(w, x, dense_ffn, k, norms, layer_output_scale=1.0, eps=1e-6, act=ACT_GELU_TANH,
                     pool: Pool | None = None):
    """gemma4/forward.zig:403-497 on a synth.MoEWeights; norms: dict with
    pre_ffw_norm_2, router_scale, down_exps_scale (or None), post_ffw_norm_2,
    post_ffw_norm.  Returns (new x, ids, router probabilities)."""
    x = _f32(x).copy()
    ids = np.zeros(k, dtype=np.uint32)
    wt = np.zeros(k, dtype=np.float32)
    ds = norms.get("down_exps_scale")
    rc = lib().lto_gemma4_moe_block(
        _p(x), _p(_f32(dense_ffn)), w.d_model, _p(_u8(w.router)), w.router_type, w.n_experts, _p(_u8(w.gate_up)),
        _gut(w), _p(_u8(w.down)), _dnt(w), w.down_cols, k, w.d_expert, _p(_f32(norms["pre_ffw_norm_2"])),
        _p(_f32(norms["router_scale"])), None if ds is None else _p(_f32(ds)), _p(_f32(norms["post_ffw_norm_2"])),
        _p(_f32(norms["post_ffw_norm"])), layer_output_scale, eps, act, _pp(pool), _p(ids), _p(wt))
    if rc:
        raise ValueError(f"gemma4_moe_block failed ({rc})")
    return x, ids, wt
