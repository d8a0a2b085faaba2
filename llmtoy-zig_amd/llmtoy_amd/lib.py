"""ctypes binding of libllmtoy_hip.so (include/llmtoy_hip.h).

Python mirror of llmtoy-zig's op-level API on the decode path:
  quant_matvec(out, W, x)        <- ops/math.zig:133-171 quantMatvec
  moe_forward(out, x, router, gate_up, down, k, d_expert)
                                 <- ops/moe.zig:18-77 moeForward
  run_expert_batch(...)          <- gemma4/gpu_weights.zig:2748 runExpertBatch
Errors: the C status codes become LtError subclasses.  UnsupportedError is
the reference's "fall back to the CPU path" condition (a null MatvecSession
or error.ExpertNotOnGpu); InvalidError stands for the reference's shape
assertions.

Arrays: numpy arrays are host memory (the call is synchronous, LT_HOST_IO);
llmtoy_amd.hip.DeviceArray (or a CUDA tensor of a framework that shares this
HIP runtime) is passed as a device pointer (the call is enqueued on the
context's stream; call Context.sync()).  There is no CPU fallback here: the
library must be built (make -C llmtoy-zig_amd) and a GPU must be present.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import ggml

LT_OK, LT_ERR_UNSUPPORTED, LT_ERR_INVALID, LT_ERR_DEVICE, LT_ERR_OOM = range(5)
LT_HOST_IO, LT_MOE_NORM_TOPK, LT_MOE_ACCUMULATE = 1, 2, 4
LT_MOE_UNFUSED = 1 << 3
LT_MOE_DETERMINISTIC = 1 << 4
LT_NORM_PRECISE = 1 << 5
LT_NORM_ONE_PLUS_W = 1 << 6
ACT_SILU, ACT_GELU_TANH = 0, 1

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libllmtoy_hip.so")


class LtError(RuntimeError):
    code = -1

    def __init__(self, msg, code=None):
        super().__init__(msg)
        if code is not None:
            self.code = code


class UnsupportedError(LtError):
    code = LT_ERR_UNSUPPORTED


class InvalidError(LtError):
    code = LT_ERR_INVALID


class DeviceError(LtError):
    code = LT_ERR_DEVICE


class OomError(LtError):
    code = LT_ERR_OOM


_ERRS = {LT_ERR_UNSUPPORTED: UnsupportedError, LT_ERR_INVALID: InvalidError, LT_ERR_DEVICE: DeviceError,
         LT_ERR_OOM: OomError}

EXPORTS = [
    "lt_init", "lt_destroy", "lt_last_error", "lt_sync", "lt_stream", "lt_tensor_upload", "lt_tensor_read", "lt_tensor_clone",
    "lt_tensor_free", "lt_tensor_bytes", "lt_stream_read", "lt_matvec", "lt_ffn_dense", "lt_moe_router_topk", "lt_expert_gate_up_id",
    "lt_expert_down_id", "lt_moe_forward", "lt_moe_forward_noalloc", "lt_moe_prefill", "lt_rmsnorm", "lt_add_rmsnorm",
    "lt_rmsnorm_weighted_raw_scaled", "lt_moe_tail", "lt_gemma4_moe_block", "lt_profile_report",
]

_lib = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load libllmtoy_hip.so and declare signatures.  Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run `make -C llmtoy-zig_amd` (or __graft_entry__.build())")
    lib = C.CDLL(path)
    vp, sz, u32, i32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int
    sig = {
        "lt_init": (i32, [i32, C.POINTER(vp)]),
        "lt_destroy": (None, [vp]),
        "lt_last_error": (C.c_char_p, [vp]),
        "lt_sync": (i32, [vp]),
        "lt_stream": (vp, [vp]),
        "lt_tensor_upload": (i32, [vp, vp, sz, u32, sz, sz, sz, C.POINTER(vp)]),
        "lt_tensor_read": (i32, [vp, vp, vp, sz]),
        "lt_tensor_clone": (i32, [vp, vp, C.POINTER(vp)]),
        "lt_tensor_free": (i32, [vp, vp]),
        "lt_tensor_bytes": (sz, [vp]),
        "lt_stream_read": (i32, [vp, vp, sz]),
        "lt_matvec": (i32, [vp, vp, vp, vp, u32]),
        "lt_ffn_dense": (i32, [vp, vp, vp, vp, vp, vp, u32, u32]),
        "lt_moe_router_topk": (i32, [vp, vp, vp, vp, u32, u32, vp, vp, vp]),
        "lt_expert_gate_up_id": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp, u32]),
        "lt_expert_down_id": (i32, [vp, vp, vp, vp, vp, u32, vp, u32]),
        "lt_moe_forward": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp]),
        "lt_moe_forward_noalloc": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp]),
        "lt_moe_prefill": (i32, [vp, vp, vp, u32, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp]),
        "lt_rmsnorm": (i32, [vp, vp, vp, vp, u32, u32, C.c_float, u32]),
        "lt_add_rmsnorm": (i32, [vp, vp, vp, vp, vp, u32, u32, C.c_float, u32]),
        "lt_rmsnorm_weighted_raw_scaled": (i32, [vp, vp, vp, vp, vp, vp, C.c_float, u32, C.c_float, u32]),
        "lt_moe_tail": (i32, [vp, vp, vp, vp, vp, vp, C.c_float, u32, C.c_float, u32]),
        "lt_profile_report": (sz, [vp, vp, sz]),
        "lt_gemma4_moe_block": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_float, C.c_float, u32, u32,
                                      u32, u32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _is_torch(a) -> bool:
    return type(a).__module__.startswith("torch")


def _ptr(a):
    """(pointer, is_host) of a numpy array or torch CUDA tensor; None passes through."""
    if a is None:
        return None, None
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise InvalidError("array must be C-contiguous")
        return a.ctypes.data, True
    if hasattr(a, "ptr") and hasattr(a, "dtype"):  # hip.DeviceArray / DeviceView
        return a.ptr, False
    if _is_torch(a):
        if not a.is_contiguous():
            raise InvalidError("tensor must be contiguous")
        return a.data_ptr(), not a.is_cuda
    raise TypeError(f"unsupported array type {type(a)}")


class Tensor:
    """A device-resident GGUF tensor (MatvecSession / GpuWeights upload)."""

    def __init__(self, ctx: "Context", handle, ggml_type, rows, cols, n_experts):
        self.ctx, self.handle = ctx, handle
        self.type, self.rows, self.cols, self.n_experts = ggml_type, rows, cols, n_experts

    @property
    def nbytes(self) -> int:
        return int(self.ctx.lib.lt_tensor_bytes(self.handle))

    def read(self) -> np.ndarray:
        """The tensor's GGUF block bytes, read back from the device."""
        out = np.empty(self.nbytes, np.uint8)
        self.ctx._check(self.ctx.lib.lt_tensor_read(self.ctx.ptr, self.handle, out.ctypes.data, out.nbytes))
        return out

    def clone(self) -> "Tensor":
        h = C.c_void_p()
        self.ctx._check(self.ctx.lib.lt_tensor_clone(self.ctx.ptr, self.handle, C.byref(h)))
        return Tensor(self.ctx, h, self.type, self.rows, self.cols, self.n_experts)

    def free(self):
        if self.handle:
            self.ctx.lib.lt_tensor_free(self.ctx.ptr, self.handle)
            self.handle = None


class Context:
    """One device context (GpuContext + GpuWeights)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        p = C.c_void_p()
        rc = self.lib.lt_init(device, C.byref(p))
        if rc != LT_OK:
            raise _ERRS.get(rc, LtError)(f"lt_init({device}) failed with status {rc}", rc)
        self.ptr = p

    def close(self):
        if self.ptr:
            self.lib.lt_destroy(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, rc):
        if rc != LT_OK:
            msg = self.lib.lt_last_error(self.ptr).decode(errors="replace")
            raise _ERRS.get(rc, LtError)(msg, rc)

    def sync(self):
        self._check(self.lib.lt_sync(self.ptr))

    def profile_report(self) -> str:
        """lt_profile_report: the LT_PROFILE tables ("" when profiling is off)."""
        n = int(self.lib.lt_profile_report(self.ptr, None, 0))
        if n == 0:
            return ""
        buf = C.create_string_buffer(n + 1)
        self.lib.lt_profile_report(self.ptr, buf, n + 1)
        return buf.value.decode(errors="replace")

    @property
    def stream(self) -> int:
        return int(self.lib.lt_stream(self.ptr) or 0)

    def upload(self, data: np.ndarray, ggml_type: int, rows: int, cols: int, n_experts: int = 1) -> Tensor:
        data = np.ascontiguousarray(data)
        h = C.c_void_p()
        self._check(self.lib.lt_tensor_upload(self.ptr, data.ctypes.data, data.nbytes, ggml_type, rows, cols,
                                               n_experts, C.byref(h)))
        return Tensor(self, h, ggml_type, rows, cols, n_experts)

    # ---- op-level mirror ------------------------------------------------
    def _io(self, *arrays):
        kinds = {_ptr(a)[1] for a in arrays if a is not None}
        if len(kinds) > 1:
            raise InvalidError("mix of host and device arrays")
        return LT_HOST_IO if kinds == {True} else 0

    def quant_matvec(self, out, W: Tensor, x):
        """out[rows] = W . x (quantMatvec, ops/math.zig:133-171)."""
        fl = self._io(out, x)
        self._check(self.lib.lt_matvec(self.ptr, _ptr(out)[0], W.handle, _ptr(x)[0], fl))
        return out

    def stream_read(self, ptr: int, nbytes: int):
        """Enqueue one read of nbytes of device memory at ptr (the read-ceiling probe)."""
        self._check(self.lib.lt_stream_read(self.ptr, C.c_void_p(ptr), nbytes))

    def ffn_dense(self, out, Wg: Tensor, Wu: Tensor, Wd: Tensor, x, act=ACT_SILU, unfused=False):
        """unfused: gate/up and down as two launches instead of the single-launch kernel."""
        fl = self._io(out, x) | (LT_MOE_UNFUSED if unfused else 0)
        self._check(self.lib.lt_ffn_dense(self.ptr, _ptr(out)[0], Wg.handle, Wu.handle, Wd.handle, _ptr(x)[0],
                                          act, fl))
        return out

    def router_topk(self, router: Tensor, x, k: int, ids, weights, bias=None, norm_topk=False, scores=None):
        """routerTopKSoftmax (gemma4/forward.zig:648-668): ids/weights in selection order;
        scores (optional) gets logits of unselected and probabilities of selected experts."""
        fl = self._io(x, ids, weights, bias, scores) | (LT_MOE_NORM_TOPK if norm_topk else 0)
        self._check(self.lib.lt_moe_router_topk(self.ptr, router.handle, _ptr(x)[0], _ptr(bias)[0], k, fl,
                                                _ptr(ids)[0], _ptr(weights)[0], _ptr(scores)[0]))

    def expert_gate_up_id(self, gate_up: Tensor, x, ids, k, d_expert, down_cols, h, act=ACT_SILU):
        fl = self._io(x, ids, h)
        self._check(self.lib.lt_expert_gate_up_id(self.ptr, gate_up.handle, _ptr(x)[0], _ptr(ids)[0], k, d_expert,
                                                  down_cols, act, _ptr(h)[0], fl))

    def expert_down_id(self, down: Tensor, h, ids, weights, k, out, accumulate=False):
        fl = self._io(h, ids, weights, out) | (LT_MOE_ACCUMULATE if accumulate else 0)
        self._check(self.lib.lt_expert_down_id(self.ptr, down.handle, _ptr(h)[0], _ptr(ids)[0], _ptr(weights)[0],
                                               k, _ptr(out)[0], fl))

    def moe_forward(self, out, x, router: Tensor, gate_up: Tensor, down: Tensor, k: int, d_expert: int,
                    act=ACT_SILU, norm_topk=False, accumulate=False, bias=None, shared=None, out_ids=None,
                    out_w=None, unfused=False, deterministic=False):
        """One token through the MoE layer (moeForward, ops/moe.zig:18-77).

        shared = (Wg, Wu, Wd) adds a dense shared FFN (Gemma4 layer).
        unfused = True runs router, gate/up and down as separate launches
        instead of the single-launch kernel.  deterministic = True adds the
        expert outputs in slot order (bit-identical run to run); by default
        the single-launch kernel adds them with float atomics."""
        fl = self._io(out, x, bias, out_ids, out_w)
        fl |= (LT_MOE_NORM_TOPK if norm_topk else 0) | (LT_MOE_ACCUMULATE if accumulate else 0)
        fl |= LT_MOE_UNFUSED if unfused else 0
        fl |= LT_MOE_DETERMINISTIC if deterministic else 0
        sg, su, sd = (t.handle for t in shared) if shared else (None, None, None)
        self._check(self.lib.lt_moe_forward(self.ptr, _ptr(out)[0], _ptr(x)[0], router.handle, _ptr(bias)[0],
                                            gate_up.handle, down.handle, sg, su, sd, k, d_expert, act, fl,
                                            _ptr(out_ids)[0], _ptr(out_w)[0]))
        return out

    def moe_forward_noalloc(self, out, x, router: Tensor, gate_up: Tensor, down: Tensor, k: int, d_expert: int,
                            act=ACT_SILU, norm_topk=False, accumulate=False, bias=None, shared=None, out_ids=None,
                            out_w=None, deterministic=False):
        """lt_moe_forward_noalloc: moe_forward on the library's static scratch
        (no device allocation); device arrays only."""
        fl = (LT_MOE_NORM_TOPK if norm_topk else 0) | (LT_MOE_ACCUMULATE if accumulate else 0)
        fl |= LT_MOE_DETERMINISTIC if deterministic else 0
        if self._io(out, x, bias, out_ids, out_w):
            raise InvalidError("moe_forward_noalloc takes device arrays only")
        sg, su, sd = (t.handle for t in shared) if shared else (None, None, None)
        self._check(self.lib.lt_moe_forward_noalloc(self.ptr, _ptr(out)[0], _ptr(x)[0], router.handle, _ptr(bias)[0],
                                                    gate_up.handle, down.handle, sg, su, sd, k, d_expert, act,
                                                    fl, _ptr(out_ids)[0], _ptr(out_w)[0]))
        return out

    def moe_prefill(self, out, X, router: Tensor, gate_up: Tensor, down: Tensor, k: int, d_expert: int,
                    act=ACT_SILU, norm_topk=False, bias=None, out_ids=None, out_w=None):
        T = X.shape[0]
        fl = self._io(out, X, bias, out_ids, out_w) | (LT_MOE_NORM_TOPK if norm_topk else 0)
        self._check(self.lib.lt_moe_prefill(self.ptr, _ptr(out)[0], _ptr(X)[0], T, router.handle, _ptr(bias)[0],
                                            gate_up.handle, down.handle, k, d_expert, act, fl, _ptr(out_ids)[0],
                                            _ptr(out_w)[0]))
        return out


def _norm_io(ctx, *arrays):
    return ctx._io(*arrays)


def _rows_n(x):
    shape = getattr(x, "shape", (len(x),))
    return (1, shape[0]) if len(shape) == 1 else (shape[0], shape[1])


def rmsnorm(ctx: Context, out, x, w=None, eps=1e-6, precise=False, one_plus_w=False):
    """math.rmsnorm (w given) / rmsnormRaw (w None) on each row of x ([n] or [rows, n])."""
    rows, n = _rows_n(x)
    fl = _norm_io(ctx, out, x, w) | (LT_NORM_PRECISE if precise else 0) | (LT_NORM_ONE_PLUS_W if one_plus_w else 0)
    ctx._check(ctx.lib.lt_rmsnorm(ctx.ptr, _ptr(out)[0], _ptr(x)[0], _ptr(w)[0], rows, n, eps, fl))
    return out


def add_rmsnorm(ctx: Context, out, a, b, w, eps=1e-6, precise=False, one_plus_w=False):
    rows, n = _rows_n(a)
    fl = _norm_io(ctx, out, a, b, w) | (LT_NORM_PRECISE if precise else 0) | (LT_NORM_ONE_PLUS_W if one_plus_w else 0)
    ctx._check(ctx.lib.lt_add_rmsnorm(ctx.ptr, _ptr(out)[0], _ptr(a)[0], _ptr(b)[0], _ptr(w)[0], rows, n, eps, fl))
    return out


def rmsnorm_weighted_raw_scaled(ctx: Context, weighted_out, raw_scaled_out, x, w, raw_scale, raw_global_scale,
                                eps=1e-6, precise=False):
    fl = _norm_io(ctx, weighted_out, raw_scaled_out, x, w, raw_scale) | (LT_NORM_PRECISE if precise else 0)
    ctx._check(ctx.lib.lt_rmsnorm_weighted_raw_scaled(ctx.ptr, _ptr(weighted_out)[0], _ptr(raw_scaled_out)[0],
                                                      _ptr(x)[0], _ptr(w)[0], _ptr(raw_scale)[0], raw_global_scale,
                                                      _rows_n(x)[1], eps, fl))


def moe_tail(ctx: Context, x, moe, dense_ffn, post_ffw_norm_2, post_ffw_norm, layer_output_scale=1.0, eps=1e-6,
             precise=False):
    """gemma4/forward.zig:482-497 in one launch; x is updated in place."""
    fl = _norm_io(ctx, x, moe, dense_ffn, post_ffw_norm_2, post_ffw_norm) | (LT_NORM_PRECISE if precise else 0)
    ctx._check(ctx.lib.lt_moe_tail(ctx.ptr, _ptr(x)[0], _ptr(moe)[0], _ptr(dense_ffn)[0], _ptr(post_ffw_norm_2)[0],
                                   _ptr(post_ffw_norm)[0], layer_output_scale, _rows_n(x)[1], eps, fl))
    return x


def gemma4_moe_block(ctx: Context, x, dense_ffn, router: Tensor, gate_up: Tensor, down: Tensor, k: int,
                     d_expert: int, norms: dict, layer_output_scale=1.0, eps=1e-6, act=ACT_GELU_TANH,
                     precise=False, norm_topk=False, out_ids=None, out_w=None, unfused=False, deterministic=False):
    """The Gemma4 MoE block of one token (gemma4/forward.zig:403-497); x is
    updated in place.  norms: pre_ffw_norm_2, router_scale, down_exps_scale
    (or None), post_ffw_norm_2, post_ffw_norm.  unfused: separate launches
    even where the single-launch kernel covers the block; deterministic: the
    separate launches' slot-order adds (bit-identical run to run)."""
    ds = norms.get("down_exps_scale")
    vecs = [norms["pre_ffw_norm_2"], norms["router_scale"], ds, norms["post_ffw_norm_2"], norms["post_ffw_norm"]]
    fl = _norm_io(ctx, x, dense_ffn, *vecs, out_ids, out_w)
    fl |= (LT_NORM_PRECISE if precise else 0) | (LT_MOE_NORM_TOPK if norm_topk else 0)
    fl |= (LT_MOE_UNFUSED if unfused else 0) | (LT_MOE_DETERMINISTIC if deterministic else 0)
    ctx._check(ctx.lib.lt_gemma4_moe_block(ctx.ptr, _ptr(x)[0], _ptr(dense_ffn)[0], router.handle, gate_up.handle,
                                           down.handle, *(_ptr(v)[0] for v in vecs), layer_output_scale, eps, k,
                                           d_expert, act, fl, _ptr(out_ids)[0], _ptr(out_w)[0]))
    return x


def upload_moe(ctx: Context, w) -> tuple:
    """Upload a synth.MoEWeights or gguf.MoELayer: returns (router, gate_up,
    down) tensors.  Expert types default to Q4_K (synth.MoEWeights)."""
    router = ctx.upload(w.router, w.router_type, w.n_experts, w.d_model)
    gate_up = ctx.upload(w.gate_up, getattr(w, "gate_up_type", ggml.Q4_K), 2 * w.d_expert, w.d_model, w.n_experts)
    down = ctx.upload(w.down, getattr(w, "down_type", ggml.Q4_K), w.d_model, w.down_cols, w.n_experts)
    return router, gate_up, down
