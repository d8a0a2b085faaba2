"""Minimal ctypes access to the HIP runtime that libllmtoy_hip.so links
(/opt/rocm/lib/libamdhip64.so.7): device buffers, events, stream capture
into graphs.  Plumbing for callers of the C ABI that want device pointers
(tests, bench.py) without bringing in a second HIP runtime (torch bundles
its own)."""
from __future__ import annotations

import ctypes as C

import numpy as np

_hip = None

H2D, D2H, D2D = 1, 2, 3


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so.7", mode=C.RTLD_GLOBAL)
        vp, sz = C.c_void_p, C.c_size_t
        for name, res, args in [
            ("hipMalloc", C.c_int, [C.POINTER(vp), sz]),
            ("hipFree", C.c_int, [vp]),
            ("hipMemcpy", C.c_int, [vp, vp, sz, C.c_int]),
            ("hipMemcpyAsync", C.c_int, [vp, vp, sz, C.c_int, vp]),
            ("hipMemset", C.c_int, [vp, C.c_int, sz]),
            ("hipDeviceSynchronize", C.c_int, []),
            ("hipStreamSynchronize", C.c_int, [vp]),
            ("hipEventCreate", C.c_int, [C.POINTER(vp)]),
            ("hipEventDestroy", C.c_int, [vp]),
            ("hipEventRecord", C.c_int, [vp, vp]),
            ("hipEventSynchronize", C.c_int, [vp]),
            ("hipEventElapsedTime", C.c_int, [C.POINTER(C.c_float), vp, vp]),
            ("hipStreamBeginCapture", C.c_int, [vp, C.c_int]),
            ("hipStreamEndCapture", C.c_int, [vp, C.POINTER(vp)]),
            ("hipGraphInstantiate", C.c_int, [C.POINTER(vp), vp, vp, C.c_char_p, sz]),
            ("hipGraphLaunch", C.c_int, [vp, vp]),
            ("hipGraphExecDestroy", C.c_int, [vp]),
            ("hipGraphDestroy", C.c_int, [vp]),
            ("hipGetErrorString", C.c_char_p, [C.c_int]),
        ]:
            fn = getattr(_hip, name)
            fn.restype, fn.argtypes = res, args
    return _hip


def check(rc: int, what: str = "hip"):
    if rc != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(rc).decode()} ({rc})")


class DeviceArray:
    """A device allocation with a numpy shape/dtype (C-contiguous)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(np.atleast_1d(shape).tolist()) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(hip().hipMalloc(C.byref(p), max(self.nbytes, 256)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        check(hip().hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def row(self, i: int) -> "DeviceView":
        stride = self.nbytes // self.shape[0]
        return DeviceView(self.ptr + i * stride, self.shape[1:], self.dtype)

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None


class DeviceView:
    """A non-owning device pointer with a shape (e.g. one row of a DeviceArray)."""

    def __init__(self, ptr, shape, dtype):
        self.ptr, self.shape, self.dtype = ptr, tuple(shape), np.dtype(dtype)


class Event:
    def __init__(self):
        p = C.c_void_p()
        check(hip().hipEventCreate(C.byref(p)), "hipEventCreate")
        self.ptr = p.value

    def record(self, stream: int):
        check(hip().hipEventRecord(self.ptr, stream), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        check(hip().hipEventSynchronize(end.ptr), "hipEventSynchronize")
        ms = C.c_float()
        check(hip().hipEventElapsedTime(C.byref(ms), self.ptr, end.ptr), "hipEventElapsedTime")
        return float(ms.value)

    def destroy(self):
        if self.ptr:
            hip().hipEventDestroy(self.ptr)
            self.ptr = None


class Graph:
    """Capture the work a callable enqueues on `stream` into a hipGraph."""

    RELAXED = 2

    def __init__(self, stream: int, fn):
        self.stream = stream
        g = C.c_void_p()
        check(hip().hipStreamBeginCapture(stream, self.RELAXED), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            rc = hip().hipStreamEndCapture(stream, C.byref(g))
        check(rc, "hipStreamEndCapture")
        self.graph = g.value
        e = C.c_void_p()
        check(hip().hipGraphInstantiate(C.byref(e), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = e.value

    def launch(self):
        check(hip().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def destroy(self):
        if self.exec:
            hip().hipGraphExecDestroy(self.exec)
            hip().hipGraphDestroy(self.graph)
            self.exec = self.graph = None


def sync_stream(stream: int):
    check(hip().hipStreamSynchronize(stream), "hipStreamSynchronize")
