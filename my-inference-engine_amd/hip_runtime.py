"""Minimal ctypes access to the HIP runtime that libqmv_hip.so itself links
(device memory, copies, streams, events, stream capture into graphs).

The benchmark and the tests use this instead of torch: torch ships its own
libamdhip64.so.7 with the same soname, and two runtimes in one process do
not mix. Loading libqmv_hip.so first and then asking for libamdhip64.so.7
returns the runtime it already loaded.
"""
from __future__ import annotations

import ctypes

import numpy as np

_rt = None

H2D, D2H, D2D = 1, 2, 3
CAPTURE_MODE_GLOBAL = 0


def rt():
    global _rt
    if _rt is None:
        import importlib

        importlib.import_module("my-inference-engine_amd").hip_lib()  # load the runtime it links
        lib = ctypes.CDLL("libamdhip64.so.7")
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        sigs = {
            "hipMalloc": [ctypes.POINTER(vp), sz], "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, i], "hipMemcpyAsync": [vp, vp, sz, i, vp],
            "hipMemset": [vp, i, sz], "hipDeviceSynchronize": [], "hipSetDevice": [i],
            "hipStreamCreate": [ctypes.POINTER(vp)], "hipStreamDestroy": [vp], "hipStreamSynchronize": [vp],
            "hipEventCreate": [ctypes.POINTER(vp)], "hipEventDestroy": [vp], "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp], "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipStreamBeginCapture": [vp, i], "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, sz], "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp], "hipGraphDestroy": [vp], "hipGetErrorString": [i],
        }
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hipGetErrorString" else ctypes.c_int
        _rt = lib
    return _rt


def check(err, what=""):
    if err != 0:
        raise RuntimeError(f"{what}: HIP error {err}: {rt().hipGetErrorString(err).decode()}")


class DeviceBuffer:
    """Owned device allocation."""

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        check(rt().hipMalloc(ctypes.byref(p), max(1, nbytes)), "hipMalloc")
        self.ptr = p.value
        self.nbytes = nbytes

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(rt().hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        check(rt().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill(self, byte: int = 0) -> None:
        check(rt().hipMemset(self.ptr, byte, self.nbytes), "hipMemset")

    def free(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A HIP stream (default priority), destroyed by destroy() or on leaving a
    ``with`` block after its work has finished."""

    def __init__(self):
        s = ctypes.c_void_p()
        check(rt().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(rt().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            rt().hipStreamSynchronize(self.handle)
            rt().hipStreamDestroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream) -> None:
        check(rt().hipEventRecord(self.handle, stream.handle), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(rt().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            rt().hipEventDestroy(self.handle)
            self.handle = None


class Graph:
    """Captures everything enqueued on `stream` between begin() and end();
    destroy() (or leaving a ``with`` block) frees the executable graph and the
    graph after the stream's work has finished."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.graph = None
        self.exec = None

    def begin(self) -> None:
        check(rt().hipStreamBeginCapture(self.stream.handle, CAPTURE_MODE_GLOBAL), "hipStreamBeginCapture")

    def end(self) -> None:
        g = ctypes.c_void_p()
        check(rt().hipStreamEndCapture(self.stream.handle, ctypes.byref(g)), "hipStreamEndCapture")
        self.graph = g.value
        e = ctypes.c_void_p()
        check(rt().hipGraphInstantiate(ctypes.byref(e), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = e.value

    def replay(self) -> None:
        check(rt().hipGraphLaunch(self.exec, self.stream.handle), "hipGraphLaunch")

    def destroy(self) -> None:
        if self.stream.handle:
            rt().hipStreamSynchronize(self.stream.handle)
        if self.exec:
            rt().hipGraphExecDestroy(self.exec)
            self.exec = None
        if self.graph:
            rt().hipGraphDestroy(self.graph)
            self.graph = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


def synchronize() -> None:
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")
