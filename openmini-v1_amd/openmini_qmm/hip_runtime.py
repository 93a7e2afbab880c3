"""Minimal ctypes access to the HIP runtime that libopenmini_qmm.so itself loaded:
events (for timing on the stream a kernel runs on) and graphs.

Only libamdhip64.so.7 already mapped into the process is used, so the library and
the timing calls share one runtime.
"""
from __future__ import annotations

import ctypes

from . import _native

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _native.lib()  # maps libamdhip64.so.7 as a dependency of the library
        H = ctypes.CDLL("libamdhip64.so.7")
        p, i = ctypes.c_void_p, ctypes.c_int
        for name, res, args in [
            ("hipEventCreate", i, [ctypes.POINTER(p)]),
            ("hipEventDestroy", i, [p]),
            ("hipEventRecord", i, [p, p]),
            ("hipEventSynchronize", i, [p]),
            ("hipEventElapsedTime", i, [ctypes.POINTER(ctypes.c_float), p, p]),
            ("hipDeviceSynchronize", i, []),
            ("hipStreamBeginCapture", i, [p, i]),
            ("hipStreamEndCapture", i, [p, ctypes.POINTER(p)]),
            ("hipGraphInstantiate", i, [ctypes.POINTER(p), p, p, p, ctypes.c_size_t]),
            ("hipGraphLaunch", i, [p, p]),
            ("hipGraphExecDestroy", i, [p]),
            ("hipGraphDestroy", i, [p]),
            ("hipGetErrorString", ctypes.c_char_p, [i]),
        ]:
            fn = getattr(H, name)
            fn.restype = res
            fn.argtypes = args
        _hip = H
    return _hip


def _ck(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {hip().hipGetErrorString(rc).decode()} ({rc})")


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        _ck(hip().hipEventCreate(ctypes.byref(self.h)), "hipEventCreate")

    def record(self, stream=None):
        _ck(hip().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self):
        _ck(hip().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _ck(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        if getattr(self, "h", None) and _hip is not None:
            hip().hipEventDestroy(self.h)


class Graph:
    """Captures the launches made by `fn(stream)` on `stream` into a HIP graph."""

    CAPTURE_MODE_THREAD_LOCAL = 1

    def __init__(self, stream, fn):
        H = hip()
        self.graph = ctypes.c_void_p()
        self.exec = ctypes.c_void_p()
        _ck(H.hipStreamBeginCapture(stream, self.CAPTURE_MODE_THREAD_LOCAL), "hipStreamBeginCapture")
        try:
            fn(stream)
        finally:
            _ck(H.hipStreamEndCapture(stream, ctypes.byref(self.graph)), "hipStreamEndCapture")
        _ck(H.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0),
            "hipGraphInstantiate")

    def launch(self, stream):
        _ck(hip().hipGraphLaunch(self.exec, stream), "hipGraphLaunch")

    def __del__(self):
        if _hip is None:
            return
        if getattr(self, "exec", None):
            hip().hipGraphExecDestroy(self.exec)
        if getattr(self, "graph", None):
            hip().hipGraphDestroy(self.graph)
