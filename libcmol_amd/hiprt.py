"""Minimal HIP runtime access for timing: events recorded on a given stream."""
from __future__ import annotations

import ctypes as C
import os

_rt = None


def rt():
    global _rt
    if _rt is None:
        for name in ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _rt = C.CDLL(name)
                break
            except OSError:
                continue
        if _rt is None:
            raise RuntimeError("libamdhip64.so not found")
        _rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        _rt.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        _rt.hipEventSynchronize.argtypes = [C.c_void_p]
        _rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        _rt.hipEventDestroy.argtypes = [C.c_void_p]
        _rt.hipDeviceSynchronize.argtypes = []
        _rt.hipStreamSynchronize.argtypes = [C.c_void_p]
    return _rt


class EventTimer:
    """Pair of HIP events on one stream; elapsed() in milliseconds."""

    def __init__(self, stream):
        self.stream = C.c_void_p(stream if isinstance(stream, int) else getattr(stream, "value", stream))
        self.a, self.b = C.c_void_p(), C.c_void_p()
        _ck(rt().hipEventCreate(C.byref(self.a)))
        _ck(rt().hipEventCreate(C.byref(self.b)))

    def start(self):
        _ck(rt().hipEventRecord(self.a, self.stream))

    def stop(self):
        _ck(rt().hipEventRecord(self.b, self.stream))

    def elapsed(self) -> float:
        _ck(rt().hipEventSynchronize(self.b))
        ms = C.c_float()
        _ck(rt().hipEventElapsedTime(C.byref(ms), self.a, self.b))
        return ms.value

    def close(self):
        rt().hipEventDestroy(self.a)
        rt().hipEventDestroy(self.b)


def device_synchronize():
    _ck(rt().hipDeviceSynchronize())


def _ck(rc):
    if rc != 0:
        raise RuntimeError(f"HIP runtime call failed: {rc}")
