"""Minimal ctypes access to the HIP runtime that libprism_hip.so links (libamdhip64.so.7).

Device buffers, copies, synchronisation and HIP events for the tests and the
benchmark, without a second HIP runtime in the process.
"""

from __future__ import annotations

import ctypes

import numpy as np

_hip = None

H2D, D2H, D2D = 1, 2, 3


def hip():
    global _hip
    if _hip is None:
        L = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        sig = {
            "hipMalloc": [ctypes.POINTER(P), S],
            "hipFree": [P],
            "hipMemcpy": [P, P, S, I],
            "hipMemset": [P, I, S],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [P],
            "hipEventCreate": [ctypes.POINTER(P)],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), P, P],
            "hipEventDestroy": [P],
            "hipGetDeviceCount": [ctypes.POINTER(I)],
            "hipDeviceGetAttribute": [ctypes.POINTER(I), I, I],
            "hipGetErrorString": [I],
            "hipStreamBeginCapture": [P, I],
            "hipStreamEndCapture": [P, ctypes.POINTER(P)],
            "hipGraphInstantiate": [ctypes.POINTER(P), P, P, P, S],
            "hipGraphLaunch": [P, P],
            "hipGraphExecDestroy": [P],
            "hipGraphDestroy": [P],
            "hipMemcpyAsync": [P, P, S, I, P],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hipGetErrorString" else I
        _hip = L
    return _hip


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {hip().hipGetErrorString(rc).decode()} ({rc})")


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def cu_count(device: int = 0) -> int:
    v = ctypes.c_int(0)
    # 63 = hipDeviceAttributeMultiprocessorCount (hip_runtime_api.h, ROCm 7)
    check(hip().hipDeviceGetAttribute(ctypes.byref(v), 63, device), "hipDeviceGetAttribute")
    return v.value


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """Owned device allocation with numpy copy helpers."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), f"hipMalloc({nbytes})")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(hip().hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(hip().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def to_numpy(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self) -> None:
        check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def data_ptr(self) -> int:
        return self.ptr

    def numel(self) -> int:
        return self.nbytes

    def element_size(self) -> int:
        return 1

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def copy_d2d(dst: int, src: int, nbytes: int) -> None:
    check(hip().hipMemcpy(dst, src, nbytes, D2D), "hipMemcpy D2D")


class Graph:
    """A HIP graph captured from the work a callable enqueues on `stream`."""

    def __init__(self, stream, enqueue):
        check(hip().hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")  # thread-local mode
        try:
            enqueue()
        finally:
            g = ctypes.c_void_p()
            rc = hip().hipStreamEndCapture(stream, ctypes.byref(g))
        check(rc, "hipStreamEndCapture")
        self.graph = g.value
        ex = ctypes.c_void_p()
        check(hip().hipGraphInstantiate(ctypes.byref(ex), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = ex.value
        self.stream = stream

    def launch(self) -> None:
        check(hip().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        # Replays may still be queued: drain the stream before freeing the executable.
        try:
            if getattr(self, "stream", None) is not None:
                hip().hipStreamSynchronize(self.stream)
            if getattr(self, "exec", None):
                hip().hipGraphExecDestroy(self.exec)
            if getattr(self, "graph", None):
                hip().hipGraphDestroy(self.graph)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(p)), "hipEventCreate")
        self.ev = p.value

    def record(self, stream=None) -> None:
        check(hip().hipEventRecord(self.ev, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(self.ev), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.ev:
                hip().hipEventDestroy(self.ev)
        except Exception:
            pass
