"""Minimal ctypes binding of the HIP runtime: device buffers, copies, streams
and events for the tests, the benchmark and the smoke check.

The runtime is the ``libamdhip64.so.7`` that ``libq3k.so`` itself links
(loaded first, RTLD_GLOBAL), so the kernels and these calls share one HIP
runtime instance.  Nothing here imports torch.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import load as _load_q3k

HIP_MEMCPY_H2D = 1
HIP_MEMCPY_D2H = 2
HIP_MEMCPY_D2D = 3
HIP_STREAM_CAPTURE_MODE_THREAD_LOCAL = 1

_hip = None


class HipRuntimeError(RuntimeError):
    pass


def runtime() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _load_q3k()
        lib = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        p, sz = ctypes.c_void_p, ctypes.c_size_t
        sig = {
            "hipGetDeviceCount": [ctypes.POINTER(ctypes.c_int)],
            "hipSetDevice": [ctypes.c_int],
            "hipGetDevice": [ctypes.POINTER(ctypes.c_int)],
            "hipMalloc": [ctypes.POINTER(p), sz],
            "hipFree": [p],
            "hipMemcpy": [p, p, sz, ctypes.c_int],
            "hipMemcpyAsync": [p, p, sz, ctypes.c_int, p],
            "hipMemset": [p, ctypes.c_int, sz],
            "hipMemsetAsync": [p, ctypes.c_int, sz, p],
            "hipDeviceSynchronize": [],
            "hipStreamCreate": [ctypes.POINTER(p)],
            "hipStreamDestroy": [p],
            "hipStreamSynchronize": [p],
            "hipEventCreate": [ctypes.POINTER(p)],
            "hipEventDestroy": [p],
            "hipEventRecord": [p, p],
            "hipEventSynchronize": [p],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), p, p],
            "hipGetLastError": [],
            "hipDeviceGetAttribute": [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int],
            "hipMemGetInfo": [ctypes.POINTER(sz), ctypes.POINTER(sz)],
            "hipStreamBeginCapture": [p, ctypes.c_int],
            "hipStreamEndCapture": [p, ctypes.POINTER(p)],
            "hipGraphInstantiate": [ctypes.POINTER(p), p, p, p, sz],
            "hipGraphLaunch": [p, p],
            "hipGraphExecDestroy": [p],
            "hipGraphDestroy": [p],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        lib.hipGetErrorString.argtypes = [ctypes.c_int]
        lib.hipGetErrorString.restype = ctypes.c_char_p
        _hip = lib
    return _hip


def check(status: int, what: str = "HIP call") -> None:
    if status != 0:
        msg = runtime().hipGetErrorString(status).decode()
        raise HipRuntimeError(f"{what} failed: {status} {msg}")


def device_count() -> int:
    n = ctypes.c_int(0)
    st = runtime().hipGetDeviceCount(ctypes.byref(n))
    return n.value if st == 0 else 0


def available() -> bool:
    try:
        return device_count() > 0
    except OSError:
        return False


def synchronize() -> None:
    check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


def get_device() -> int:
    d = ctypes.c_int(-1)
    check(runtime().hipGetDevice(ctypes.byref(d)), "hipGetDevice")
    return d.value


def set_device(i: int) -> None:
    check(runtime().hipSetDevice(i), "hipSetDevice")


def mem_info() -> tuple[int, int]:
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    check(runtime().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceBuffer:
    """An owning device allocation of ``nbytes`` bytes (hipMalloc, 256-byte aligned)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = None
        if self.nbytes > 0:
            p = ctypes.c_void_p()
            check(runtime().hipMalloc(ctypes.byref(p), self.nbytes), f"hipMalloc({self.nbytes})")
            self.ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds buffer")
        if arr.nbytes:
            check(runtime().hipMemcpy(self.ptr + offset, arr.ctypes.data, arr.nbytes, HIP_MEMCPY_H2D), "hipMemcpy H2D")

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download exceeds buffer")
        if out.nbytes:
            check(runtime().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, HIP_MEMCPY_D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, other: "DeviceBuffer", nbytes: int | None = None, offset: int = 0) -> None:
        """self[offset : offset + n] = other[0 : n] (n = nbytes, or all of self)."""
        n = self.nbytes if nbytes is None else nbytes
        if offset < 0 or offset + n > self.nbytes or n > other.nbytes:
            raise ValueError("device copy exceeds a buffer")
        if n:
            check(runtime().hipMemcpy(self.ptr + offset, other.ptr, n, HIP_MEMCPY_D2D), "hipMemcpy D2D")

    def tile_from(self, block: "DeviceBuffer") -> None:
        """Fills the whole buffer with repeats of ``block`` (device-to-device copies)."""
        off = 0
        while off < self.nbytes:
            n = min(block.nbytes, self.nbytes - off)
            self.copy_from(block, n, off)
            off += n

    def fill_bytes(self, value: int) -> None:
        if self.nbytes:
            check(runtime().hipMemset(self.ptr, value, self.nbytes), "hipMemset")

    def free(self) -> None:
        if self.ptr is not None:
            runtime().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        check(runtime().hipStreamCreate(ctypes.byref(p)), "hipStreamCreate")
        self.ptr = p.value

    def synchronize(self) -> None:
        check(runtime().hipStreamSynchronize(self.ptr), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.ptr is not None:
            runtime().hipStreamDestroy(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(runtime().hipEventCreate(ctypes.byref(p)), "hipEventCreate")
        self.ptr = p.value

    def record(self, stream=None) -> None:
        check(runtime().hipEventRecord(self.ptr, getattr(stream, "ptr", stream)), "hipEventRecord")

    def synchronize(self) -> None:
        check(runtime().hipEventSynchronize(self.ptr), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        check(runtime().hipEventElapsedTime(ctypes.byref(ms), self.ptr, end.ptr), "hipEventElapsedTime")
        return ms.value

    def destroy(self) -> None:
        if self.ptr is not None:
            runtime().hipEventDestroy(self.ptr)
            self.ptr = None


class Graph:
    """The launches `record()` makes on `stream`, captured into a HIP graph
    and instantiated for replay (hipStreamBeginCapture ... hipGraphInstantiate).
    Nothing runs during capture; every replay runs the captured kernels with
    the arguments they were launched with, so in-place ops act on whatever the
    buffers hold at replay time."""

    def __init__(self, stream: Stream, record):
        rt = runtime()
        check(rt.hipStreamBeginCapture(stream.ptr, HIP_STREAM_CAPTURE_MODE_THREAD_LOCAL), "hipStreamBeginCapture")
        graph = ctypes.c_void_p()
        try:
            record()
        except BaseException:
            rt.hipStreamEndCapture(stream.ptr, ctypes.byref(graph))
            if graph.value:
                rt.hipGraphDestroy(graph.value)
            raise
        check(rt.hipStreamEndCapture(stream.ptr, ctypes.byref(graph)), "hipStreamEndCapture")
        self.graph = graph.value
        self.exec = None
        exe = ctypes.c_void_p()
        try:
            check(rt.hipGraphInstantiate(ctypes.byref(exe), self.graph, None, None, 0), "hipGraphInstantiate")
        except BaseException:
            self.destroy()
            raise
        self.exec = exe.value

    def launch(self, stream: Stream) -> None:
        check(runtime().hipGraphLaunch(self.exec, stream.ptr), "hipGraphLaunch")

    def destroy(self) -> None:
        rt = runtime()
        if self.exec is not None:
            rt.hipGraphExecDestroy(self.exec)
            self.exec = None
        if self.graph is not None:
            rt.hipGraphDestroy(self.graph)
            self.graph = None
