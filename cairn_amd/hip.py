"""The HIP runtime as the Python toolchain uses it: device memory, copies, streams, events and the device's own
description, through ctypes on libamdhip64. Plumbing for tests and benchmarks only; the GEMM library itself is
C++/HIP and never calls into Python.

Every call is checked: a HIP error raises HipError with the runtime's message.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

_H2D, _D2H, _D2D = 1, 2, 3
_NOT_READY = 600  # hipErrorNotReady
_ATTR_CUS, _ATTR_CLOCK_KHZ, _ATTR_MEM_CLOCK_KHZ, _ATTR_L2 = 63, 5, 60, 19


class HipError(RuntimeError):
    pass


def _load() -> C.CDLL:
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    for name in (rocm / "lib/libamdhip64.so", "libamdhip64.so", "libamdhip64.so.7"):
        try:
            return C.CDLL(str(name))
        except OSError:
            continue
    raise HipError("libamdhip64.so not found: the HIP runtime is required")


_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
        _lib.hipGetErrorString.restype = C.c_char_p
        _lib.hipGetErrorString.argtypes = [C.c_int]
        for name, args in {
            "hipMalloc": [C.POINTER(C.c_void_p), C.c_size_t],
            "hipFree": [C.c_void_p],
            "hipMemcpy": [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int],
            "hipMemcpyAsync": [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p],
            "hipMemset": [C.c_void_p, C.c_int, C.c_size_t],
            "hipDeviceSynchronize": [],
            "hipGetDeviceCount": [C.POINTER(C.c_int)],
            "hipSetDevice": [C.c_int],
            "hipStreamCreate": [C.POINTER(C.c_void_p)],
            "hipStreamDestroy": [C.c_void_p],
            "hipStreamSynchronize": [C.c_void_p],
            "hipEventCreate": [C.POINTER(C.c_void_p)],
            "hipEventDestroy": [C.c_void_p],
            "hipEventRecord": [C.c_void_p, C.c_void_p],
            "hipEventSynchronize": [C.c_void_p],
            "hipEventElapsedTime": [C.POINTER(C.c_float), C.c_void_p, C.c_void_p],
            "hipDeviceGetAttribute": [C.POINTER(C.c_int), C.c_int, C.c_int],
            "hipDeviceGetName": [C.c_char_p, C.c_int, C.c_int],
            "hipGetLastError": [],
            "hipStreamQuery": [C.c_void_p],
            "hipStreamBeginCapture": [C.c_void_p, C.c_int],
            "hipStreamEndCapture": [C.c_void_p, C.POINTER(C.c_void_p)],
            "hipGraphInstantiate": [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t],
            "hipGraphLaunch": [C.c_void_p, C.c_void_p],
            "hipGraphExecDestroy": [C.c_void_p],
            "hipGraphDestroy": [C.c_void_p],
            "hipGraphGetNodes": [C.c_void_p, C.c_void_p, C.POINTER(C.c_size_t)],
        }.items():
            f = getattr(_lib, name)
            f.restype = C.c_int
            f.argtypes = args
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().hipGetErrorString(status).decode()
        raise HipError(f"{what}: {msg} ({status})" if what else f"{msg} ({status})")


def device_count() -> int:
    n = C.c_int(0)
    if lib().hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


def synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def attribute(attr: int, device: int = 0) -> int:
    v = C.c_int(0)
    check(lib().hipDeviceGetAttribute(C.byref(v), attr, device), "hipDeviceGetAttribute")
    return v.value


def describe(device: int = 0) -> dict:
    """What the runtime says of the device: name, CUs, peak engine clock, memory clock and L2."""
    name = C.create_string_buffer(256)
    check(lib().hipDeviceGetName(name, 256, device), "hipDeviceGetName")
    return {
        "name": name.value.decode(errors="replace"),
        "cus": attribute(_ATTR_CUS, device),
        "clock_mhz": attribute(_ATTR_CLOCK_KHZ, device) / 1000.0,
        "memory_clock_mhz": attribute(_ATTR_MEM_CLOCK_KHZ, device) / 1000.0,
        "l2_bytes": attribute(_ATTR_L2, device),
    }


class Buffer:
    """Device memory of `nbytes`, freed when closed or collected."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().hipMalloc(C.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def of(cls, array: np.ndarray) -> "Buffer":
        buf = cls(array.nbytes)
        buf.upload(array)
        return buf

    def upload(self, array: np.ndarray, offset: int = 0) -> None:
        array = np.ascontiguousarray(array)
        if offset + array.nbytes > self.nbytes:
            raise ValueError("upload past the buffer")
        check(lib().hipMemcpy(C.c_void_p(self.ptr + offset), array.ctypes.data_as(C.c_void_p), array.nbytes, _H2D),
              "hipMemcpy h2d")  # fmt: skip

    def download(self, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the buffer")
        check(lib().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset), out.nbytes, _D2H),
              "hipMemcpy d2h")  # fmt: skip
        return out

    def copy_from(self, other: "Buffer") -> None:
        if other.nbytes > self.nbytes:
            raise ValueError("copy past the buffer")
        check(lib().hipMemcpy(C.c_void_p(self.ptr), C.c_void_p(other.ptr), other.nbytes, _D2D), "hipMemcpy d2d")

    def zero(self) -> None:
        check(lib().hipMemset(C.c_void_p(self.ptr), 0, self.nbytes), "hipMemset")

    def close(self) -> None:
        if self.ptr:
            lib().hipFree(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    """A stream at the default priority."""

    def __init__(self):
        s = C.c_void_p()
        check(lib().hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(lib().hipStreamSynchronize(C.c_void_p(self.handle)), "hipStreamSynchronize")

    def idle(self) -> bool:
        """Whether everything queued on the stream has finished (hipStreamQuery), without waiting."""
        status = lib().hipStreamQuery(C.c_void_p(self.handle))
        if status == _NOT_READY:
            return False
        check(status, "hipStreamQuery")
        return True

    def close(self) -> None:
        if self.handle:
            lib().hipStreamDestroy(C.c_void_p(self.handle))
            self.handle = None


class Graph:
    """What `queue(stream)` queues on `stream`, captured (hipStreamBeginCapture, global mode) into an executable
    graph; launch() replays it on a stream."""

    def __init__(self, stream: Stream, queue):
        check(lib().hipStreamBeginCapture(C.c_void_p(stream.handle), 0), "hipStreamBeginCapture")
        try:
            queue(stream)
        finally:
            g = C.c_void_p()
            check(lib().hipStreamEndCapture(C.c_void_p(stream.handle), C.byref(g)), "hipStreamEndCapture")
        self.graph = g.value
        count = C.c_size_t(0)
        check(lib().hipGraphGetNodes(C.c_void_p(self.graph), None, C.byref(count)), "hipGraphGetNodes")
        self.nodes = count.value
        e = C.c_void_p()
        check(lib().hipGraphInstantiate(C.byref(e), C.c_void_p(self.graph), None, None, 0), "hipGraphInstantiate")
        self.exe = e.value

    def launch(self, stream: Stream) -> None:
        check(lib().hipGraphLaunch(C.c_void_p(self.exe), C.c_void_p(stream.handle)), "hipGraphLaunch")

    def close(self) -> None:
        if self.exe:
            lib().hipGraphExecDestroy(C.c_void_p(self.exe))
            lib().hipGraphDestroy(C.c_void_p(self.graph))
            self.exe = self.graph = None


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        check(lib().hipEventRecord(C.c_void_p(self.handle), C.c_void_p(stream.handle if stream else None)),
              "hipEventRecord")  # fmt: skip

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(C.c_void_p(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        check(lib().hipEventElapsedTime(C.byref(ms), C.c_void_p(self.handle), C.c_void_p(end.handle)),
              "hipEventElapsedTime")  # fmt: skip
        return ms.value

    def close(self) -> None:
        if self.handle:
            lib().hipEventDestroy(C.c_void_p(self.handle))
            self.handle = None
