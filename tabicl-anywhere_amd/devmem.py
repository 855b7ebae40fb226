"""Device memory and event timing through the HIP runtime (libamdhip64), for callers that keep inputs resident in
HBM and time work on the library's own stream: `DeviceBuffer` (hipMalloc / hipMemcpy / hipFree) and `EventTimer`
(hipEventRecord on a given stream, hipEventElapsedTime)."""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np

_rt = None
H2D, D2H = 1, 2


def rt():
    global _rt
    if _rt is None:
        for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6", ctypes.util.find_library("amdhip64")):
            if not name:
                continue
            try:
                _rt = ctypes.CDLL(name)
                break
            except OSError:
                continue
        if _rt is None:
            raise OSError("the HIP runtime (libamdhip64) is not available")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        for fn, args in {
            "hipMalloc": [ctypes.POINTER(vp), sz], "hipFree": [vp], "hipMemcpy": [vp, vp, sz, ctypes.c_int],
            "hipMemset": [vp, ctypes.c_int, sz], "hipEventCreate": [ctypes.POINTER(vp)], "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp], "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp], "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [vp],
        }.items():
            f = getattr(_rt, fn)
            f.restype, f.argtypes = ctypes.c_int, args
    return _rt


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"graphics card: {what} failed with HIP status {rc}")


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _ok(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 256)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def of(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _ok(rt().hipMemcpy(ctypes.c_void_p(self.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, H2D), "hipMemcpy")

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        _ok(rt().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr), out.nbytes, D2H), "hipMemcpy")
        return out

    def free(self) -> None:
        if self.ptr:
            rt().hipFree(ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class EventTimer:
    """Milliseconds between two events recorded on `stream` (a hipStream_t as an int)."""

    def __init__(self, stream: int):
        self.stream = ctypes.c_void_p(stream)
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        _ok(rt().hipEventCreate(ctypes.byref(self.a)), "hipEventCreate")
        _ok(rt().hipEventCreate(ctypes.byref(self.b)), "hipEventCreate")

    def start(self) -> None:
        _ok(rt().hipEventRecord(self.a, self.stream), "hipEventRecord")

    def stop(self) -> float:
        _ok(rt().hipEventRecord(self.b, self.stream), "hipEventRecord")
        _ok(rt().hipEventSynchronize(self.b), "hipEventSynchronize")
        ms = ctypes.c_float()
        _ok(rt().hipEventElapsedTime(ctypes.byref(ms), self.a, self.b), "hipEventElapsedTime")
        return float(ms.value)


def copy(dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
    """Device-to-device copy of nbytes (hipMemcpy, kind device-to-device)."""
    assert nbytes <= dst.nbytes and nbytes <= src.nbytes
    _ok(rt().hipMemcpy(ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), nbytes, 3), "hipMemcpy")


def synchronize() -> None:
    _ok(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")
