"""Minimal ctypes binding of the HIP runtime: device memory, copies, streams
and events.  Used by the Python host layer, the tests and the benchmark to
hand device-resident buffers to the sampler's C ABI."""
from __future__ import annotations

import ctypes
import os

import numpy as np

_rt = None


class HipError(RuntimeError):
    pass


def runtime() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        names = ["libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"]
        last = None
        for n in names:
            try:
                _rt = ctypes.CDLL(n)
                break
            except OSError as e:  # pragma: no cover - depends on the image
                last = e
        if _rt is None:
            raise HipError(f"cannot load the HIP runtime: {last}")
        R = _rt
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        R.hipGetErrorString.restype = ctypes.c_char_p
        R.hipGetErrorString.argtypes = [ctypes.c_int]
        R.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        R.hipSetDevice.argtypes = [ctypes.c_int]
        R.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        R.hipFree.argtypes = [vp]
        R.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        R.hipMemcpyAsync.argtypes = [vp, vp, sz, ctypes.c_int, vp]
        R.hipMemset.argtypes = [vp, ctypes.c_int, sz]
        R.hipDeviceSynchronize.argtypes = []
        R.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        R.hipStreamDestroy.argtypes = [vp]
        R.hipStreamSynchronize.argtypes = [vp]
        R.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        R.hipEventDestroy.argtypes = [vp]
        R.hipEventRecord.argtypes = [vp, vp]
        R.hipEventSynchronize.argtypes = [vp]
        R.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
    return _rt


def check(code: int, what: str = "") -> None:
    if code != 0:
        msg = runtime().hipGetErrorString(code).decode()
        raise HipError(f"{what}: {msg} ({code})")


def device_count() -> int:
    try:
        n = ctypes.c_int(0)
        if runtime().hipGetDeviceCount(ctypes.byref(n)) != 0:
            return 0
        return n.value
    except HipError:
        return 0


H2D, D2H, D2D = 1, 2, 3


class DeviceArray:
    """A device allocation that remembers its numpy dtype and shape."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = ctypes.c_void_p()
        check(runtime().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1)), "hipMalloc")

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    @property
    def addr(self) -> int:
        return int(self.ptr.value or 0)

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(runtime().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(runtime().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, other: "DeviceArray") -> None:
        assert other.nbytes == self.nbytes
        check(runtime().hipMemcpy(self.ptr, other.ptr, self.nbytes, D2D), "hipMemcpy D2D")

    def free(self) -> None:
        if self.ptr.value:
            runtime().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(runtime().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    def synchronize(self) -> None:
        check(runtime().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle.value:
            runtime().hipStreamDestroy(self.handle)
            self.handle = ctypes.c_void_p()


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(runtime().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream: Stream | None = None) -> None:
        check(runtime().hipEventRecord(self.handle, stream.handle if stream else None),
              "hipEventRecord")

    def synchronize(self) -> None:
        check(runtime().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(runtime().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle),
              "hipEventElapsedTime")
        return float(ms.value)


def synchronize() -> None:
    check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


def gpu_available() -> bool:
    return os.environ.get("HIP_VISIBLE_DEVICES", "x") != "" and device_count() > 0
