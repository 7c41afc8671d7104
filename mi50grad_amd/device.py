"""Device memory, copies, streams and events through libkvattn.

``GPUDevice`` keeps the method names of the reference's ``GPUDevice``
(hip_dispatch.py:594-703: malloc, free, upload, download, memset,
memcpy_d2d, synchronize, cleanup) so engine-style callers work unchanged;
``DeviceArray`` adds a typed view for tests and the benchmark.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


class GPUDevice:
    """One GPU, addressed through integer device pointers."""

    def __init__(self, device_id: int = 0):
        self.device_id = device_id
        _lib.call("kva_dev_set", device_id)
        self._allocations: list[int] = []

    def _ensure_device(self):
        _lib.call("kva_dev_set", self.device_id)

    def malloc(self, size: int) -> int:
        p = ctypes.c_void_p()
        _lib.call("kva_dev_malloc", ctypes.byref(p), max(1, int(size)))
        self._allocations.append(p.value)
        return p.value

    def free(self, ptr: int) -> None:
        _lib.call("kva_dev_free", ptr)
        if ptr in self._allocations:
            self._allocations.remove(ptr)

    def upload(self, device_ptr: int, host_data) -> None:
        buf = bytes(host_data) if not isinstance(host_data, (bytes, bytearray)) else host_data
        _lib.call("kva_memcpy_h2d", device_ptr, buf, len(buf))

    def download(self, device_ptr: int, size: int) -> bytes:
        buf = ctypes.create_string_buffer(size)
        _lib.call("kva_memcpy_d2h", buf, device_ptr, size)
        return buf.raw

    def memset(self, ptr: int, value: int, size: int) -> None:
        _lib.call("kva_memset", ptr, value, size)

    def memcpy_d2d(self, dst: int, src: int, size: int) -> None:
        _lib.call("kva_memcpy_d2d", dst, src, size)

    def synchronize(self) -> None:
        _lib.call("kva_dev_synchronize")

    def launch_cached(self, spec, stream: int = 0) -> None:
        """Launch a pre-built spec of the decode launch cache with its
        current parameter values (hip_dispatch.py:681-689)."""
        self._ensure_device()
        spec.launch(stream or None)

    def cleanup(self) -> None:
        for p in list(self._allocations):
            self.free(p)

    def release(self) -> None:
        self.cleanup()

    # typed helpers -------------------------------------------------------
    def array(self, host: np.ndarray) -> "DeviceArray":
        return DeviceArray.from_host(self, host)

    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)


class DeviceArray:
    """A device buffer with a numpy shape and dtype (row-major)."""

    def __init__(self, dev: GPUDevice, shape, dtype, ptr: int | None = None):
        self.dev = dev
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = ptr if ptr is not None else dev.malloc(self.nbytes)
        self._owned = ptr is None

    @classmethod
    def from_host(cls, dev: GPUDevice, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host)
        arr = cls(dev, host.shape, host.dtype)
        arr.copy_from(host)
        return arr

    def copy_from(self, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host, dtype=self.dtype)
        assert host.nbytes == self.nbytes, (host.shape, self.shape)
        _lib.call("kva_memcpy_h2d", self.ptr, host.ctypes.data, self.nbytes)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _lib.call("kva_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def zero(self) -> None:
        _lib.call("kva_memset", self.ptr, 0, self.nbytes)

    def free(self) -> None:
        if self._owned and self.ptr:
            self.dev.free(self.ptr)
            self.ptr = 0


class Stream:
    def __init__(self):
        h = ctypes.c_void_p()
        _lib.call("kva_stream_create", ctypes.byref(h))
        self.handle = h.value

    def synchronize(self) -> None:
        _lib.call("kva_stream_synchronize", self.handle)

    def destroy(self) -> None:
        if self.handle:
            _lib.call("kva_stream_destroy", self.handle)
            self.handle = None


class Event:
    def __init__(self):
        h = ctypes.c_void_p()
        _lib.call("kva_event_create", ctypes.byref(h))
        self.handle = h.value

    def record(self, stream=None) -> None:
        _lib.call("kva_event_record", self.handle, stream)

    def synchronize(self) -> None:
        _lib.call("kva_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _lib.call("kva_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            _lib.call("kva_event_destroy", self.handle)
            self.handle = None


def device_count() -> int:
    n = ctypes.c_int32()
    _lib.call("kva_dev_count", ctypes.byref(n))
    return n.value


def device_props() -> dict:
    """Compute units, peak shader clock, memory clock (kHz) and memory bus
    width (bits) of the current device (kva_dev_props)."""
    v = [ctypes.c_int32() for _ in range(4)]
    _lib.call("kva_dev_props", *[ctypes.byref(x) for x in v])
    return {"n_cu": v[0].value, "clock_khz": v[1].value, "mem_clock_khz": v[2].value, "mem_bus_bits": v[3].value}
