"""Host mirror of the reference device runtime (src/gpu/device.h:73-184):
Device, Queue, DeviceBuffer, HostBuffer (pinned staging), completion points.

Every method calls straight into libdlhip.so; numpy arrays are only host
staging for tests and the benchmark.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


class DeviceBuffer:
    """gpu::DeviceBuffer: device memory owned by one Device."""

    def __init__(self, device: "Device", nbytes: int, alignment: int = 256, staging: bool = False):
        handle = C.c_void_p()
        if staging:
            _lib.call("dl_staging_alloc", device.handle, nbytes, C.byref(handle))
        else:
            _lib.call("dl_buffer_alloc", device.handle, nbytes, alignment, C.byref(handle))
        self.device = device
        self.handle = handle
        self._native = _lib.Native("dl_buffer_free", handle, device._native)
        self.nbytes = nbytes
        self.staging = staging
        address = C.c_void_p()
        _lib.call("dl_buffer_address", handle, C.byref(address))
        self.address = address.value

    def ptr(self, offset: int = 0) -> C.c_void_p:
        """Address (device for device buffers) plus a byte offset."""
        return C.c_void_p(self.address + offset)

    def free(self) -> None:
        if self.handle:
            self.handle = None
            self._native.release()

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()


class HostBuffer(DeviceBuffer):
    """gpu::HostBuffer: pinned, host-mapped staging memory."""

    def __init__(self, device: "Device", nbytes: int):
        super().__init__(device, nbytes, staging=True)

    def view(self, dtype=np.uint8) -> np.ndarray:
        raw = (C.c_uint8 * self.nbytes).from_address(self.address)
        return np.frombuffer(raw, dtype=np.uint8).view(dtype)


class Event:
    def __init__(self, device: "Device"):
        handle = C.c_void_p()
        _lib.call("dl_event_create", device.handle, C.byref(handle))
        self.handle = handle
        self._native = _lib.Native("dl_event_destroy", handle, device._native)

    def record(self, queue: "Queue") -> None:
        _lib.call("dl_event_record", self.handle, queue.handle)

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        _lib.call("dl_event_elapsed_ms", self.handle, later.handle, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()


class Queue:
    """gpu::Queue: ordered submission with completion points."""

    def __init__(self, device: "Device"):
        handle = C.c_void_p()
        _lib.call("dl_queue_create", device.handle, C.byref(handle))
        self.device = device
        self.handle = handle
        self._native = _lib.Native("dl_queue_destroy", handle, device._native)

    def upload(self, dst: DeviceBuffer, src: HostBuffer, nbytes: int, dst_offset=0, src_offset=0):
        _lib.call("dl_queue_upload", self.handle, dst.handle, dst_offset, src.handle, src_offset, nbytes)

    def download(self, dst: HostBuffer, src: DeviceBuffer, nbytes: int, dst_offset=0, src_offset=0):
        _lib.call("dl_queue_download", self.handle, dst.handle, dst_offset, src.handle, src_offset, nbytes)

    def copy(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int, dst_offset=0, src_offset=0):
        _lib.call("dl_queue_copy", self.handle, dst.handle, dst_offset, src.handle, src_offset, nbytes)

    def write(self, dst: DeviceBuffer, array: np.ndarray, dst_offset: int = 0) -> None:
        a = np.ascontiguousarray(array)
        _lib.call("dl_queue_write", self.handle, dst.handle, dst_offset, a.ctypes.data_as(C.c_void_p), a.nbytes)

    def read(self, src: DeviceBuffer, dtype, count: int, src_offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _lib.call("dl_queue_read", self.handle, out.ctypes.data_as(C.c_void_p), src.handle, src_offset, out.nbytes)
        return out

    def mark(self) -> int:
        point = C.c_uint64()
        _lib.call("dl_queue_mark", self.handle, C.byref(point))
        return point.value

    def wait(self, point: int) -> None:
        _lib.call("dl_queue_wait", self.handle, point)

    def drain(self) -> None:
        _lib.call("dl_queue_drain", self.handle)

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()


class Device:
    """gpu::Device opened through gpu::cuda::open_device's replacement."""

    def __init__(self, ordinal: int = 0):
        handle = C.c_void_p()
        _lib.call("dl_device_open", ordinal, C.byref(handle))
        self.handle = handle
        self._native = _lib.Native("dl_device_close", handle)
        info = _lib.DeviceInfo()
        _lib.call("dl_device_info_get", handle, C.byref(info))
        self.name = info.name.decode()
        self.arch = info.arch.decode()
        self.compute_units = info.compute_units
        self.total_bytes = info.total_bytes

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()

    def allocate(self, nbytes: int, alignment: int = 256) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes, alignment)

    def allocate_staging(self, nbytes: int) -> HostBuffer:
        return HostBuffer(self, nbytes)

    def create_queue(self) -> Queue:
        return Queue(self)

    def query_memory(self) -> tuple[int, int]:
        free, total = C.c_uint64(), C.c_uint64()
        _lib.call("dl_memory_snapshot", self.handle, C.byref(free), C.byref(total))
        return free.value, total.value

    def upload_array(self, queue: Queue, array: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(array)
        buf = self.allocate(max(a.nbytes, 1))
        queue.write(buf, a)
        return buf
