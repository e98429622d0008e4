"""Host mirror of the reference's NLA device objects: DeviceInjection
(src/inference/injection/device.h:29-47), DeviceDirection and
DeviceIntervention (src/inference/steering/device.h:30-68).

Construction validates what the reference validates on the host (shapes,
types, scale/strength, region bounds) and raises the same exception
classes; the numerical work and every value check run on the GPU through
libdlhip.so, and the status words stay in device memory (read back only
for provenance, as the reference's status()/norm()/count() regions).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from .runtime import Device, DeviceBuffer, Queue

BF16 = "bfloat16"
F32 = "float32"
_DTYPE = {BF16: 1, F32: 2}
_BYTES = {BF16: 2, F32: 4}


@dataclass(frozen=True)
class Region:
    """A borrowed byte range of a device buffer (gpu::ConstDeviceRegion)."""

    owner: DeviceBuffer
    offset: int
    bytes: int

    def ptr(self) -> C.c_void_p:
        return self.owner.ptr(self.offset)


def _check_region(region: Region, nbytes: int, alignment: int) -> None:
    if (region.owner is None or region.bytes != nbytes or region.offset % alignment
            or region.offset > region.owner.nbytes or region.bytes > region.owner.nbytes - region.offset):
        raise ValueError("region bounds/alignment")


class DeviceInjection:
    """Normalizes a BF16/FP32 source row to `scale` * h / ||h|| on the GPU
    (injection.cu:49-98); output(), norm() and status() are device regions."""

    def __init__(self, device: Device, queue: Queue, source: Region, source_type: str, output_type: str,
                 width: int, scale: float):
        if source_type not in _DTYPE or output_type not in _DTYPE:
            raise ValueError("unsupported injection type")
        if (source.owner is None or source.offset % _BYTES[source_type] or source.bytes != width * _BYTES[source_type]
                or source.offset > source.owner.nbytes or source.bytes > source.owner.nbytes - source.offset
                or not math.isfinite(scale) or scale <= 0):
            raise ValueError("invalid injection source")
        self.device, self.queue, self.source = device, queue, source
        self.source_type, self.output_type, self.width, self.scale = source_type, output_type, width, scale
        self.storage = device.allocate(self.required_bytes(width, output_type), 4)

    @staticmethod
    def required_bytes(width: int, output_type: str) -> int:
        out = C.c_uint64()
        _lib.call("dl_injection_bytes", width, _DTYPE.get(output_type, 0), C.byref(out))
        return out.value

    def submit(self) -> None:
        _lib.call("dl_injection_submit", self.queue.handle, self.source.ptr(), _DTYPE[self.source_type],
                  _DTYPE[self.output_type], self.width, self.scale, self.storage.ptr())

    def output(self) -> Region:
        return Region(self.storage, 8, self.width * _BYTES[self.output_type])

    def norm(self) -> Region:
        return Region(self.storage, 0, 4)

    def status(self) -> Region:
        return Region(self.storage, 4, 4)


class DeviceDirection:
    """(edited - original) / ||edited - original|| into FP32 device storage
    (steering.cu:69-100); finish() drains, checks the status word and
    returns the direction region."""

    def __init__(self, device: Device, queue: Queue, original: Region, edited: Region, dtype: str, width: int):
        if dtype not in _DTYPE:
            raise ValueError("steering storage type")
        self.required_bytes(width)
        _check_region(original, width * _BYTES[dtype], _BYTES[dtype])
        _check_region(edited, width * _BYTES[dtype], _BYTES[dtype])
        self.device, self.queue, self.original, self.edited = device, queue, original, edited
        self.dtype, self.width = dtype, width
        self.storage = device.allocate(self.required_bytes(width), 4)
        self.submitted = self.completed = False

    @staticmethod
    def required_bytes(width: int) -> int:
        out = C.c_uint64()
        _lib.call("dl_direction_bytes", width, C.byref(out))
        return out.value

    def submit(self) -> None:
        if self.submitted:
            raise RuntimeError("direction already submitted")
        _lib.call("dl_direction_submit", self.queue.handle, self.original.ptr(), self.edited.ptr(),
                  _DTYPE[self.dtype], self.width, self.storage.ptr())
        self.submitted = True

    def finish(self) -> Region:
        if not self.submitted or self.completed:
            raise RuntimeError("direction completion state")
        status = int(self.queue.read(self.storage, np.uint32, 1)[0])
        if status:
            raise ValueError("reconstructions have zero or nonfinite difference")
        self.completed = True
        return Region(self.storage, 8, self.width * 4)


class DeviceIntervention:
    """One-row residual steering h += (strength * ||h||) * u on the GPU
    (steering.cu:100-159); status() and count() are device regions."""

    required_bytes = 8

    def __init__(self, device: Device, queue: Queue, direction: Region, width: int, position: int,
                 strength: float, dtype: str):
        DeviceDirection.required_bytes(width)
        _check_region(direction, width * 4, 4)
        if not math.isfinite(strength) or strength < 0 or dtype not in _DTYPE:
            raise ValueError("invalid residual intervention")
        self.device, self.queue, self.direction = device, queue, direction
        self.width, self.position, self.strength, self.dtype = width, position, strength, dtype
        self.state = device.allocate(self.required_bytes, 4)

    def initialize(self) -> None:
        _lib.call("dl_intervention_initialize", self.queue.handle, self.state.ptr())

    def submit(self, residual: Region, position: Region, rows: int) -> None:
        if rows <= 0:
            raise OverflowError("intervention extent")
        _check_region(residual, rows * self.width * _BYTES[self.dtype], _BYTES[self.dtype])
        _check_region(position, 8, 8)
        _lib.call("dl_intervention_submit", self.queue.handle, residual.ptr(), _DTYPE[self.dtype], rows,
                  self.width, self.direction.ptr(), position.ptr(), self.position, self.strength,
                  self.state.ptr())

    def status(self) -> Region:
        return Region(self.state, 0, 4)

    def count(self) -> Region:
        return Region(self.state, 4, 4)
