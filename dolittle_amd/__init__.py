"""dolittle_amd: MI355X (gfx950) backend for Dolittle's Qwen3-8B token loop.

The compute path is libdlhip.so (hand-written HIP kernels behind the C ABI
of include/dolittle_hip.h).  This package is the host-side mirror of the
reference interface for Python callers, tests and the benchmark.
"""
from ._lib import (DeviceError, DolittleError, InvalidArgument, LengthError, Poisoned,  # noqa: F401
                   header_functions, load)
from .runtime import Device, DeviceBuffer, Event, HostBuffer, Queue  # noqa: F401

__all__ = ["Device", "DeviceBuffer", "HostBuffer", "Queue", "Event", "load", "header_functions",
           "DolittleError", "InvalidArgument", "LengthError", "DeviceError", "Poisoned"]
