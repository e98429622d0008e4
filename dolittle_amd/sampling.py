"""DeviceCategorical mirror (src/inference/sampling/device.h:58-85) over the
C ABI of include/dolittle_hip.h.

Selection follows the host law of src/inference/sampling/categorical.cpp:
146-201 bit for bit; results are (token, status) with status 0 ok, 1 for a
NaN/+inf logit and 2 when no logit is finite.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _lib
from .runtime import Device, DeviceBuffer, Queue


@dataclass(frozen=True)
class Settings:
    """src/inference/sampling/sampler.h:45-55 (mode "greedy"/"categorical")."""
    mode: str = "greedy"
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0

    def ctype(self) -> _lib.Sampling:
        if self.mode not in ("greedy", "categorical"):
            raise _lib.InvalidArgument("invalid sampling settings")
        return _lib.Sampling(0 if self.mode == "greedy" else 1, self.top_k, self.temperature, self.top_p)


class DeviceCategorical:
    """Prepared device selector over one BF16 logits row of `vocabulary`."""

    def __init__(self, device: Device, queue: Queue, vocabulary: int, dtype: str = "bf16",
                 budget: int | None = None):
        self.device, self.queue, self.vocabulary = device, queue, vocabulary
        if budget is None:
            budget = self.required_bytes(vocabulary)
        code = {"bf16": 1, "f32": 2}.get(dtype)
        if code is None:
            raise _lib.InvalidArgument("unsupported sampling storage")
        handle = C.c_void_p()
        _lib.call("dl_sampler_create", device.handle, queue.handle, vocabulary, code, budget,
                  C.byref(handle))
        self.handle = handle
        self._native = _lib.Native("dl_sampler_destroy", handle, device._native, queue._native)

    @staticmethod
    def required_bytes(vocabulary: int) -> int:
        out = C.c_uint64(0)
        _lib.call("dl_sampler_required_bytes", vocabulary, C.byref(out))
        return out.value

    def _row(self, row, offset: int) -> C.c_void_p:
        if isinstance(row, DeviceBuffer):
            return row.ptr(offset)
        return C.c_void_p(int(row) + offset)

    def submit(self, row, settings: Settings, draw_bits: int, offset: int = 0) -> None:
        """Diagnostic selection with explicit draw bits (device.h:70-71)."""
        s = settings.ctype()
        _lib.call("dl_sampler_submit", self.handle, self._row(row, offset), self.vocabulary * 2,
                  C.byref(s), draw_bits)

    def start(self, settings: Settings, seed: int, stop_ids=()) -> None:
        s = settings.ctype()
        ids = (C.c_uint32 * max(1, len(stop_ids)))(*stop_ids)
        _lib.call("dl_sampler_start", self.handle, C.byref(s), seed, ids, len(stop_ids))

    def submit_next(self, row, offset: int = 0) -> None:
        _lib.call("dl_sampler_submit_next", self.handle, self._row(row, offset), self.vocabulary * 2)

    def result(self) -> tuple[int, int]:
        token, status = C.c_uint32(0), C.c_uint32(0)
        _lib.call("dl_sampler_result", self.handle, C.byref(token), C.byref(status))
        return token.value, status.value

    def result_address(self) -> int:
        out = C.c_void_p()
        _lib.call("dl_sampler_result_address", self.handle, C.byref(out))
        return out.value

    def terminal_address(self) -> int:
        out = C.c_void_p()
        _lib.call("dl_sampler_terminal_address", self.handle, C.byref(out))
        return out.value

    def current_token_address(self) -> int:
        out = C.c_void_p()
        _lib.call("dl_sampler_current_token_address", self.handle, C.byref(out))
        return out.value

    def set_exact(self, exact: bool) -> None:
        """Diagnostic: decide every selection by the exact serial replay."""
        _lib.call("dl_sampler_set_exact", self.handle, int(exact))

    def exact_replays(self) -> int:
        out = C.c_uint64(0)
        _lib.call("dl_sampler_exact_replays", self.handle, C.byref(out))
        return out.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.handle = None
            self._native.release()

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()
