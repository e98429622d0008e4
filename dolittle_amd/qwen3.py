"""Qwen3 resident model and cached forward plan over libdlhip.so.

Mirrors the reference's load_resident_model / prepare_cached_forward /
generate flow (src/inference/executor.h:242-342,
src/inference/generation.h:129-138) for the Qwen3-8B recipe
(src/models/qwen3/model.cpp:343-409).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib
from .runtime import Device, Queue

ROLE = {
    "embedding": 0, "lm_head": 1, "final_norm": 2, "input_norm": 3, "q": 4, "k": 5, "v": 6,
    "q_norm": 7, "k_norm": 8, "o": 9, "post_norm": 10, "gate": 11, "up": 12, "down": 13,
}
REASON = {0: "limit", 1: "eos", 2: "cancelled", 3: "failure"}
EVENT_KIND = {0: "consumed", 1: "selected", 2: "terminal", 3: "injection"}


@dataclass
class Qwen3Config:
    """src/models/qwen3/model.h:125-137; defaults are Qwen3-8B."""
    layers: int = 36
    hidden: int = 4096
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 12288
    vocab: int = 151936
    tied_embeddings: bool = True
    rms_eps: float = 1e-6
    rope_theta: float = 1e6

    def ctype(self) -> _lib.Qwen3Config:
        return _lib.Qwen3Config(self.layers, self.hidden, self.q_heads, self.kv_heads, self.head_dim, self.ffn,
                                self.vocab, 1 if self.tied_embeddings else 0, self.rms_eps, 0, self.rope_theta)

    def shape(self, role: str) -> tuple:
        D, QW, KW = self.hidden, self.q_heads * self.head_dim, self.kv_heads * self.head_dim
        return {
            "embedding": (self.vocab, D), "lm_head": (self.vocab, D), "final_norm": (D,),
            "input_norm": (D,), "post_norm": (D,), "q_norm": (self.head_dim,), "k_norm": (self.head_dim,),
            "q": (QW, D), "k": (KW, D), "v": (KW, D), "o": (D, QW), "gate": (self.ffn, D),
            "up": (self.ffn, D), "down": (D, self.ffn),
        }[role]

    def projection_bytes_per_token(self) -> int:
        """BF16 projection weight bytes read per decoded token (incl. LM head)."""
        D, QW, KW, F = self.hidden, self.q_heads * self.head_dim, self.kv_heads * self.head_dim, self.ffn
        per_block = (QW * D + 2 * KW * D + D * QW + 2 * F * D + D * F) * 2
        return self.layers * per_block + self.vocab * D * 2


@dataclass
class SamplingSettings:
    """src/inference/sampling/sampler.h:45-55."""
    mode: str = "greedy"
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0

    def ctype(self) -> _lib.Sampling:
        return _lib.Sampling(0 if self.mode == "greedy" else 1, self.top_k, self.temperature, self.top_p)


class Qwen3Model:
    """Resident parameters in the backend's packed layout."""

    def __init__(self, device: Device, queue: Queue, config: Qwen3Config):
        self.device, self.queue, self.config = device, queue, config
        cfg = config.ctype()
        handle = C.c_void_p()
        _lib.call("dl_qwen3_create", device.handle, queue.handle, C.byref(cfg), C.byref(handle))
        self.handle = handle
        self._native = _lib.Native("dl_qwen3_destroy", handle, device._native, queue._native)

    def fill_synthetic(self, seed: int, weight_std: float = 0.02) -> None:
        _lib.call("dl_qwen3_fill_synthetic", self.handle, self.queue.handle, seed, C.c_float(weight_std))

    def write(self, role: str, layer: int, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array, dtype=np.uint16).reshape(-1)
        _lib.call("dl_qwen3_write_tensor", self.handle, self.queue.handle, ROLE[role], layer,
                  a.ctypes.data_as(_lib.u16p), a.size)

    def read(self, role: str, layer: int = 0) -> np.ndarray:
        shape = self.config.shape(role)
        out = np.empty(int(np.prod(shape)), dtype=np.uint16)
        _lib.call("dl_qwen3_read_tensor", self.handle, self.queue.handle, ROLE[role], layer,
                  out.ctypes.data_as(_lib.u16p), out.size)
        return out.reshape(shape)

    def resident_bytes(self) -> int:
        n = C.c_uint64()
        _lib.call("dl_qwen3_resident_bytes", self.handle, C.byref(n))
        return n.value

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()


class Plan:
    """Cached forward plan for `batch` sequences with `capacity` positions."""

    def __init__(self, model: Qwen3Model, batch: int = 1, capacity: int = 8192):
        self.model, self.batch, self.capacity = model, batch, capacity
        handle = C.c_void_p()
        _lib.call("dl_plan_create", model.handle, model.queue.handle, batch, capacity, C.byref(handle))
        self.handle = handle
        self._native = _lib.Native("dl_plan_destroy", handle, model._native)
        self.max_new = 0

    # -- diagnostic chunk path
    def forward(self, tokens: Sequence[int]) -> None:
        a = np.ascontiguousarray(tokens, dtype=np.uint32)
        _lib.call("dl_plan_forward", self.handle, a.ctypes.data_as(_lib.u32p), a.size)

    def device_bytes(self) -> int:
        out = C.c_uint64(0)
        _lib.call("dl_plan_device_bytes", self.handle, C.byref(out))
        return out.value

    def seek(self, position: int) -> None:
        _lib.call("dl_plan_seek", self.handle, position)

    def position(self) -> int:
        p = C.c_uint64()
        _lib.call("dl_plan_position", self.handle, C.byref(p))
        return p.value

    def reset(self) -> None:
        _lib.call("dl_plan_reset", self.handle)

    def logits(self, seq: int = 0) -> np.ndarray:
        out = np.empty(self.model.config.vocab, dtype=np.uint16)
        _lib.call("dl_plan_read_logits", self.handle, seq, out.ctypes.data_as(_lib.u16p))
        return out

    def hidden(self, seq: int = 0) -> np.ndarray:
        out = np.empty(self.model.config.hidden, dtype=np.uint16)
        _lib.call("dl_plan_read_hidden", self.handle, seq, out.ctypes.data_as(_lib.u16p))
        return out

    def write_cache(self, layer: int, first: int, keys: np.ndarray, values: np.ndarray, seq: int = 0) -> None:
        k = np.ascontiguousarray(keys, dtype=np.uint16).reshape(-1)
        v = np.ascontiguousarray(values, dtype=np.uint16).reshape(-1)
        per_row = self.model.config.kv_heads * self.model.config.head_dim
        _lib.call("dl_plan_write_cache", self.handle, seq, layer, first, k.size // per_row,
                  k.ctypes.data_as(_lib.u16p), v.ctypes.data_as(_lib.u16p))

    def read_cache(self, layer: int, first: int, count: int, seq: int = 0) -> tuple[np.ndarray, np.ndarray]:
        per_row = self.model.config.kv_heads * self.model.config.head_dim
        k = np.empty(count * per_row, dtype=np.uint16)
        v = np.empty(count * per_row, dtype=np.uint16)
        _lib.call("dl_plan_read_cache", self.handle, seq, layer, first, count, k.ctypes.data_as(_lib.u16p),
                  v.ctypes.data_as(_lib.u16p))
        return k, v

    # -- hooks
    def set_capture(self, layer: int) -> None:
        _lib.call("dl_plan_set_capture", self.handle, layer)

    def read_capture(self, seq: int, first: int, count: int) -> np.ndarray:
        out = np.empty(count * self.model.config.hidden, dtype=np.uint16)
        _lib.call("dl_plan_read_capture", self.handle, seq, first, count, out.ctypes.data_as(_lib.u16p))
        return out.reshape(count, self.model.config.hidden)

    def set_steering(self, seq: int, layer: int, vector: Optional[np.ndarray]) -> None:
        if vector is None:
            _lib.call("dl_plan_set_steering", self.handle, seq, layer, None)
            return
        v = np.ascontiguousarray(vector, dtype=np.float32)
        _lib.call("dl_plan_set_steering", self.handle, seq, layer, v.ctypes.data_as(C.POINTER(C.c_float)))

    def set_embedding_override(self, position: int, row: Optional[np.ndarray], seq_mask: int) -> None:
        if row is None:
            _lib.call("dl_plan_set_embedding_override", self.handle, 0, None, 0)
            return
        r = np.ascontiguousarray(row, dtype=np.uint16)
        _lib.call("dl_plan_set_embedding_override", self.handle, position, r.ctypes.data_as(_lib.u16p), seq_mask)

    def set_injection(self, injection, position: int, seq_mask: int = 1) -> None:
        """Live injection (executor.cpp:1583-1632): the output row of a
        DeviceInjection (dolittle_amd.interventions) replaces the embedding
        of prompt position `position` for the sequences in `seq_mask`; its
        status gates the loop.  None removes it."""
        if injection is None:
            _lib.call("dl_plan_set_injection", self.handle, 0, None, 0, 0)
            return
        from .interventions import _DTYPE
        self._injection = injection  # the plan reads its storage until replaced
        _lib.call("dl_plan_set_injection", self.handle, position, injection.storage.ptr(),
                  _DTYPE[injection.output_type], seq_mask)

    def set_intervention(self, seq: int, layer: int, position: int, direction, strength: float) -> None:
        """Residual intervention (executor.cpp:1717-1748) on block `layer`'s
        output row of sequence `seq` at `position`.  `direction` is a device
        Region of `hidden` FP32 values (DeviceDirection.finish()) or a host
        FP32 array; None or strength 0 removes it."""
        if direction is None:
            _lib.call("dl_plan_set_intervention", self.handle, seq, -1, 0, None, C.c_float(0.0))
            return
        if isinstance(direction, np.ndarray):
            v = np.ascontiguousarray(direction, dtype=np.float32)
            if v.size != self.model.config.hidden:
                raise ValueError("direction width")
            ptr = v.ctypes.data_as(C.c_void_p)
        else:
            if direction.bytes != self.model.config.hidden * 4:
                raise ValueError("direction width")
            ptr = direction.ptr()
        _lib.call("dl_plan_set_intervention", self.handle, seq, layer, position, ptr, C.c_float(strength))

    def read_intervention(self) -> tuple[int, int]:
        status, count = C.c_uint32(), C.c_uint32()
        _lib.call("dl_plan_read_intervention", self.handle, C.byref(status), C.byref(count))
        return status.value, count.value

    # -- device-owned loop
    def _args(self, prompt, sampling, seeds, stop_ids):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        s = (sampling or SamplingSettings()).ctype()
        seeds_a = np.ascontiguousarray(seeds if seeds is not None else [0] * self.batch, dtype=np.uint64)
        stops = np.ascontiguousarray(stop_ids if stop_ids else [0], dtype=np.uint32)
        return p, s, seeds_a, stops, (len(stop_ids) if stop_ids else 0)

    def generate(self, prompt, max_new: int, sampling: Optional[SamplingSettings] = None, seeds=None,
                 stop_ids: Optional[Sequence[int]] = None) -> None:
        p, s, seeds_a, stops, n = self._args(prompt, sampling, seeds, stop_ids)
        _lib.call("dl_plan_generate", self.handle, p.ctypes.data_as(_lib.u32p), p.size, max_new, C.byref(s),
                  seeds_a.ctypes.data_as(_lib.u64p), stops.ctypes.data_as(_lib.u32p), n)
        self.max_new = max_new

    def prepare_generation(self, prompt, max_new: int, sampling: Optional[SamplingSettings] = None, seeds=None,
                           stop_ids: Optional[Sequence[int]] = None) -> None:
        p, s, seeds_a, stops, n = self._args(prompt, sampling, seeds, stop_ids)
        _lib.call("dl_plan_prepare_generation", self.handle, p.ctypes.data_as(_lib.u32p), p.size, max_new,
                  C.byref(s), seeds_a.ctypes.data_as(_lib.u64p), stops.ctypes.data_as(_lib.u32p), n)
        self.max_new = max_new

    def prefill(self, prompt, mfma: bool = False) -> None:
        """Prompt pass over positions [0, len(prompt) - 1); a following
        generate() with the same prompt resumes at the last prompt position.

        The default is the chunked exact pass: its caches, logits and tokens
        are bit-identical to consuming the prompt one position per step.
        mfma=True opts into the MFMA GEMM pass, a tolerance path: the MFMA
        units accumulate in their own order, so one projection is within one
        BF16 ulp of the exact chain and the flips compound over the blocks
        (at 36 Qwen3-8B blocks the first logits move by a few tenths and a
        greedy stream can leave the exact one after a few tokens)."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        _lib.call("dl_plan_prefill_mfma" if mfma else "dl_plan_prefill", self.handle,
                  p.ctypes.data_as(_lib.u32p), p.size)

    def decode_steps(self, steps: int) -> None:
        _lib.call("dl_plan_decode_steps", self.handle, steps)

    def collect(self) -> tuple[np.ndarray, list[dict]]:
        n = max(self.max_new, 1)
        tokens = np.zeros(self.batch * n, dtype=np.uint32)
        results = (_lib.GenerationResult * self.batch)()
        _lib.call("dl_plan_collect", self.handle, tokens.ctypes.data_as(_lib.u32p), n, results)
        out = []
        for r in results:
            out.append({"generated": r.generated, "reason": REASON.get(r.reason, r.reason), "status": r.status,
                        "active": bool(r.reserved), "position": r.position})
        return tokens.reshape(self.batch, n), out

    def request_stop(self) -> None:
        _lib.call("dl_plan_request_stop", self.handle)

    # -- DeviceSequence event journal (src/inference/decoding/device.h:86-137)
    def collect_event(self, seq: int, index: int, wait: bool = True) -> Optional[dict]:
        """Event `index` of sequence `seq` as a dict, or None when `wait` is
        False and it is not published yet."""
        ev = _lib.SequenceEvent()
        ready = C.c_int(0)
        _lib.call("dl_plan_collect_event", self.handle, seq, index, 1 if wait else 0, C.byref(ev), C.byref(ready))
        if not ready.value:
            return None
        return {"kind": EVENT_KIND.get(ev.kind, ev.kind), "status": ev.status, "position": ev.position,
                "count": ev.count, "token": ev.token, "norm": ev.norm}

    def event_count(self, seq: int = 0) -> int:
        n = C.c_uint64()
        _lib.call("dl_plan_event_count", self.handle, seq, C.byref(n))
        return n.value

    def events(self, seq: int = 0) -> list[dict]:
        """Every event of sequence `seq` up to and including its terminal
        event (waits for it)."""
        out = []
        while not out or out[-1]["kind"] != "terminal":
            out.append(self.collect_event(seq, len(out)))
        return out

    def set_step_window(self, steps: int) -> None:
        _lib.call("dl_plan_set_step_window", self.handle, steps)

    def steps_enqueued(self) -> int:
        n = C.c_uint64()
        _lib.call("dl_plan_steps_enqueued", self.handle, C.byref(n))
        return n.value

    def __del__(self):
        native = getattr(self, "_native", None)
        if native is not None:
            native.release()
