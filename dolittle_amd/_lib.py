"""ctypes binding of libdlhip.so (the C ABI declared in include/dolittle_hip.h).

The product path has no CPU fallback: if the HIP library is missing this
module raises at import of the first entry point that needs it.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libdlhip.so")
HEADER = os.path.join(HERE, "..", "include", "dolittle_hip.h")

_lib = None
_finalizing = False


def _mark_finalizing() -> None:
    global _finalizing
    _finalizing = True


atexit.register(_mark_finalizing)


class Native:
    """A native handle and the handles it was created from (its parents).

    The C ABI requires dependents to go first: a device outlives its queues
    and buffers, a queue and model outlive their plans (src/gpu/device.h:
    "Device ... outlives every resource and queue it creates").  Python may
    finalize the objects of one garbage cycle in any order, so destruction
    is deferred: a handle is destroyed once its owner released it and every
    handle created from it is destroyed, then its parents are reconsidered."""

    __slots__ = ("destroy", "handle", "parents", "dependents", "released", "destroyed")

    def __init__(self, destroy: str, handle, *parents: "Native"):
        self.destroy, self.handle, self.parents = destroy, handle, tuple(p for p in parents if p is not None)
        self.dependents, self.released, self.destroyed = 0, False, False
        for parent in self.parents:
            parent.dependents += 1

    def release(self) -> None:
        self.released = True
        self._collect()

    def _collect(self) -> None:
        if not self.released or self.dependents or self.destroyed:
            return
        self.destroyed = True
        if not _finalizing:
            try:
                call(self.destroy, self.handle)
            except Exception:
                pass
        for parent in self.parents:
            parent.dependents -= 1
            parent._collect()


def releasing() -> bool:
    """False once the interpreter is shutting down.  Objects still alive then
    (for example held by a stored traceback) are finalized in no particular
    order, so a plan could be destroyed after its queue; their destructors
    leave native handles to the process exit instead."""
    return not _finalizing

u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
vp = C.c_void_p
vpp = C.POINTER(C.c_void_p)
u64 = C.c_uint64
u32 = C.c_uint32
i32 = C.c_int32
cint = C.c_int


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 64), ("compute_units", C.c_uint32),
                ("reserved", C.c_uint32), ("total_bytes", C.c_uint64)]


class Qwen3Config(C.Structure):
    _fields_ = [("layers", C.c_uint32), ("hidden", C.c_uint32), ("q_heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ffn", C.c_uint32),
                ("vocab", C.c_uint32), ("tied_embeddings", C.c_uint32), ("rms_eps", C.c_float),
                ("reserved", C.c_uint32), ("rope_theta", C.c_double)]


class Sampling(C.Structure):
    _fields_ = [("mode", C.c_uint32), ("top_k", C.c_uint32), ("temperature", C.c_double),
                ("top_p", C.c_double)]


class GenerationResult(C.Structure):
    _fields_ = [("generated", C.c_uint32), ("reason", C.c_uint32), ("status", C.c_uint32),
                ("reserved", C.c_uint32), ("position", C.c_uint64)]


class SequenceEvent(C.Structure):
    _fields_ = [("kind", C.c_uint8), ("reserved", C.c_uint8 * 3), ("status", C.c_uint32), ("position", C.c_uint64),
                ("count", C.c_uint64), ("token", C.c_uint32), ("norm", C.c_float)]


class ArchiveLimits(C.Structure):
    _fields_ = [("max_header_bytes", C.c_uint64), ("max_metadata_bytes", C.c_uint64),
                ("max_tensor_count", C.c_uint64)]


class Artifact(C.Structure):
    _fields_ = [("relative_path", C.c_char_p), ("byte_size", C.c_uint64), ("sha256", C.c_char_p)]


class ArchiveRequest(C.Structure):
    _fields_ = [("root", C.c_char_p), ("repository", C.c_char_p), ("revision", C.c_char_p),
                ("artifacts", C.POINTER(Artifact)), ("shards", C.POINTER(C.c_char_p)), ("index", C.c_char_p),
                ("max_header_bytes", C.c_uint64), ("max_metadata_bytes", C.c_uint64),
                ("max_tensor_count", C.c_uint64), ("artifact_count", C.c_uint32), ("shard_count", C.c_uint32),
                ("verification_workers", C.c_uint32), ("integrity", C.c_int32)]


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("shape", C.POINTER(C.c_uint64)), ("payload", C.c_void_p),
                ("data_offset", C.c_uint64), ("byte_count", C.c_uint64), ("rank", C.c_uint32),
                ("dtype", C.c_int32)]


# name -> argument types (all return int status)
SIGNATURES = {
    "dl_device_open": [cint, vpp],
    "dl_device_close": [vp],
    "dl_device_info_get": [vp, C.POINTER(DeviceInfo)],
    "dl_memory_snapshot": [vp, u64p, u64p],
    "dl_buffer_alloc": [vp, u64, u64, vpp],
    "dl_staging_alloc": [vp, u64, vpp],
    "dl_buffer_free": [vp],
    "dl_buffer_address": [vp, vpp],
    "dl_buffer_size": [vp, u64p],
    "dl_queue_create": [vp, vpp],
    "dl_queue_destroy": [vp],
    "dl_queue_upload": [vp, vp, u64, vp, u64, u64],
    "dl_queue_download": [vp, vp, u64, vp, u64, u64],
    "dl_queue_copy": [vp, vp, u64, vp, u64, u64],
    "dl_queue_write": [vp, vp, u64, vp, u64],
    "dl_queue_read": [vp, vp, vp, u64, u64],
    "dl_queue_mark": [vp, u64p],
    "dl_queue_wait": [vp, u64],
    "dl_queue_drain": [vp],
    "dl_event_create": [vp, vpp],
    "dl_event_destroy": [vp],
    "dl_event_record": [vp, vp],
    "dl_event_elapsed_ms": [vp, vp, C.POINTER(C.c_float)],
    "dl_projection": [vp, cint, vp, vp, vp, u64, u64, u64, vp],
    "dl_rms_norm": [vp, cint, vp, vp, vp, u64, u64, C.c_float],
    "dl_rotary": [vp, cint, vp, vp, u64, u64, u64, u64, C.c_double, vp, cint],
    "dl_attention_scale": [vp, vp, u64],
    "dl_attention": [vp, cint, vp, vp, vp, vp, u64, u64, u64, u64, u64, vp, u64, vp],
    "dl_embedding": [vp, cint, vp, vp, vp, u64, u64, u64],
    "dl_add": [vp, cint, vp, vp, vp, u64],
    "dl_silu_multiply": [vp, cint, vp, vp, vp, u64],
    "dl_gather_rows": [vp, vp, vp, u64, u64p, u64],
    "dl_projection_packed_bytes": [u64, u64, u64p],
    "dl_projection_pack": [vp, vp, vp, u64, u64],
    "dl_projection_packed": [vp, vp, vp, vp, u64, u64, u64, vp],
    "dl_qwen3_create": [vp, vp, C.POINTER(Qwen3Config), vpp],
    "dl_qwen3_destroy": [vp],
    "dl_qwen3_fill_synthetic": [vp, vp, u64, C.c_float],
    "dl_qwen3_write_tensor": [vp, vp, cint, u32, u16p, u64],
    "dl_qwen3_read_tensor": [vp, vp, cint, u32, u16p, u64],
    "dl_qwen3_resident_bytes": [vp, u64p],
    "dl_plan_create": [vp, vp, u32, u32, vpp],
    "dl_plan_destroy": [vp],
    "dl_plan_reset": [vp],
    "dl_plan_position": [vp, u64p],
    "dl_plan_write_cache": [vp, u32, u32, u64, u64, u16p, u16p],
    "dl_plan_read_cache": [vp, u32, u32, u64, u64, u16p, u16p],
    "dl_plan_seek": [vp, u64],
    "dl_plan_read_hidden": [vp, u32, u16p],
    "dl_plan_forward": [vp, u32p, u32],
    "dl_plan_read_logits": [vp, u32, u16p],
    "dl_plan_logits_address": [vp, u32, vpp],
    "dl_plan_set_capture": [vp, i32],
    "dl_plan_read_capture": [vp, u32, u64, u64, u16p],
    "dl_plan_set_steering": [vp, u32, i32, C.POINTER(C.c_float)],
    "dl_plan_set_embedding_override": [vp, u64, u16p, u32],
    "dl_plan_set_injection": [vp, u64, vp, cint, u32],
    "dl_plan_set_intervention": [vp, u32, i32, u64, vp, C.c_float],
    "dl_plan_read_intervention": [vp, u32p, u32p],
    "dl_plan_generate": [vp, u32p, u32, u32, C.POINTER(Sampling), u64p, u32p, u32],
    "dl_plan_prepare_generation": [vp, u32p, u32, u32, C.POINTER(Sampling), u64p, u32p, u32],
    "dl_plan_decode_steps": [vp, u32],
    "dl_plan_collect": [vp, u32p, u32, C.POINTER(GenerationResult)],
    "dl_plan_bench_prepare": [vp],
    "dl_plan_launch_kernel": [vp, u32, u32, u32],
    "dl_plan_set_grid": [vp, u32, u32],
    "dl_plan_request_stop": [vp],
    "dl_plan_collect_event": [vp, u32, u64, cint, vp, C.POINTER(cint)],
    "dl_plan_event_count": [vp, u32, C.POINTER(u64)],
    "dl_plan_set_step_window": [vp, u32],
    "dl_queue_transfer": [vp, vp, vp, u64],
    "dl_plan_device_bytes": [vp, u64p],
    "dl_sequence_device_bytes": [u64p],
    "dl_sequence_host_bytes": [u64, u64, u64, u64p],
    "dl_sequence_create": [vp, u64, u64, u64, cint, vpp],
    "dl_sequence_destroy": [vp],
    "dl_sequence_position_address": [vp, vpp],
    "dl_sequence_begin": [vp, vp, vp, vp, u64, vp, u64, vp, vp, vp, vp],
    "dl_sequence_begin_stage": [vp, cint],
    "dl_sequence_end_stage": [vp],
    "dl_sequence_begin_selection": [vp],
    "dl_sequence_capture": [vp, vp, u64, vp, u64, u64, u64],
    "dl_sequence_replace": [vp, vp, u64, vp, u64, u64, u64],
    "dl_sequence_complete": [vp],
    "dl_sequence_resources": [vp, u64p, u64p],
    "dl_sequence_start": [vp],
    "dl_sequence_request_stop": [vp],
    "dl_sequence_drain": [vp],
    "dl_sequence_collect": [vp, u64, cint, vp, C.POINTER(cint)],
    "dl_sequence_event_count": [vp, u64p],
    "dl_plan_steps_enqueued": [vp, C.POINTER(u64)],
    "dl_plan_prefill": [vp, u32p, u32],
    "dl_plan_prefill_mfma": [vp, u32p, u32],
    "dl_plan_read_prefill_hidden": [vp, u64, u64, u16p],
    "dl_plan_read_prefill_buffer": [vp, u32, u64, u64, u16p],
    "dl_prefill_projection": [vp, vp, vp, vp, vp, u64, u64, u64],
    "dl_prefill_attention": [vp, vp, vp, vp, vp, u64, u64, u64, u64, u64],
    "dl_prefill_gate_up": [vp, vp, vp, vp, vp, u64, u64, u64],
    "dl_sampler_required_bytes": [u64, C.POINTER(u64)],
    "dl_sampler_create": [vp, vp, u64, cint, u64, vpp],
    "dl_sampler_destroy": [vp],
    "dl_sampler_submit": [vp, vp, u64, C.POINTER(Sampling), u64],
    "dl_sampler_start": [vp, C.POINTER(Sampling), u64, u32p, u32],
    "dl_sampler_submit_next": [vp, vp, u64],
    "dl_sampler_result_address": [vp, vpp],
    "dl_sampler_terminal_address": [vp, vpp],
    "dl_sampler_current_token_address": [vp, vpp],
    "dl_sampler_result": [vp, u32p, u32p],
    "dl_sampler_set_exact": [vp, cint],
    "dl_sampler_exact_replays": [vp, C.POINTER(u64)],
    "dl_sample_noalloc": [vp, vp, u64, u64, C.POINTER(Sampling), u64, u32p],
    "dl_injection_bytes": [u64, cint, u64p],
    "dl_injection_submit": [vp, vp, cint, cint, u64, C.c_float, vp],
    "dl_direction_bytes": [u64, u64p],
    "dl_direction_submit": [vp, vp, vp, cint, u64, vp],
    "dl_intervention_initialize": [vp, vp],
    "dl_intervention_submit": [vp, vp, cint, u64, u64, vp, vp, u64, C.c_float, vp],
    "dl_safetensors_parse_header": [C.c_char_p, u64, u64, C.POINTER(ArchiveLimits), vpp],
    "dl_safetensors_open": [C.POINTER(ArchiveRequest), vpp],
    "dl_archive_destroy": [vp],
    "dl_archive_tensor_count": [vp, u64p],
    "dl_archive_tensor_info": [vp, u64, C.POINTER(TensorInfo)],
    "dl_archive_find": [vp, C.c_char_p, C.POINTER(TensorInfo)],
    "dl_archive_identity": [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.POINTER(C.c_char_p)],
    "dl_archive_artifact": [vp, C.c_char_p, vpp, u64p],
    "dl_sha256_hex": [vp, u64, C.c_char_p],
    "dl_qwen3_parse_config": [C.c_char_p, u64, cint, u64, C.POINTER(Qwen3Config), u64p],
    "dl_qwen3_tensor_name": [cint, u32, C.c_char_p, u64],
    "dl_qwen3_bind_parameters": [C.POINTER(Qwen3Config), cint, vp],
    "dl_qwen3_bind_archive": [vp, C.c_char_p, C.POINTER(Qwen3Config), u64p, u64p],
    "dl_qwen3_load": [vp, vp, vp, C.c_char_p],
}


class DolittleError(RuntimeError):
    """Base class; the subclass mirrors the reference exception type."""


class InvalidArgument(DolittleError, ValueError):
    pass


class LengthError(DolittleError):
    pass


class DeviceError(DolittleError):
    pass


class Poisoned(DeviceError):
    pass


_STATUS = {1: InvalidArgument, 2: LengthError, 3: DeviceError, 4: Poisoned}


def header_functions() -> list[str]:
    """Every function declared by include/dolittle_hip.h."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|const char\*)\s+(dl_[a-z0-9_]+)\s*\(", text, flags=re.M)


def load():
    """Loads libdlhip.so; raises if the HIP extension is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise ImportError(f"libdlhip.so is not built ({LIBRARY}); run `python -m dolittle_amd.build`")
    lib = C.CDLL(LIBRARY)
    lib.dl_last_error.restype = C.c_char_p
    lib.dl_last_error.argtypes = []
    for name, args in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            continue  # reported by missing_exports() and the ABI test
        fn.argtypes = args
        fn.restype = cint
    _lib = lib
    return lib


def missing_exports() -> list[str]:
    """Functions declared by the header but not exported by the library."""
    lib = load()
    missing = []
    for name in header_functions():
        try:
            getattr(lib, name)
        except AttributeError:
            missing.append(name)
    return missing


def check(status: int) -> None:
    if status != 0:
        message = load().dl_last_error().decode(errors="replace")
        raise _STATUS.get(status, DolittleError)(message or f"status {status}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
