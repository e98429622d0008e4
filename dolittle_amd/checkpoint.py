"""Checkpoint archives and the Qwen3 checkpoint binding over libdlhip.so.

Mirrors safetensors::parse_header and safetensors::open
(src/tensors/formats/safetensors.h:101-117), and qwen3::parse_config,
bind_parameters and bind_causal_lm (src/models/qwen3/checkpoint.h:104-123).
Parsing, integrity checks, binding and the upload run in the library's C++
code; this module only marshals arguments.  Errors raise the library's
InvalidArgument / LengthError / DeviceError, the reference's
invalid_argument / length_error / runtime_error.

`write_safetensors` writes the standard file format (eight-byte
little-endian header length, JSON header, payload) for tests and tools.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import dataclass
from typing import Mapping, Optional, Sequence

import numpy as np

from . import _lib

DTYPE_NAME = {1: "BF16", 2: "F32", 3: "U32"}
WEIGHT_TYPE = {"bfloat16": 1, "float32": 2}
INTEGRITY = {"sha256": 0, "prepared_setup": 1}


@dataclass(frozen=True)
class TensorEntry:
    name: str
    dtype: str
    shape: tuple
    data_offset: int
    byte_count: int


@dataclass(frozen=True)
class ArtifactSpec:
    """formats::Artifact: a declared file, its size and SHA-256."""
    relative_path: str
    byte_size: int
    sha256: str

    @staticmethod
    def of(root: str, relative_path: str) -> "ArtifactSpec":
        path = os.path.join(root, relative_path)
        with open(path, "rb") as f:
            data = f.read()
        return ArtifactSpec(relative_path, len(data), sha256_hex(data))


def _entry(info: _lib.TensorInfo) -> TensorEntry:
    shape = tuple(info.shape[i] for i in range(info.rank))
    return TensorEntry(info.name.decode(), DTYPE_NAME.get(info.dtype, str(info.dtype)), shape, info.data_offset,
                       info.byte_count)


class Archive:
    """An opened archive or a decoded header catalog (TensorArchive)."""

    def __init__(self, handle: C.c_void_p):
        self.handle = handle

    def tensors(self) -> list[TensorEntry]:
        n = C.c_uint64()
        _lib.call("dl_archive_tensor_count", self.handle, C.byref(n))
        out = []
        for i in range(n.value):
            info = _lib.TensorInfo()
            _lib.call("dl_archive_tensor_info", self.handle, i, C.byref(info))
            out.append(_entry(info))
        return out

    def payload(self, name: str) -> bytes:
        info = _lib.TensorInfo()
        _lib.call("dl_archive_find", self.handle, name.encode(), C.byref(info))
        if not info.payload:
            return b""
        return C.string_at(info.payload, info.byte_count)

    def artifact(self, path: str) -> bytes:
        data, size = C.c_void_p(), C.c_uint64()
        _lib.call("dl_archive_artifact", self.handle, path.encode(), C.byref(data), C.byref(size))
        return C.string_at(data, size.value) if size.value else b""

    def identity(self) -> tuple[str, str, str]:
        repo, rev, digest = C.c_char_p(), C.c_char_p(), C.c_char_p()
        _lib.call("dl_archive_identity", self.handle, C.byref(repo), C.byref(rev), C.byref(digest))
        return repo.value.decode(), rev.value.decode(), digest.value.decode()

    def close(self) -> None:
        if self.handle:
            _lib.call("dl_archive_destroy", self.handle)
            self.handle = None

    def __del__(self):
        if not _lib.releasing():
            return
        try:
            self.close()
        except Exception:
            pass


def parse_header(header: bytes, data_bytes: int, max_header_bytes: int = 1 << 20,
                 max_metadata_bytes: int = 1 << 20, max_tensor_count: int = 100) -> Archive:
    """safetensors::parse_header: the JSON header alone (no eight-byte prefix)."""
    limits = _lib.ArchiveLimits(max_header_bytes, max_metadata_bytes, max_tensor_count)
    handle = C.c_void_p()
    _lib.call("dl_safetensors_parse_header", header, len(header), data_bytes, C.byref(limits), C.byref(handle))
    return Archive(handle)


def open_archive(root: str, repository: str, revision: str, artifacts: Sequence[ArtifactSpec],
                 shards: Sequence[str], index: Optional[str] = None, max_header_bytes: int = 100 << 20,
                 max_metadata_bytes: int = 256 << 20, max_tensor_count: int = 1 << 16,
                 verification_workers: int = 1, integrity: str = "sha256") -> Archive:
    """safetensors::open over explicitly declared artifacts and shards."""
    arts = (_lib.Artifact * max(len(artifacts), 1))()
    for i, a in enumerate(artifacts):
        arts[i] = _lib.Artifact(a.relative_path.encode(), a.byte_size, a.sha256.encode())
    names = (C.c_char_p * max(len(shards), 1))(*[s.encode() for s in shards])
    request = _lib.ArchiveRequest(root.encode(), repository.encode(), revision.encode(), arts, names,
                                  index.encode() if index else None, max_header_bytes, max_metadata_bytes,
                                  max_tensor_count, len(artifacts), len(shards), verification_workers,
                                  INTEGRITY.get(integrity, -1))
    handle = C.c_void_p()
    _lib.call("dl_safetensors_open", C.byref(request), C.byref(handle))
    return Archive(handle)


def _config(c: _lib.Qwen3Config):
    from .qwen3 import Qwen3Config
    return Qwen3Config(c.layers, c.hidden, c.q_heads, c.kv_heads, c.head_dim, c.ffn, c.vocab,
                       bool(c.tied_embeddings), c.rms_eps, c.rope_theta)


def parse_config(text: bytes, weight_type: str = "bfloat16", max_metadata_bytes: int = 16 << 20):
    """qwen3::parse_config -> (Qwen3Config, context limit)."""
    out, context = _lib.Qwen3Config(), C.c_uint64()
    _lib.call("dl_qwen3_parse_config", text, len(text), WEIGHT_TYPE.get(weight_type, 0), max_metadata_bytes,
              C.byref(out), C.byref(context))
    return _config(out), context.value


def tensor_name(role: str, layer: int = 0) -> str:
    from .qwen3 import ROLE
    buf = C.create_string_buffer(256)
    _lib.call("dl_qwen3_tensor_name", ROLE[role], layer, buf, len(buf))
    return buf.value.decode()


def bind_parameters(config, weight_type: str, catalog: Archive) -> None:
    """qwen3::bind_parameters: raises unless the catalog is exactly the config's parameters."""
    c = config.ctype()
    _lib.call("dl_qwen3_bind_parameters", C.byref(c), WEIGHT_TYPE.get(weight_type, 0), catalog.handle)


def bind_archive(archive: Archive, configuration_artifact: str = "config.json"):
    """bind_causal_lm -> (Qwen3Config, context limit, parameter bytes)."""
    out, context, total = _lib.Qwen3Config(), C.c_uint64(), C.c_uint64()
    _lib.call("dl_qwen3_bind_archive", archive.handle, configuration_artifact.encode(), C.byref(out),
              C.byref(context), C.byref(total))
    return _config(out), context.value, total.value


def load_qwen3(device, queue, archive: Archive, configuration_artifact: str = "config.json"):
    """Creates a resident model from the archive's config and uploads its parameters."""
    from .qwen3 import Qwen3Model
    config, _, _ = bind_archive(archive, configuration_artifact)
    model = Qwen3Model(device, queue, config)
    _lib.call("dl_qwen3_load", model.handle, queue.handle, archive.handle, configuration_artifact.encode())
    model._archive = archive  # provenance; the resident copy no longer needs the mapping
    return model


def sha256_hex(data: bytes) -> str:
    out = C.create_string_buffer(65)
    buf = C.create_string_buffer(data, len(data)) if data else None
    _lib.call("dl_sha256_hex", buf, len(data), out)
    return out.value.decode()


_NUMPY = {"BF16": np.uint16, "F32": np.float32, "U32": np.uint32}


def write_safetensors(path: str, tensors: Mapping[str, tuple], metadata: Optional[dict] = None) -> None:
    """Writes {name: (dtype name, array)} in the safetensors format: payloads
    in name order, the header padded with spaces to eight bytes."""
    header, offset, blobs = {}, 0, []
    for name in sorted(tensors):
        dtype, array = tensors[name]
        a = np.ascontiguousarray(array, dtype=_NUMPY[dtype])
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [offset, offset + a.nbytes]}
        offset += a.nbytes
        blobs.append(a.tobytes())
    if metadata is not None:
        header["__metadata__"] = metadata
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * ((8 - len(text) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little"))
        f.write(text)
        for b in blobs:
            f.write(b)
