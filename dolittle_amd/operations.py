"""Host mirror of the reference operation catalog (src/kernels/operations.h:
169-271): the eight Operation types, validate_operation, prepare() and
PreparedOperation.{workspace, initialize, operands, implementation_name,
submit}.

Validation restates src/kernels/operations.cpp:28-204 (same conditions,
same exception classes); submission calls the gfx950 kernels of
libdlhip.so through the C ABI.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from typing import Optional, Sequence, Union

from . import _lib
from .runtime import Device, DeviceBuffer, Queue

BF16 = "bfloat16"
F32 = "float32"
U32 = "uint32"
_DTYPE = {BF16: 1, F32: 2}
_ELEMENT_BYTES = {BF16: 2, F32: 4, U32: 4}


@dataclass(frozen=True)
class TensorId:
    value: int


@dataclass(frozen=True)
class Embedding:
    tokens: TensorId
    weight: TensorId
    output: TensorId


@dataclass(frozen=True)
class Projection:
    input: TensorId
    weight: TensorId
    output: TensorId


@dataclass(frozen=True)
class RmsNorm:
    input: TensorId
    weight: TensorId
    output: TensorId
    epsilon: float


@dataclass(frozen=True)
class Rotary:
    input: TensorId
    output: TensorId
    first_position: int
    theta: float


@dataclass(frozen=True)
class CausalAttention:
    query: TensorId
    key: TensorId
    value: TensorId
    output: TensorId


@dataclass(frozen=True)
class Add:
    left: TensorId
    right: TensorId
    output: TensorId


@dataclass(frozen=True)
class SiluMultiply:
    gate: TensorId
    up: TensorId
    output: TensorId


@dataclass(frozen=True)
class GatherRows:
    input: TensorId
    output: TensorId
    rows: tuple


Operation = Union[Embedding, Projection, RmsNorm, Rotary, CausalAttention, Add, SiluMultiply, GatherRows]


@dataclass(frozen=True)
class Layout:
    """Dense row-major layout (src/tensors/tensor.h)."""
    element_type: str
    shape: tuple

    @property
    def elements(self) -> int:
        return math.prod(self.shape)

    @property
    def nbytes(self) -> int:
        return self.elements * _ELEMENT_BYTES[self.element_type]


@dataclass(frozen=True)
class ComputationMode:
    activation_storage: str = BF16
    reduction_accumulation: str = F32


@dataclass(frozen=True)
class RowPolicy:
    max_rows: int = 0
    last_row: bool = False


@dataclass(frozen=True)
class OperandUse:
    tensor: TensorId
    access: str  # "read" | "write"


@dataclass(frozen=True)
class OperandRequirement:
    tensor: TensorId
    access: str
    alignment: int


@dataclass
class BufferBinding:
    tensor: TensorId
    storage: DeviceBuffer
    offset: int = 0
    nbytes: int = 0
    positioned_output: bool = False

    def address(self) -> C.c_void_p:
        return self.storage.ptr(self.offset)


@dataclass
class ExecutionExtent:
    """operations.h:234-239: first position, active rows, optional device
    position (a DeviceBuffer holding a uint64) and device capacity."""
    first_position: int = 0
    active_rows: int = 0
    device_position: Optional[DeviceBuffer] = None
    device_capacity: int = 0


@dataclass
class ContiguousLayerView:
    """One layer of a contiguous KV cache, rows [capacity, kv_heads, width]
    (src/inference/cache/contiguous.h:82-118)."""
    keys: DeviceBuffer
    values: DeviceBuffer
    capacity: int


def _require(condition: bool) -> None:
    if not condition:
        raise _lib.InvalidArgument("operation descriptor violates its contract")


def _trailing(layout: Layout) -> int:
    return math.prod(layout.shape[1:])


def validate_operation(operation: Operation, layouts: Sequence[Layout],
                       mode: ComputationMode) -> list[OperandUse]:
    """operations.cpp:192-204 and the per-operation rules above it."""
    _require(mode.activation_storage in (BF16, F32) and mode.reduction_accumulation == F32)
    uses: list[OperandUse] = []

    def operand(tid: TensorId, access: str, etype: str) -> Layout:
        _require(0 <= tid.value < len(layouts))
        layout = layouts[tid.value]
        _require(layout.element_type == etype and layout.elements > 0)
        for use in uses:
            if use.tensor.value == tid.value:
                _require(use.access == "read" and access == "read")
                return layout
        uses.append(OperandUse(tid, access))
        return layout

    storage = mode.activation_storage
    read = lambda t: operand(t, "read", storage)  # noqa: E731
    write = lambda t: operand(t, "write", storage)  # noqa: E731
    op = operation
    if isinstance(op, Embedding):
        ids, w, out = operand(op.tokens, "read", U32), read(op.weight), write(op.output)
        _require(len(ids.shape) == 1 and len(w.shape) == 2 and len(out.shape) == 2)
        _require(out.shape[0] == ids.shape[0] and out.shape[1] == w.shape[1])
    elif isinstance(op, Projection):
        x, w, y = read(op.input), read(op.weight), write(op.output)
        _require(len(x.shape) >= 2 and len(y.shape) >= 2 and len(w.shape) == 2)
        _require(x.shape[0] == y.shape[0] and _trailing(x) == w.shape[1] and _trailing(y) == w.shape[0])
    elif isinstance(op, RmsNorm):
        x, w, y = read(op.input), read(op.weight), write(op.output)
        _require(len(x.shape) > 0 and len(w.shape) == 1)
        _require(x.shape == y.shape and x.shape[-1] == w.shape[0])
        _require(math.isfinite(op.epsilon) and op.epsilon > 0)
    elif isinstance(op, Rotary):
        x, y = read(op.input), write(op.output)
        _require(len(x.shape) == 3 and x.shape == y.shape)
        _require(x.shape[2] % 2 == 0 and math.isfinite(op.theta) and op.theta > 0)
        if op.first_position > 2**64 - 1 - (x.shape[0] - 1):
            raise _lib.LengthError("rotary position range overflows")
    elif isinstance(op, CausalAttention):
        q, k, v, y = read(op.query), read(op.key), read(op.value), write(op.output)
        _require(len(q.shape) == 3 and len(k.shape) == 3)
        _require(k.shape == v.shape and q.shape == y.shape)
        _require(q.shape[0] == k.shape[0] and q.shape[2] == k.shape[2] and q.shape[1] % k.shape[1] == 0)
    elif isinstance(op, (Add, SiluMultiply)):
        a, b = (op.left, op.right) if isinstance(op, Add) else (op.gate, op.up)
        la, lb, ly = read(a), read(b), write(op.output)
        _require(la.shape == lb.shape and la.shape == ly.shape)
    elif isinstance(op, GatherRows):
        x, y = read(op.input), write(op.output)
        _require(len(x.shape) > 0 and len(y.shape) == len(x.shape))
        _require(len(op.rows) > 0 and y.shape[0] == len(op.rows))
        _require(all(x.shape[i] == y.shape[i] for i in range(1, len(x.shape))))
        for i, r in enumerate(op.rows):
            _require(r < x.shape[0])
            _require(i == 0 or op.rows[i - 1] < r)
    else:
        _require(False)
    return uses


class PreparedOperation:
    """A validated operation bound to this backend (operations.h:240-266)."""

    def __init__(self, device: Device, operation: Operation, layouts: Sequence[Layout],
                 mode: ComputationMode, rows: RowPolicy):
        self.device = device
        self.operation = operation
        self.layouts = list(layouts)
        self.mode = mode
        self.rows = rows
        self.dtype = _DTYPE[mode.activation_storage]
        self._uses = validate_operation(operation, layouts, mode)

    def workspace(self) -> tuple[int, int]:
        """Only attention owns a persistent constant: the FP32 scale."""
        return (4, 4) if isinstance(self.operation, CausalAttention) else (0, 1)

    def initialize(self, queue: Queue, workspace: Optional[DeviceBuffer], offset: int = 0) -> None:
        if isinstance(self.operation, CausalAttention):
            width = self.layouts[self.operation.query.value].shape[2]
            _lib.call("dl_attention_scale", queue.handle, workspace.ptr(offset), width)

    def operands(self) -> list[OperandRequirement]:
        return [OperandRequirement(u.tensor, u.access, _ELEMENT_BYTES[self.layouts[u.tensor.value].element_type])
                for u in self._uses]

    def implementation_name(self) -> str:
        return "gfx950." + type(self.operation).__name__

    def submit(self, queue: Queue, bindings: Sequence[BufferBinding], workspace: Optional[DeviceBuffer] = None,
               extent: Optional[ExecutionExtent] = None, cache: Optional[ContiguousLayerView] = None,
               workspace_offset: int = 0) -> None:
        by_id = {b.tensor.value: b for b in bindings}
        for use in self._uses:
            binding = by_id.get(use.tensor.value)
            if binding is None or binding.storage is None:
                raise _lib.InvalidArgument("operation binding missing")
            if binding.offset + self.layouts[use.tensor.value].nbytes > binding.storage.nbytes:
                raise _lib.InvalidArgument("operation binding outside its buffer")
        op, L, q = self.operation, self.layouts, queue.handle
        addr = lambda t: by_id[t.value].address()  # noqa: E731
        dev_pos = C.c_void_p(extent.device_position.address) if extent and extent.device_position else None
        first = extent.first_position if extent else 0
        rows = L[_first_id(op).value].shape[0]
        if extent and extent.active_rows:
            rows = min(rows, extent.active_rows)
        if isinstance(op, Embedding):
            V, D = L[op.weight.value].shape
            _lib.call("dl_embedding", q, self.dtype, addr(op.tokens), addr(op.weight), addr(op.output), rows, D, V)
        elif isinstance(op, Projection):
            O, I = L[op.weight.value].shape
            out_pos = dev_pos if by_id[op.output.value].positioned_output else None
            _lib.call("dl_projection", q, self.dtype, addr(op.input), addr(op.weight), addr(op.output), rows, I, O,
                      out_pos)
        elif isinstance(op, RmsNorm):
            width = L[op.weight.value].shape[0]
            total_rows = L[op.input.value].elements // width
            _lib.call("dl_rms_norm", q, self.dtype, addr(op.input), addr(op.weight), addr(op.output), total_rows,
                      width, C.c_float(op.epsilon))
        elif isinstance(op, Rotary):
            _, heads, width = L[op.input.value].shape
            positioned = 1 if by_id[op.output.value].positioned_output else 0
            _lib.call("dl_rotary", q, self.dtype, addr(op.input), addr(op.output), rows, heads, width,
                      op.first_position + first, C.c_double(op.theta), dev_pos, positioned)
        elif isinstance(op, CausalAttention):
            _, hq, width = L[op.query.value].shape
            hkv = L[op.key.value].shape[1]
            if workspace is None:
                raise _lib.InvalidArgument("attention requires its initialized workspace")
            scale = workspace.ptr(workspace_offset)
            if cache is not None:
                keys, values, capacity = cache.keys.ptr(), cache.values.ptr(), cache.capacity
            else:
                keys, values, capacity = addr(op.key), addr(op.value), rows
            _lib.call("dl_attention", q, self.dtype, addr(op.query), keys, values, addr(op.output), rows, hq, hkv,
                      width, first, dev_pos, capacity, scale)
        elif isinstance(op, Add):
            _lib.call("dl_add", q, self.dtype, addr(op.left), addr(op.right), addr(op.output),
                      L[op.left.value].elements)
        elif isinstance(op, SiluMultiply):
            _lib.call("dl_silu_multiply", q, self.dtype, addr(op.gate), addr(op.up), addr(op.output),
                      L[op.gate.value].elements)
        elif isinstance(op, GatherRows):
            row_bytes = L[op.input.value].nbytes // L[op.input.value].shape[0]
            arr = (C.c_uint64 * len(op.rows))(*op.rows)
            _lib.call("dl_gather_rows", q, addr(op.input), addr(op.output), row_bytes, arr, len(op.rows))


def _first_id(op: Operation) -> TensorId:
    if isinstance(op, Embedding):
        return op.tokens
    if isinstance(op, (Projection, RmsNorm, Rotary, GatherRows)):
        return op.input
    if isinstance(op, CausalAttention):
        return op.query
    if isinstance(op, Add):
        return op.left
    return op.gate


def prepare(device: Device, operation: Operation, layouts: Sequence[Layout],
            mode: ComputationMode = ComputationMode(), rows: RowPolicy = RowPolicy()) -> PreparedOperation:
    """kernels::prepare (operations.h:268-271)."""
    return PreparedOperation(device, operation, layouts, mode, rows)
