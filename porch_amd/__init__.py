"""porch_amd — porch's tensor API on the MI355X (gfx950) fused-graph backend.

A Python mirror of porch's C++ API (reference include/porch/tensor.hpp,
ops.hpp, backend.hpp) over the C ABI of libporch_amd.so: the same names,
argument meanings and error behaviour, so programs and tests read like the
reference's.  Expressions record a DAG of IR nodes; materialisation sends
the DAG as a node table to porch_materialize, which plans it into fused
gfx950 kernels (compiled by hiprtc, cached by graph hash) and launches them
on the calling thread's stream.

Exceptions mirror the C++ ones: InvalidArgument (std::invalid_argument,
also a ValueError), OutOfRange (std::out_of_range, also an IndexError),
PorchError (std::runtime_error) and CompilationError.
"""

from __future__ import annotations

import builtins
import ctypes
import os
import json
import threading
from typing import Iterable, Sequence

import numpy as np

from ._lib import (
    OP,
    CompilationError,
    Graph,
    InvalidArgument,
    JitStats,
    Node,
    OutOfRange,
    PorchError,
    check,
    lib,
)

__all__ = [
    "device", "all", "slice", "tensor", "tensor_layout", "tensor_expr", "full", "zeros", "add",
    "subtract", "multiply", "divide", "matmul", "batched_matmul", "reshape", "unsqueeze",
    "transpose", "permute", "broadcast_to", "concat", "sum", "max", "maximum", "minimum",
    "exp", "reciprocal", "materialize", "relu", "softmax", "logistic",
    "backend", "backend_kind", "backend_for", "is_backend_available",
    "backend_name", "is_available", "synchronize", "plan", "kernel_source",
    "jit_stats", "reset_jit_cache", "serialize", "InvalidArgument",
    "OutOfRange", "PorchError", "CompilationError",
]


# ----------------------------------------------------------------------------
# placement, subscripts
# ----------------------------------------------------------------------------


class device:
    """A GPU ordinal (reference include/porch/tensor.hpp:15-31)."""

    __slots__ = ("_ordinal",)

    def __init__(self, ordinal: int = 0):
        self._ordinal = int(ordinal)

    def ordinal(self) -> int:
        return self._ordinal

    def is_cuda(self) -> bool:  # reference spelling of "is a GPU"
        return True

    def is_gpu(self) -> bool:
        return True

    def __eq__(self, other) -> bool:
        return isinstance(other, device) and other._ordinal == self._ordinal

    def __hash__(self) -> int:
        return hash(self._ordinal)

    def __repr__(self) -> str:
        return f"device({self._ordinal})"


class _All:
    def __repr__(self) -> str:
        return "all"


all = _All()  # noqa: A001 - porch's spelling


class slice:  # noqa: N801 - porch's spelling
    """[start, stop) with a positive step (reference tensor.hpp:37-41)."""

    __slots__ = ("start", "stop", "step")

    def __init__(self, start: int, stop: int, step: int = 1):
        self.start = int(start)
        self.stop = int(stop)
        self.step = int(step)


# ----------------------------------------------------------------------------
# device buffers
# ----------------------------------------------------------------------------


class _Buffer:
    """Owns one porch_buffer handle."""

    __slots__ = ("handle",)

    def __init__(self, handle: int | None):
        self.handle = handle

    def __del__(self):
        if self.handle:
            lib.porch_buffer_release(self.handle)
            self.handle = None

    @classmethod
    def empty(cls) -> "_Buffer":
        out = ctypes.c_void_p()
        check(lib.porch_buffer_create(0, ctypes.byref(out)))
        return cls(out.value)

    @classmethod
    def upload(cls, values: np.ndarray) -> "_Buffer":
        out = ctypes.c_void_p()
        check(lib.porch_buffer_create(values.nbytes, ctypes.byref(out)))
        buf = cls(out.value)
        if values.size:
            check(lib.porch_copy_to_device(buf.handle, values.ctypes.data, values.size))
        return buf

    def size_bytes(self) -> int:
        return int(lib.porch_buffer_size(self.handle))

    def empty_buffer(self) -> bool:
        return self.size_bytes() == 0

    def device_pointer(self) -> int:
        return int(lib.porch_buffer_device_pointer(self.handle))

    def download(self, count: int) -> np.ndarray:
        host = np.empty(count, dtype=np.float32)
        if count:
            check(lib.porch_copy_to_host(self.handle, host.ctypes.data, count))
        return host


class _Storage:
    __slots__ = ("buffer", "host", "lock")

    def __init__(self, buffer: _Buffer, host: np.ndarray | None):
        self.buffer = buffer
        self.host = host
        self.lock = threading.Lock()


# ----------------------------------------------------------------------------
# IR nodes
# ----------------------------------------------------------------------------


class _Node:
    __slots__ = ("kind", "input", "scalar", "lhs", "rhs", "shape", "strides",
                 "offset", "axis", "keepdim")

    def __init__(self, kind: str, lhs: "_Node | None" = None, rhs: "_Node | None" = None):
        self.kind = kind
        self.input = None
        self.scalar = 0.0
        self.lhs = lhs
        self.rhs = rhs
        self.shape: list[int] = []
        self.strides: list[int] = []
        self.offset = 0
        self.axis = 0
        self.keepdim = False


def serialize(root: "_Node | tensor_expr"):
    """Node table of an expression: (nodes, dims, input tensors).

    Inputs are numbered in first-visit order (lhs before rhs), the order in
    which the reference collects them (src/tensor.cpp:261-277).
    """
    if isinstance(root, tensor_expr):
        root = root._root
    order: list[_Node] = []
    index: dict[int, int] = {}
    stack = [(root, False)]
    while stack:
        node, expanded = stack.pop()
        if id(node) in index:
            continue
        if not expanded:
            stack.append((node, True))
            if node.rhs is not None and id(node.rhs) not in index:
                stack.append((node.rhs, False))
            if node.lhs is not None and id(node.lhs) not in index:
                stack.append((node.lhs, False))
            continue
        index[id(node)] = len(order)
        order.append(node)
    nodes = (Node * len(order))()
    dims: list[int] = []
    inputs: list[tensor] = []
    slot_of: dict[int, int] = {}
    placement = None
    for i, node in enumerate(order):
        c = nodes[i]
        c.op = OP[node.kind]
        c.lhs = index[id(node.lhs)] if node.lhs is not None else -1
        c.rhs = index[id(node.rhs)] if node.rhs is not None else -1
        c.input = -1
        c.scalar = node.scalar
        c.axis = node.axis
        c.keepdim = 1 if node.keepdim else 0
        c.offset = node.offset
        shape = node.shape
        if node.kind == "input":
            t = node.input
            if placement is None:
                placement = t.placement()
            elif placement != t.placement():
                raise InvalidArgument("tensor expression devices must match")
            key = id(t._state)
            if key not in slot_of:
                slot_of[key] = len(inputs)
                inputs.append(t)
            c.input = slot_of[key]
            # strided storage enters as its flat span, read through a slice
            shape = list(t.shape()) if t.is_contiguous() else [t._state.layout.span()]
        c.rank = len(shape)
        c.dims = len(dims)
        dims.extend(shape)
        if node.kind == "slice":
            dims.extend(node.strides)
    dims_array = (ctypes.c_int64 * builtins.max(len(dims), 1))(*dims)
    return nodes, dims_array, len(dims), inputs, placement


def _graph(nodes, dims, n_dims) -> Graph:
    return Graph(
        ctypes.cast(nodes, ctypes.POINTER(Node)), len(nodes),
        ctypes.cast(dims, ctypes.POINTER(ctypes.c_int64)), n_dims,
    )


def _infer(root: _Node):
    nodes, dims, n_dims, inputs, placement = serialize(root)
    g = _graph(nodes, dims, n_dims)
    shape = (ctypes.c_int64 * 64)()
    rank = ctypes.c_int32()
    scalar = ctypes.c_int32()
    check(lib.porch_infer_shape(ctypes.byref(g), shape, 64, ctypes.byref(rank),
                                ctypes.byref(scalar)))
    return [shape[i] for i in range(rank.value)], bool(scalar.value), inputs, placement


# ----------------------------------------------------------------------------
# tensor
# ----------------------------------------------------------------------------


class _State:
    __slots__ = ("shape", "placement", "storage", "expression", "lock", "layout", "dense",
                 "__weakref__")

    def __init__(self, shape: Sequence[int], placement: device):
        self.shape = tuple(int(e) for e in shape)
        self.placement = placement
        self.storage: _Storage | None = None
        self.expression: _Node | None = None
        self.lock = threading.Lock()
        self.layout: tensor_layout | None = None  # strided storage; None: contiguous
        self.dense: tensor | None = None          # strided: row-major copy for data()

    def realized(self) -> _Storage:
        storage = self.storage
        if storage is not None:
            return storage
        with self.lock:  # materialise exactly once
            if self.storage is None:
                self.storage = _materialize_node(self.expression)._state.storage
            return self.storage


def _contiguous_strides(shape: Sequence[int]) -> tuple[int, ...]:
    strides = [1] * len(shape)
    stride = 1
    for d in range(len(shape) - 1, -1, -1):
        strides[d] = stride
        stride *= shape[d]
    return tuple(strides)


def _checked_numel(shape: Sequence[int]) -> int:
    count = 1
    for extent in shape:
        if extent < 0:
            raise InvalidArgument("tensor shape extents must be non-negative")
        count *= extent
    return count


class tensor_layout:  # noqa: N801 - porch's spelling
    """porch::tensor_layout: shape, element strides and storage offset, with
    the reference's checks (src/tensor.cpp:1089-1116)."""

    __slots__ = ("_shape", "_strides", "_offset")

    def __init__(self, shape: Sequence[int], strides: Sequence[int] | None = None,
                 storage_offset: int = 0):
        self._shape = tuple(int(e) for e in shape)
        if strides is None:
            self._strides = _contiguous_strides(self._shape)
            self._offset = 0
        else:
            self._strides = tuple(int(e) for e in strides)
            self._offset = int(storage_offset)
            if len(self._strides) != len(self._shape):
                raise InvalidArgument("tensor layout rank mismatch")
            if self._offset < 0:
                raise InvalidArgument("tensor layout offset must be non-negative")
            if any(st < 0 for st in self._strides):
                raise InvalidArgument("tensor layout strides must be non-negative")
        _checked_numel(self._shape)

    def shape(self) -> tuple[int, ...]:
        return self._shape

    def strides(self) -> tuple[int, ...]:
        return self._strides

    def storage_offset(self) -> int:
        return self._offset

    def rank(self) -> int:
        return len(self._shape)

    def numel(self) -> int:
        return _checked_numel(self._shape)

    def is_contiguous(self) -> bool:
        return self._offset == 0 and self._strides == _contiguous_strides(self._shape)

    def span(self) -> int:
        """Floats of storage the layout reaches."""
        if self.numel() == 0:
            return 0
        return self._offset + builtins.sum((e - 1) * st for e, st in zip(self._shape, self._strides)) + 1


class tensor:  # noqa: N801 - porch's spelling
    """porch::tensor: a shared handle to realized or pending values.

    tensor(shape, values, placement=device()) uploads host values;
    tensor(expr) records a pending expression (the reference's implicit
    tensor_expr -> tensor conversion) that materialises once on first use;
    tensor(layout, storage, placement=device()) reads existing device storage
    (a device_data() buffer) through a strided layout, an extension: the
    reference rejects non-contiguous storage (src/tensor.cpp:1193-1197).
    """

    __slots__ = ("_state",)

    def __init__(self, shape, values=None, placement: device | None = None):
        placement = placement if placement is not None else device()
        if isinstance(shape, tensor_layout):
            layout, buffer = shape, values
            if not isinstance(buffer, _Buffer):
                raise InvalidArgument("strided tensors take a device buffer as storage")
            if buffer.size_bytes() < layout.span() * 4:
                raise InvalidArgument("tensor device storage is too small")
            self._state = _State(layout.shape(), placement)
            self._state.storage = _Storage(buffer, None)
            if not layout.is_contiguous():
                self._state.layout = layout
            return
        if isinstance(shape, tensor_expr):
            out_shape, scalar, inputs, where = _infer(shape._root)
            if not inputs:
                raise InvalidArgument("tensor expression must reference at least one tensor")
            if scalar:
                raise InvalidArgument("scalar expression cannot convert to a tensor")
            _checked_numel(out_shape)
            self._state = _State(out_shape, where)
            self._state.expression = shape._root
            return
        shape = [int(e) for e in shape]
        count = _checked_numel(shape)
        host = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
        if host.size != count:
            raise InvalidArgument("tensor data size does not match shape")
        self._state = _State(shape, placement)
        buffer = _Buffer.upload(host) if count else _Buffer.empty()
        self._state.storage = _Storage(buffer, host.copy())

    @classmethod
    def _realized(cls, shape, buffer: _Buffer, host, placement: device) -> "tensor":
        t = cls.__new__(cls)
        t._state = _State(shape, placement)
        t._state.storage = _Storage(buffer, host)
        return t

    # metadata
    def shape(self) -> tuple[int, ...]:
        return self._state.shape

    def strides(self) -> tuple[int, ...]:
        if self._state.layout is not None:
            return self._state.layout.strides()
        return _contiguous_strides(self._state.shape)

    def storage_offset(self) -> int:
        return 0 if self._state.layout is None else self._state.layout.storage_offset()

    def is_contiguous(self) -> bool:
        return self._state.layout is None

    def layout(self) -> tensor_layout:
        if self._state.layout is not None:
            return self._state.layout
        return tensor_layout(self._state.shape)

    def rank(self) -> int:
        return len(self._state.shape)

    def numel(self) -> int:
        return _checked_numel(self._state.shape)

    def placement(self) -> device:
        return self._state.placement

    # values
    def data(self) -> np.ndarray:
        """Host values (read-only view); materialises and waits for the GPU.
        Strided storage is gathered into row-major order on the device once."""
        if self._state.layout is not None:
            with self._state.lock:
                if self._state.dense is None:
                    self._state.dense = materialize(tensor_expr(self))
            return self._state.dense.data()
        storage = self._state.realized()
        with storage.lock:
            if storage.host is None:
                storage.host = storage.buffer.download(self.numel())
            view = storage.host.view()
        view.flags.writeable = False
        return view

    def cpu(self) -> np.ndarray:
        return np.array(self.data(), copy=True)

    def _storage_values(self) -> np.ndarray:
        """The raw storage (for strided storage: the span its layout reaches),
        as the node table's input slot holds it."""
        if self._state.layout is None:
            return self.data()
        storage = self._state.realized()
        with storage.lock:
            if storage.host is None:
                storage.host = storage.buffer.download(self._state.layout.span())
            return storage.host

    def device_data(self) -> _Buffer:
        return self._state.realized().buffer

    def realize(self) -> "tensor":
        self._state.realized()
        return self

    def synchronize(self) -> None:
        self._state.realized()
        check(lib.porch_synchronize())

    def __getitem__(self, indices) -> "tensor_expr":
        if not isinstance(indices, tuple):
            indices = (indices,)
        if len(indices) > self.rank():
            raise InvalidArgument("too many tensor indices")
        # restrict the tensor's strided view of its storage one subscript
        # at a time; axes past the last subscript stay whole
        base = self.storage_offset()
        extent = list(self.shape())
        step = list(self.strides())
        axis = 0
        for index in indices:
            if isinstance(index, builtins.slice):
                index = slice(0 if index.start is None else index.start,
                              extent[axis] if index.stop is None else index.stop,
                              1 if index.step is None else index.step)
            if isinstance(index, _All):
                axis += 1
            elif isinstance(index, slice):
                base += _narrow_axis(extent, step, axis, index)
                axis += 1
            else:
                base += _fix_axis(extent, step, axis, int(index))
        # the base and steps count storage elements: over strided storage
        # the slice reads the raw storage, not the tensor's view
        source = tensor_expr(self)._root if self.is_contiguous() else _storage_node(self)
        node = _Node("slice", source)
        node.shape = extent
        node.strides = step
        node.offset = base
        return tensor_expr._wrap(node)

    # arithmetic records expressions
    def __add__(self, other):
        return tensor_expr(self) + other

    def __radd__(self, other):
        return tensor_expr(other) + tensor_expr(self)

    def __sub__(self, other):
        return tensor_expr(self) - other

    def __rsub__(self, other):
        return tensor_expr(other) - tensor_expr(self)

    def __mul__(self, other):
        return tensor_expr(self) * other

    def __rmul__(self, other):
        return tensor_expr(other) * tensor_expr(self)

    def __truediv__(self, other):
        return tensor_expr(self) / other

    def __rtruediv__(self, other):
        return tensor_expr(other) / tensor_expr(self)


def _storage_node(value: "tensor") -> _Node:
    node = _Node("input")
    node.input = value
    return node


def _fix_axis(extent: list, step: list, axis: int, at: int) -> int:
    """Subscripts `axis` with an integer (counted from the end when
    negative): removes the axis and returns the storage offset it adds."""
    n = extent[axis]
    c = at + n if at < 0 else at
    if c < 0 or c >= n:
        raise OutOfRange("tensor index is out of bounds")
    offset = c * step[axis]
    del extent[axis], step[axis]
    return offset


def _narrow_axis(extent: list, step: list, axis: int, r: "slice") -> int:
    """Subscripts `axis` with a range: endpoints counted from the end when
    negative and clamped to [0, extent]; keeps every r.step-th coordinate
    from the first.  Returns the storage offset it adds."""
    if r.step <= 0:
        raise InvalidArgument("tensor slice step must be positive")
    n = extent[axis]
    first, end = (builtins.min(builtins.max(e + n if e < 0 else e, 0), n) for e in (r.start, r.stop))
    offset = first * step[axis]
    extent[axis] = (end - first - 1) // r.step + 1 if end > first else 0
    step[axis] *= r.step
    return offset


class tensor_expr:  # noqa: N801 - porch's spelling
    """porch::tensor_expr: an immutable DAG of IR nodes."""

    __slots__ = ("_root",)

    def __init__(self, value):
        if isinstance(value, tensor_expr):
            self._root = value._root
        elif isinstance(value, tensor):
            state = value._state
            if state.storage is None and state.expression is not None:
                self._root = state.expression  # inline a pending tensor
            elif state.layout is not None:
                # strided storage: the view is a slice of the raw storage
                view = _Node("slice", _storage_node(value))
                view.shape = list(state.layout.shape())
                view.strides = list(state.layout.strides())
                view.offset = state.layout.storage_offset()
                self._root = view
            else:
                self._root = _storage_node(value)
        else:
            node = _Node("scalar")
            node.scalar = float(np.float32(value))
            self._root = node

    @classmethod
    def _wrap(cls, node: _Node) -> "tensor_expr":
        e = cls.__new__(cls)
        e._root = node
        return e

    def eval(self) -> tensor:
        return materialize(self)

    def shape(self) -> list[int]:
        shape, scalar, _, _ = _infer(self._root)
        return [] if scalar else shape

    def rank(self) -> int:
        return len(self.shape())

    def numel(self) -> int:
        return _checked_numel(self.shape())

    def __add__(self, other):
        return _binary("add", self, other)

    def __radd__(self, other):
        return _binary("add", other, self)

    def __sub__(self, other):
        return _binary("subtract", self, other)

    def __rsub__(self, other):
        return _binary("subtract", other, self)

    def __mul__(self, other):
        return _binary("multiply", self, other)

    def __rmul__(self, other):
        return _binary("multiply", other, self)

    def __truediv__(self, other):
        return _binary("divide", self, other)

    def __rtruediv__(self, other):
        return _binary("divide", other, self)


def _expr(value) -> tensor_expr:
    return value if isinstance(value, tensor_expr) else tensor_expr(value)


def _binary(kind: str, lhs, rhs) -> tensor_expr:
    return tensor_expr._wrap(_Node(kind, _expr(lhs)._root, _expr(rhs)._root))


def _unary(kind: str, value) -> tensor_expr:
    return tensor_expr._wrap(_Node(kind, _expr(value)._root))


# ----------------------------------------------------------------------------
# free functions (reference tensor.hpp:185-224, ops.hpp:7-9)
# ----------------------------------------------------------------------------


def full(shape: Sequence[int], value: float, placement: device | None = None) -> tensor:
    count = _checked_numel([int(e) for e in shape])
    return tensor(shape, np.full(count, value, dtype=np.float32), placement)


def zeros(shape: Sequence[int], placement: device | None = None) -> tensor:
    return full(shape, 0.0, placement)


def add(lhs: tensor, rhs: tensor) -> tensor:
    return materialize(tensor_expr(lhs) + tensor_expr(rhs))


def subtract(lhs: tensor, rhs: tensor) -> tensor:
    return materialize(tensor_expr(lhs) - tensor_expr(rhs))


def multiply(lhs: tensor, rhs: tensor) -> tensor:
    return materialize(tensor_expr(lhs) * tensor_expr(rhs))


def divide(lhs: tensor, rhs: tensor) -> tensor:
    return materialize(tensor_expr(lhs) / tensor_expr(rhs))


def matmul(lhs, rhs) -> tensor_expr:
    return _binary("matmul", lhs, rhs)


def batched_matmul(lhs, rhs) -> tensor_expr:
    """[B, M, K] @ [B, K, N] -> [B, M, N]: matmul per batch entry.  An
    extension with no counterpart in the reference, whose matmul is rank-2
    only; broadcast_to a rank-2 operand to share it across the batch."""
    return _binary("batched_matmul", lhs, rhs)


def reshape(value, shape: Sequence[int]) -> tensor_expr:
    node = _Node("reshape", _expr(value)._root)
    node.shape = [int(e) for e in shape]
    return tensor_expr._wrap(node)


def unsqueeze(value, axis: int) -> tensor_expr:
    node = _Node("unsqueeze", _expr(value)._root)
    node.axis = int(axis)
    return tensor_expr._wrap(node)


def transpose(value) -> tensor_expr:
    return _unary("transpose", value)


def permute(value, dims: Sequence[int]) -> tensor_expr:
    """Rank-N axis permutation: output dimension i is dimension dims[i] of
    value (numpy.transpose's convention).  An extension with no counterpart
    in the reference, whose transpose is rank-2 only."""
    node = _Node("permute", _expr(value)._root)
    node.shape = [int(d) for d in dims]
    return tensor_expr._wrap(node)


def broadcast_to(value, shape: Sequence[int]) -> tensor_expr:
    node = _Node("broadcast", _expr(value)._root)
    node.shape = [int(e) for e in shape]
    return tensor_expr._wrap(node)


def concat(lhs, rhs, axis: int) -> tensor_expr:
    node = _Node("concat", _expr(lhs)._root, _expr(rhs)._root)
    node.axis = int(axis)
    return tensor_expr._wrap(node)


def sum(value, axis: int, keepdim: bool = False) -> tensor_expr:  # noqa: A001
    node = _Node("sum", _expr(value)._root)
    node.axis = int(axis)
    node.keepdim = bool(keepdim)
    return tensor_expr._wrap(node)


def max(value, axis: int, keepdim: bool = False) -> tensor_expr:  # noqa: A001
    node = _Node("max", _expr(value)._root)
    node.axis = int(axis)
    node.keepdim = bool(keepdim)
    return tensor_expr._wrap(node)


def maximum(lhs, rhs) -> tensor_expr:
    return _binary("maximum", lhs, rhs)


def minimum(lhs, rhs) -> tensor_expr:
    return _binary("minimum", lhs, rhs)


def exp(value) -> tensor_expr:
    return _unary("exp", value)


def reciprocal(value) -> tensor_expr:
    return _unary("reciprocal", value)


def relu(value) -> tensor_expr:
    return maximum(value, 0.0)


def softmax(value, axis: int) -> tensor_expr:
    value = _expr(value)
    shape = value.shape()
    shifted = value - broadcast_to(max(value, axis, True), shape)
    numerator = exp(shifted)
    return numerator / broadcast_to(sum(numerator, axis, True), shape)


def logistic(value) -> tensor_expr:
    return reciprocal(1.0 + exp(0.0 - _expr(value)))


def _materialize_node(root: _Node) -> tensor:
    nodes, dims, n_dims, inputs, placement = serialize(root)
    g = _graph(nodes, dims, n_dims)
    handles = (ctypes.c_void_p * builtins.max(len(inputs), 1))(
        *[t._state.realized().buffer.handle for t in inputs]
    )
    out = ctypes.c_void_p()
    shape = (ctypes.c_int64 * 64)()
    rank = ctypes.c_int32()
    check(lib.porch_materialize(ctypes.byref(g), handles, len(inputs), ctypes.byref(out),
                                shape, 64, ctypes.byref(rank)))
    out_shape = [shape[i] for i in range(rank.value)]
    buffer = _Buffer(out.value)
    host = np.empty(0, dtype=np.float32) if _checked_numel(out_shape) == 0 else None
    return tensor._realized(out_shape, buffer, host, placement or device())


def materialize(expression) -> tensor:
    return _materialize_node(_expr(expression)._root)


# ----------------------------------------------------------------------------
# backend selection and runtime (reference backend.hpp, cuda_jit.hpp)
# ----------------------------------------------------------------------------


class backend_kind:  # noqa: N801
    cuda_jit = 0
    hip_jit = 0


class backend:  # noqa: N801
    def __init__(self, kind: int = backend_kind.cuda_jit):
        self._kind = kind

    def kind(self) -> int:
        return self._kind

    def is_cuda_jit(self) -> bool:
        return self._kind == backend_kind.cuda_jit

    def is_hip_jit(self) -> bool:
        return self.is_cuda_jit()

    def __eq__(self, other) -> bool:
        return isinstance(other, backend) and other._kind == self._kind


def backend_for(placement: device) -> backend:
    return backend(backend_kind.cuda_jit)


def is_available() -> bool:
    return bool(lib.porch_is_available())


def is_backend_available(target: backend) -> bool:
    return target.is_cuda_jit() and is_available()


def backend_name(target: backend) -> str:
    return "cuda-jit" if target.is_cuda_jit() else "unknown"


def synchronize() -> None:
    check(lib.porch_synchronize())


def plan(expression, compile: bool = False) -> dict:
    """The kernels porch would launch for `expression` (no device needed)."""
    nodes, dims, n_dims, _, _ = serialize(_expr(expression)._root)
    g = _graph(nodes, dims, n_dims)
    text = ctypes.create_string_buffer(1 << 20)
    check(lib.porch_plan(ctypes.byref(g), 1 if compile else 0, text, len(text)))
    return json.loads(text.value.decode())


def kernel_source(expression, index: int = 0) -> str:
    nodes, dims, n_dims, _, _ = serialize(_expr(expression)._root)
    g = _graph(nodes, dims, n_dims)
    length = ctypes.c_size_t()
    check(lib.porch_plan_source(ctypes.byref(g), index, None, 0, ctypes.byref(length)))
    text = ctypes.create_string_buffer(length.value + 1)
    check(lib.porch_plan_source(ctypes.byref(g), index, text, len(text), ctypes.byref(length)))
    return text.value.decode()


def jit_stats() -> dict:
    s = JitStats()
    check(lib.porch_get_jit_stats(ctypes.byref(s)))
    return {name: getattr(s, name) for name, _ in JitStats._fields_}


def release_cached_memory() -> int:
    """Returns the allocator's cached device blocks to the pool; the bytes."""
    released = ctypes.c_size_t()
    check(lib.porch_release_cached_memory(ctypes.byref(released)))
    return released.value


def reset_jit_cache() -> None:
    check(lib.porch_reset_jit_cache())


def set_disk_cache(directory) -> None:
    """Directory of the persistent code-object cache; None turns it off."""
    check(lib.porch_set_disk_cache(None if directory is None else os.fsencode(directory)))


def disk_cache_directory() -> str:
    text = ctypes.create_string_buffer(4096)
    check(lib.porch_disk_cache_directory(text, len(text)))
    return os.fsdecode(text.value)
