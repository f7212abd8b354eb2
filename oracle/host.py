"""ctypes wrapper of the host evaluator (oracle/host_eval.cpp).

TEST INFRASTRUCTURE ONLY: evaluates a porch node table on the CPU with the
reference's semantics, for comparison against the GPU.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "liboracle.so")

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise ImportError(f"{LIBRARY_PATH} is missing: run `make -C oracle`")
        lib = ctypes.CDLL(LIBRARY_PATH)
        lib.porch_oracle_eval.restype = ctypes.c_int32
        lib.porch_oracle_eval.argtypes = [
            ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
            ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_char_p, ctypes.c_size_t,
        ]
        lib.porch_oracle_threads.restype = ctypes.c_int32
        lib.porch_oracle_threads.argtypes = []
        _lib = lib
    return _lib


def threads() -> int:
    return int(_load().porch_oracle_threads())


def evaluate_table(nodes, dims, n_dims: int, host_inputs, out_shape) -> np.ndarray:
    """Root values of a node table (as made by porch_amd.serialize)."""
    lib = _load()
    arrays = [np.ascontiguousarray(a, dtype=np.float32).reshape(-1) for a in host_inputs]
    n = len(arrays)
    pointers = (ctypes.c_void_p * max(n, 1))(*[a.ctypes.data for a in arrays])
    counts = (ctypes.c_int64 * max(n, 1))(*[a.size for a in arrays])
    count = int(np.prod(out_shape, dtype=np.int64)) if len(out_shape) else 1
    out = np.empty(count, dtype=np.float32)
    error = ctypes.create_string_buffer(1024)
    rc = lib.porch_oracle_eval(
        ctypes.cast(nodes, ctypes.c_void_p), len(nodes), ctypes.cast(dims, ctypes.c_void_p),
        n_dims, pointers, counts, n, out.ctypes.data, count, error, len(error))
    if rc != 0:
        raise RuntimeError("oracle: " + error.value.decode())
    return out.reshape(out_shape)


def evaluate(expression, host_inputs=None) -> np.ndarray:
    """Root values of a porch_amd expression.

    `host_inputs` overrides the values of the expression's input tensors (in
    serialisation order); by default their host values are used.
    """
    import porch_amd as porch

    nodes, dims, n_dims, inputs, _ = porch.serialize(expression)
    if host_inputs is None:
        host_inputs = [t._storage_values() for t in inputs]
    shape = porch.tensor_expr(expression).shape() if not isinstance(expression, porch.tensor) \
        else list(expression.shape())
    return evaluate_table(nodes, dims, n_dims, host_inputs, shape)
