"""ctypes binding of libporch_amd.so (include/porch_amd.h).

The library is loaded from this package directory.  Importing never needs a
GPU; a missing library raises ImportError naming the build step, so no code
path can silently run without the native backend.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# PORCH_AMD_LIBRARY names another build of the same library (the
# sanitizer builds of porch_amd/Makefile) to load in its place.
LIBRARY_PATH = os.environ.get("PORCH_AMD_LIBRARY") or os.path.join(_HERE, "libporch_amd.so")

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_OUT_OF_RANGE = 2
ERR_RUNTIME = 3
ERR_COMPILATION = 4

# Node kinds (PORCH_OP_*): the reference's expr_kind order, then this
# backend's extensions (permute, batched_matmul).
OPS = (
    "input", "scalar", "add", "subtract", "multiply", "divide", "matmul",
    "slice", "reshape", "unsqueeze", "transpose", "broadcast", "concat",
    "sum", "max", "maximum", "minimum", "exp", "reciprocal", "permute", "batched_matmul",
)
OP = {name: i for i, name in enumerate(OPS)}


class Node(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_int32),
        ("lhs", ctypes.c_int32),
        ("rhs", ctypes.c_int32),
        ("input", ctypes.c_int32),
        ("scalar", ctypes.c_float),
        ("axis", ctypes.c_int32),
        ("keepdim", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64),
        ("offset", ctypes.c_int64),
    ]


class Graph(ctypes.Structure):
    _fields_ = [
        ("nodes", ctypes.POINTER(Node)),
        ("n_nodes", ctypes.c_int32),
        ("dims", ctypes.POINTER(ctypes.c_int64)),
        ("n_dims", ctypes.c_int64),
    ]


class JitStats(ctypes.Structure):
    _fields_ = [
        ("plan_hits", ctypes.c_uint64),
        ("plan_misses", ctypes.c_uint64),
        ("compiles", ctypes.c_uint64),
        ("launches", ctypes.c_uint64),
        ("codegen_ms", ctypes.c_double),
        ("compile_ms", ctypes.c_double),
        ("module_load_ms", ctypes.c_double),
        ("last_miss_ms", ctypes.c_double),
        ("last_hit_us", ctypes.c_double),
        ("disk_hits", ctypes.c_uint64),
        ("disk_ms", ctypes.c_double),
        ("device_allocs", ctypes.c_uint64),
        ("device_frees", ctypes.c_uint64),
        ("host_allocs", ctypes.c_uint64),
        ("host_frees", ctypes.c_uint64),
        ("module_loads", ctypes.c_uint64),
    ]


class PorchError(RuntimeError):
    """std::runtime_error raised by the backend (loader, driver)."""


class CompilationError(PorchError):
    """hiprtc rejected a source; `log` is the compiler output."""

    def __init__(self, log: str):
        super().__init__(log)
        self.log = log


class InvalidArgument(ValueError):
    """std::invalid_argument: shapes, axes, sizes."""


class OutOfRange(IndexError):
    """std::out_of_range: integer index out of bounds."""


_P = ctypes.c_void_p
_SIGNATURES = {
    "porch_last_error": (ctypes.c_char_p, []),
    "porch_is_available": (ctypes.c_int32, []),
    "porch_synchronize": (ctypes.c_int32, []),
    "porch_device_info": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(ctypes.c_int32),
                                           ctypes.c_char_p, ctypes.c_size_t]),
    "porch_buffer_create": (ctypes.c_int32, [ctypes.c_size_t, ctypes.POINTER(_P)]),
    "porch_buffer_release": (None, [_P]),
    "porch_buffer_size": (ctypes.c_size_t, [_P]),
    "porch_buffer_device_pointer": (ctypes.c_uint64, [_P]),
    "porch_copy_to_device": (ctypes.c_int32, [_P, _P, ctypes.c_size_t]),
    "porch_copy_to_host": (ctypes.c_int32, [_P, _P, ctypes.c_size_t]),
    "porch_compile": (ctypes.c_int32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                       ctypes.c_int32, ctypes.POINTER(_P)]),
    "porch_code_object_size": (ctypes.c_size_t, [_P]),
    "porch_code_object_data": (_P, [_P]),
    "porch_code_object_release": (None, [_P]),
    "porch_launch_fused_elementwise": (ctypes.c_int32, [_P, ctypes.c_size_t, ctypes.c_char_p,
                                                        ctypes.POINTER(_P), ctypes.c_int32,
                                                        _P, ctypes.c_size_t]),
    "porch_launch_fused_reduction": (ctypes.c_int32, [_P, ctypes.c_size_t, ctypes.c_char_p,
                                                      ctypes.POINTER(_P), ctypes.c_int32,
                                                      _P, ctypes.c_size_t]),
    "porch_infer_shape": (ctypes.c_int32, [ctypes.POINTER(Graph), ctypes.POINTER(ctypes.c_int64),
                                           ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(ctypes.c_int32)]),
    "porch_materialize": (ctypes.c_int32, [ctypes.POINTER(Graph), ctypes.POINTER(_P),
                                           ctypes.c_int32, ctypes.POINTER(_P),
                                           ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                           ctypes.POINTER(ctypes.c_int32)]),
    "porch_materialize_timed": (ctypes.c_int32, [ctypes.POINTER(Graph), ctypes.POINTER(_P),
                                                 ctypes.c_int32, ctypes.POINTER(_P),
                                                 ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                                 ctypes.POINTER(ctypes.c_int32), _P, _P]),
    "porch_plan": (ctypes.c_int32, [ctypes.POINTER(Graph), ctypes.c_int32, ctypes.c_char_p,
                                    ctypes.c_size_t]),
    "porch_plan_source": (ctypes.c_int32, [ctypes.POINTER(Graph), ctypes.c_int32,
                                           ctypes.c_char_p, ctypes.c_size_t,
                                           ctypes.POINTER(ctypes.c_size_t)]),
    "porch_get_jit_stats": (ctypes.c_int32, [ctypes.POINTER(JitStats)]),
    "porch_reset_jit_cache": (ctypes.c_int32, []),
    "porch_set_disk_cache": (ctypes.c_int32, [ctypes.c_char_p]),
    "porch_disk_cache_directory": (ctypes.c_int32, [ctypes.c_char_p, ctypes.c_size_t]),
    "porch_event_create": (ctypes.c_int32, [ctypes.POINTER(_P)]),
    "porch_event_record": (ctypes.c_int32, [_P]),
    "porch_event_synchronize": (ctypes.c_int32, [_P]),
    "porch_event_elapsed_ms": (ctypes.c_int32, [_P, _P, ctypes.POINTER(ctypes.c_float)]),
    "porch_event_release": (None, [_P]),
    "porch_flush_caches": (ctypes.c_int32, [ctypes.c_size_t]),
    "porch_release_cached_memory": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_size_t)]),
    "porch_synth_uniform": (None, [_P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_double,
                                   ctypes.c_double]),
    "porch_synth_normal": (None, [_P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_double,
                                  ctypes.c_double]),
    "porch_synth_replace": (None, [_P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_double,
                                   ctypes.c_float]),
}


# Exported by the companion library libporch_amd_noalloc.so (loaded on
# first use: it links libamdhip64, the main library does not).
NOALLOC_LIBRARY_PATH = os.path.join(_HERE, "libporch_amd_noalloc.so")
_NOALLOC_SIGNATURES = {
    "porch_materialize_noalloc": (ctypes.c_int32, [ctypes.POINTER(Graph), ctypes.POINTER(_P),
                                                   ctypes.c_int32, _P,
                                                   ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                                   ctypes.POINTER(ctypes.c_int32)]),
}
_noalloc_lib = None


def noalloc_lib() -> ctypes.CDLL:
    """libporch_amd_noalloc.so, bound on first use."""
    global _noalloc_lib
    if _noalloc_lib is None:
        if not os.path.exists(NOALLOC_LIBRARY_PATH):
            raise ImportError(f"{NOALLOC_LIBRARY_PATH} is missing: build it with `make -C porch_amd`")
        library = ctypes.CDLL(NOALLOC_LIBRARY_PATH)
        for name, (restype, argtypes) in _NOALLOC_SIGNATURES.items():
            fn = getattr(library, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _noalloc_lib = library
    return _noalloc_lib


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIBRARY_PATH):
        raise ImportError(
            f"{LIBRARY_PATH} is missing: build it with `make -C porch_amd` "
            "(or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(LIBRARY_PATH)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


lib = _load()


def check(status: int) -> None:
    """Raises the Python counterpart of the C++ exception behind `status`."""
    if status == OK:
        return
    message = lib.porch_last_error().decode("utf-8", "replace")
    if status == ERR_INVALID_ARGUMENT:
        raise InvalidArgument(message)
    if status == ERR_OUT_OF_RANGE:
        raise OutOfRange(message)
    if status == ERR_COMPILATION:
        raise CompilationError(message)
    raise PorchError(message)
