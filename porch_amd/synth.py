"""Seeded synthetic inputs and device timing helpers.

The generator is splitmix64 (output i depends only on the seed and i):
u = (x >> 40) * 2^-24, uniform = lo + (hi - lo) * u in double, normal by
Box-Muller in double over consecutive pairs.  The C implementation lives in
libporch_amd.so (porch_synth_*), so host data is identical everywhere.
"""

from __future__ import annotations

import ctypes

import numpy as np

from ._lib import check, lib


def uniform(count: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib.porch_synth_uniform(out.ctypes.data, count, seed, lo, hi)
    return out


def normal(count: int, seed: int, mean: float, std: float) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib.porch_synth_normal(out.ctypes.data, count, seed, mean, std)
    return out


def replace(values: np.ndarray, seed: int, p: float, value: float) -> np.ndarray:
    """Replaces entries where a second splitmix64 stream draws u < p."""
    assert values.dtype == np.float32 and values.flags.c_contiguous
    lib.porch_synth_replace(values.ctypes.data, values.size, seed, p, value)
    return values


class Event:
    """A HIP event recorded on the calling thread's porch stream."""

    def __init__(self):
        handle = ctypes.c_void_p()
        check(lib.porch_event_create(ctypes.byref(handle)))
        self.handle = handle.value

    def __del__(self):
        if getattr(self, "handle", None):
            lib.porch_event_release(self.handle)
            self.handle = None

    def record(self) -> None:
        check(lib.porch_event_record(self.handle))

    def synchronize(self) -> None:
        check(lib.porch_event_synchronize(self.handle))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        check(lib.porch_event_elapsed_ms(self.handle, stop.handle, ctypes.byref(ms)))
        return float(ms.value)


def flush_caches(nbytes: int = 1 << 30) -> None:
    """Writes `nbytes` of scratch on the current stream (evicts L2 + MALL)."""
    check(lib.porch_flush_caches(nbytes))


def device_info() -> dict:
    cus = ctypes.c_int32()
    clock = ctypes.c_int32()
    arch = ctypes.create_string_buffer(256)
    check(lib.porch_device_info(ctypes.byref(cus), ctypes.byref(clock), arch, len(arch)))
    return {"compute_units": cus.value, "clock_khz": clock.value,
            "arch": arch.value.decode()}
