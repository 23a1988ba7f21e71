"""Device management and memory statistics (the reference's ``tp.mlu``
device module, tensorplay_mlu/runtime.py:20-102), over the library's C
entry points instead of TensorPlay's ``_privateuse1_*`` hooks."""

from __future__ import annotations

import contextlib
import ctypes

from . import _library
from .tensor import check

__all__ = [
    "compute_units", "current_device", "device", "device_count", "empty_cache", "is_available",
    "is_initialized", "max_memory_allocated", "max_memory_reserved", "mem_get_info",
    "memory_allocated", "memory_reserved", "memory_stats", "reset_peak_memory_stats",
    "set_device", "synchronize",
]


def is_available() -> bool:
    return bool(_library().tp_amd_is_available())


def is_initialized() -> bool:
    return True


def device_count() -> int:
    return _library().tp_mlu_device_count()


def current_device() -> int:
    index = ctypes.c_int()
    check(_library().tp_amd_current_device(ctypes.byref(index)))
    return index.value


def _index(device=None) -> int:
    if device is None:
        return current_device()
    if isinstance(device, int):
        return device
    text = str(device)
    return int(text.split(":")[1]) if ":" in text else current_device()


def set_device(device) -> None:
    check(_library().tp_amd_set_device(_index(device)))


@contextlib.contextmanager
def device(index):
    """Make ``index`` the current device inside the block."""
    previous = current_device()
    set_device(index)
    try:
        yield
    finally:
        set_device(previous)


def synchronize(device=None) -> None:
    check(_library().tp_amd_synchronize(-1 if device is None else _index(device)))


def memory_stats(device=None) -> dict[str, int]:
    out = (ctypes.c_int64 * 4)()
    _library().tp_mlu_memory_stats(_index(device), out)
    return {
        "allocated_bytes": out[0],
        "reserved_bytes": out[1],
        "peak_allocated_bytes": out[2],
        "peak_reserved_bytes": out[3],
    }


def memory_allocated(device=None) -> int:
    return memory_stats(device)["allocated_bytes"]


def memory_reserved(device=None) -> int:
    return memory_stats(device)["reserved_bytes"]


def max_memory_allocated(device=None) -> int:
    return memory_stats(device)["peak_allocated_bytes"]


def max_memory_reserved(device=None) -> int:
    return memory_stats(device)["peak_reserved_bytes"]


def reset_peak_memory_stats(device=None) -> None:
    _library().tp_mlu_reset_peak_memory_stats(_index(device))


def empty_cache() -> None:
    """Hand every idle cached block back to hipFree (after the device drains)."""
    _library().tp_mlu_empty_cache()


def mem_get_info(device=None) -> tuple[int, int]:
    """hipMemGetInfo for the device: a (free_bytes, total_bytes) pair."""
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    check(_library().tp_amd_mem_get_info(_index(device), ctypes.byref(free), ctypes.byref(total)))
    return free.value, total.value


def compute_units(device=None) -> int:
    """The device's compute units (what the kernels size their grids by)."""
    units = ctypes.c_int()
    check(_library().tp_amd_compute_units(_index(device), ctypes.byref(units)))
    return units.value
