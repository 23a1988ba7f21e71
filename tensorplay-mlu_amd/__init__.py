"""MI355X (gfx950) device backend for TensorPlay's PrivateUse1 slot.

Mirrors the reference package ``tensorplay_mlu`` (tensorplay_mlu/__init__.py):
``load()`` loads the native library, initialises it, and -- where TensorPlay
itself is installed -- names the device and registers the device module.
The native part is ``libtp_amd.so`` next to this file, built in-tree for
gfx950 by ``__graft_entry__.build()`` (``make -C tensorplay-mlu_amd/csrc``).
There is no fallback: without the built library ``load()`` raises.

The directory name is not a Python identifier; import it with
``importlib.import_module("tensorplay-mlu_amd")``.
"""

from __future__ import annotations

import ctypes
import os
import threading

from . import _abi

__all__ = ["is_loaded", "library_path", "load", "rocm_home", "DEVICE_NAME"]

_HERE = os.path.dirname(os.path.abspath(__file__))
_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

#: Name given to the PrivateUse1 slot, so ``device="mlu"`` user code of the
#: reference runs unchanged; override with TP_AMD_DEVICE_NAME.
DEVICE_NAME = os.environ.get("TP_AMD_DEVICE_NAME", "mlu")


def rocm_home() -> str:
    """Root of the ROCm toolkit the backend builds against (the reference's
    ``neuware_home``, tensorplay_mlu/__init__.py:34-36)."""
    return os.environ.get("ROCM_PATH") or "/opt/rocm"


def library_path() -> str:
    return os.path.join(_HERE, "libtp_amd.so")


def is_loaded() -> bool:
    return _LIB is not None


def _library() -> ctypes.CDLL:
    if _LIB is None:
        load()
    assert _LIB is not None
    return _LIB


def load(verbose: bool = False) -> ctypes.CDLL:
    """Load and initialise the native backend (once); return the library."""
    global _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not os.path.isfile(path):
            raise RuntimeError(
                f"{path} is missing: build it with __graft_entry__.build() "
                "(make -C tensorplay-mlu_amd/csrc)")
        lib = _abi.bind(ctypes.CDLL(path))
        if lib.tp_mlu_init() != 0:
            raise RuntimeError("initialising the device backend failed: "
                               + lib.tp_mlu_last_error().decode())
        if verbose:
            print(f"loaded {path}: {lib.tp_mlu_device_count()} device(s)")
        _LIB = lib
        _register_with_tensorplay()
        return lib


def _register_with_tensorplay() -> None:
    """Name the slot and register the device module when TensorPlay is
    installed (tensorplay_mlu/__init__.py:95-99).  Operator registrations
    live in the TensorPlay adapter (csrc/tensorplay), which is compiled
    against TensorPlay's headers where they exist."""
    try:
        import tensorplay as tp  # noqa: F401
    except ImportError:
        return
    from . import runtime

    tp.utils.rename_privateuse1_backend(DEVICE_NAME)
    tp.utils.generate_methods_for_privateuse1_backend()
    tp._register_device_module(DEVICE_NAME, runtime)


def _autoload() -> None:
    """``tensorplay.backends`` entry point: load when the library is built."""
    if os.path.isfile(library_path()):
        load()
