"""Device time for a profiler (the reference's profiler hooks,
tensorplay_mlu/csrc/MLUProfiler.cpp:20-80 and MLUActivity.cpp:87-258, over
the library's ``tp_amd_timer_*`` and ``tp_amd_activity_*`` entries).

* ``Timer``: pooled HIP events on the device's stream around an operation,
  the per-operation device time TensorPlay's profiler reports.
* ``Trace``: the kernels and copies the GPU ran during a session, each with
  the id pushed around the operation that launched it.  It needs the
  process to start with ``TP_AMD_DEVICE_TRACE=1``; otherwise ``start``
  raises with the reason and only ``Timer`` works.

    with Trace() as trace:
        with trace.operation(7):
            ops.mm(a, a)
    [r for r in trace.records if r["external_id"] == 7]
"""

from __future__ import annotations

import contextlib
import ctypes

from . import _abi, _library

__all__ = ["Timer", "Trace"]


def _error(default: str) -> RuntimeError:
    message = _library().tp_mlu_last_error()
    return RuntimeError((message.decode("utf-8", "replace") if message else "") or default)


class Timer:
    """A start/end marker pair on one device's stream."""

    def __init__(self, device: int = 0) -> None:
        self.device = device
        self._start = self._end = None

    @staticmethod
    def _record(device: int):
        marker = ctypes.c_void_p()
        if _library().tp_amd_timer_record(device, ctypes.byref(marker)) != 0:
            raise _error("placing a timer failed")
        return marker.value

    def start(self) -> None:
        self._start = self._record(self.device)

    def stop(self) -> None:
        self._end = self._record(self.device)

    def elapsed_ms(self) -> float:
        """Waits for the end marker; None when a marker could not be placed."""
        if not self._start or not self._end:
            return None
        ms = ctypes.c_float()
        if _library().tp_amd_timer_elapsed_ms(self._start, self._end, ctypes.byref(ms)) != 0:
            raise _error("reading a timer failed")
        return ms.value

    def release(self) -> None:
        for marker in (self._start, self._end):
            _library().tp_amd_timer_release(marker)
        self._start = self._end = None


class Trace:
    """One kernel-level tracing session."""

    def __init__(self) -> None:
        self.records: list[dict] = []

    @staticmethod
    def available() -> bool:
        return not _library().tp_amd_activity_error()

    @staticmethod
    def unavailable_reason() -> str:
        return _library().tp_amd_activity_error().decode("utf-8", "replace")

    def start(self) -> None:
        if _library().tp_amd_activity_start() != 0:
            raise _error("starting the trace failed")

    def stop(self) -> list[dict]:
        records = ctypes.POINTER(_abi.Activity)()
        count = ctypes.c_size_t()
        if _library().tp_amd_activity_stop(ctypes.byref(records), ctypes.byref(count)) != 0:
            raise _error("stopping the trace failed")
        self.records = []
        for i in range(count.value):
            r = records[i]
            self.records.append({
                "name": r.name.decode("utf-8", "replace") if r.name else "",
                "kind": r.kind.decode(), "copy_kind": r.copy_kind,
                "start_ns": r.start_ns, "end_ns": r.end_ns,
                "external_id": None if r.external_id == _abi.NO_EXTERNAL else r.external_id,
                "correlation": r.correlation, "device": r.device, "stream": r.stream,
                "bytes": r.bytes})
        return self.records

    @contextlib.contextmanager
    def operation(self, external_id: int):
        """Launches inside carry ``external_id``."""
        if _library().tp_amd_activity_push_external(external_id) != 0:
            raise _error("pushing the operation id failed")
        try:
            yield
        finally:
            _library().tp_amd_activity_pop_external()

    def __enter__(self) -> "Trace":
        self.start()
        return self

    def __exit__(self, *exc) -> None:
        self.stop()
