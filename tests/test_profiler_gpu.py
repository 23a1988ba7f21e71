"""Device time for the profiler (the reference's MLUProfiler.cpp:20-80 and
MLUActivity.cpp:87-258; its test is tests/test_mlu.py:381-401): pooled
event timers around operations, and kernel-level records joined to the
operation that launched them."""

import json
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_timer_reports_device_time(dev, ops, amd):
    prof = __import__("importlib").import_module("tensorplay-mlu_amd.profiler")
    a = dev.from_numpy(np.random.default_rng(0).standard_normal((2048, 2048), dtype=np.float32))
    ops.mm(a, a)
    t = prof.Timer(0)
    t.start()
    for _ in range(3):
        ops.relu(ops.mm(a, a))
    t.stop()
    ms = t.elapsed_ms()
    t.release()
    # three 2048^3 fp32 products: at least 3 * 17 GFLOP at under 160 TFLOP/s
    assert 0.3 < ms < 1000.0, ms
    # markers come back to the pool and are placed again many times
    for _ in range(500):
        t.start()
        t.stop()
        assert t.elapsed_ms() >= 0.0
        t.release()
    # an absent device gives no marker and no time
    bad = prof.Timer(99)
    bad.start()
    bad.stop()
    assert bad.elapsed_ms() is None


def test_trace_joins_kernels_to_operations():
    """In a fresh process with TP_AMD_DEVICE_TRACE=1: the product's and the
    relu's kernels carry their operations' ids, the copy is a host-to-device
    copy of the tensor's bytes, and records are ordered in time."""
    env = dict(os.environ, TP_AMD_DEVICE_TRACE="1")
    print("running tests/profiler_child.py with TP_AMD_DEVICE_TRACE=1", flush=True)
    done = subprocess.run([sys.executable, "-u", os.path.join(HERE, "profiler_child.py")], env=env,
                          capture_output=True, text=True, timeout=180)
    assert done.returncode == 0, done.stdout[-2000:] + done.stderr[-2000:]
    line = [l for l in done.stdout.splitlines() if l.startswith("{")][-1]
    result = json.loads(line)
    assert result["available"], result.get("reason")
    records = result["records"]
    by_op = {}
    for r in records:
        by_op.setdefault(r["external_id"], []).append(r)
    kernels_mm = [r for r in by_op.get(11, []) if r["kind"] == "k"]
    kernels_relu = [r for r in by_op.get(12, []) if r["kind"] == "k"]
    assert kernels_mm and any("gemm" in r["name"] for r in kernels_mm), by_op.get(11)
    assert kernels_relu and all("gemm" not in r["name"] for r in kernels_relu), by_op.get(12)
    copies = [r for r in by_op.get(13, []) if r["kind"] == "m"]
    assert copies and copies[0]["copy_kind"] == 1 and copies[0]["name"] == "Memcpy HtoD", by_op.get(13)
    assert sum(r["bytes"] for r in copies) == 512 * 512 * 4
    for r in records:
        assert r["end_ns"] >= r["start_ns"] > 0 and r["device"] == 0
    # the product ran before the relu that consumed it
    assert max(r["end_ns"] for r in kernels_mm) <= min(r["start_ns"] for r in kernels_relu) + 1000
