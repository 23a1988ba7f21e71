"""Child process for tests/test_profiler_gpu.py: kernel-level tracing needs
TP_AMD_DEVICE_TRACE=1 before the HIP runtime starts, so the parent runs this
script in a fresh process with that set.  It runs a matrix product, a relu
and a host-to-device copy under three operation ids and prints the session's
records as one JSON line."""

import importlib
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def main() -> int:
    amd = importlib.import_module("tensorplay-mlu_amd")
    amd.load()
    ops = importlib.import_module("tensorplay-mlu_amd.ops")
    prof = importlib.import_module("tensorplay-mlu_amd.profiler")
    dev = importlib.import_module("tensorplay-mlu_amd.tensor").DeviceTensor
    print("child: loaded, tracing available:", prof.Trace.available(), prof.Trace.unavailable_reason(),
          flush=True)
    if not prof.Trace.available():
        print(json.dumps({"available": False, "reason": prof.Trace.unavailable_reason()}), flush=True)
        return 0
    host = np.random.default_rng(0).standard_normal((512, 512), dtype=np.float32)
    a = dev.from_numpy(host)
    ops.relu(ops.mm(a, a))  # load the kernels' code objects before the session
    out = ops.empty((512, 512), 0)
    trace = prof.Trace()
    with trace:
        with trace.operation(11):
            y = ops.mm(a, a)
        with trace.operation(12):
            ops.relu(y)
        with trace.operation(13):
            ops.copy_(out, host)
    print("child: session done,", len(trace.records), "records", flush=True)
    print(json.dumps({"available": True, "records": trace.records}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
