#!/usr/bin/env python3
"""Benchmark of the TensorPlay PrivateUse1 hot path on one MI355X.

Headline workload ("broadcast elementwise"): one
step runs the config-2 operator set on a [8192, 8192] tensor in float32 and
in bfloat16 storage -- add/sub/mul/div against a row-broadcast [8192] and a
column-broadcast [8192, 1] operand, their in-place forms, the scalar forms,
exp, log(|a|+1e-3), sqrt(|a|), pow(a, 2), relu, gelu, sigmoid, and the relu /
gelu / sigmoid backward kernels -- through the library's operator C-ABI, with
every input already resident in HBM.  ``value`` is the algorithmic bytes of
one step (2 N^2 e per forward op, 3 N^2 e per backward op; the broadcast
operand is not counted) times the steps, divided by the wall time of the
timed steps.

Also reported on the same line:
* ``roofline``: the dominant kernel (the broadcasting binary kernel, float32
  add against a row-broadcast operand), its average launch duration from
  HIP events recorded on the library's own stream, against 8 TB/s, measured
  cold: four inputs and four outputs rotated, 2 GiB, beyond the 256 MB
  Infinity Cache; ``roofline_warm`` is the same kernel on one input and
  output reused every launch;
* ``suite``: per-kernel throughput of configs 2-5, of thin (decode-step)
  products and of the neural-network layers (GB/s or TFLOP/s and the
  fraction of the matching MI355X peak), each
  from HIP events, and the reference README's benchmark rows beside the
  MLU590 times it publishes (``readme_rows``);
* ``cpu_baseline``: the repository's C oracle (a CPU port of the same
  operators, float64 arithmetic, OpenMP) timed on this host on a bounded
  sample of the same workload;
* ``suite_cpu``: the same oracle on bounded samples of the suite's other
  sections (config 3, config 4, config 5b, layer norm), each in its
  section's unit, so every suite figure has a CPU figure beside it.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-suite] [--no-cpu]
  python bench.py --profile {traffic,traffic_cold,gemm,gemm32,linear,vs_torch,vs_torch_thin,vs_torch_batch,
                             bmm,reduce,reduce_all,softmax,nn,mlp,odd,thin}   # launch sequences for rocprofv3
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
# HBM bytes per launch of the dominant kernel, measured with rocprofv3's
# FETCH_SIZE and WRITE_SIZE counters (one pass each over
# ``bench.py --profile traffic``), each scaled by what the same counter reads
# for a copy kernel of known size; recorded in
# profiles/config2_binary2d_hbm_traffic.md.
DOMINANT_TRAFFIC_BYTES = 536829485
# The same for the cold rotation (``bench.py --profile traffic_cold``),
# recorded in the same file.
COLD_TRAFFIC_BYTES = 536765611
MFMA_PEAK_TFLOPS = {"bf16": 2516.6, "fp16": 2516.6, "fp32": 157.3}
METRIC = "GEMM TFLOP/s + %MFMA peak; reduce/softmax/eltwise GB/s + %HBM peak"
N = 8192

amd = importlib.import_module("tensorplay-mlu_amd")
F32, F16, BF16 = 0, 1, 2
ESIZE = {F32: 4, BF16: 2, F16: 2}
NAME = {F32: "fp32", BF16: "bf16", F16: "fp16"}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Events:
    """A pair of HIP events on the library's stream."""

    def __init__(self, lib):
        import ctypes as C
        self.C, self.lib = C, lib
        self.start, self.stop = C.c_void_p(), C.c_void_p()
        assert lib.tp_amd_event_create(C.byref(self.start)) == 0
        assert lib.tp_amd_event_create(C.byref(self.stop)) == 0

    def time_ms(self, fn, reps: int) -> float:
        """Average milliseconds of ``fn`` over ``reps`` back-to-back calls."""
        C, lib = self.C, self.lib
        assert lib.tp_amd_event_record(self.start, 0) == 0
        for _ in range(reps):
            fn()
        assert lib.tp_amd_event_record(self.stop, 0) == 0
        ms = C.c_float()
        assert lib.tp_amd_event_elapsed_ms(self.start, self.stop, C.byref(ms)) == 0
        return ms.value / reps


def build_config2(ops, dev, dtype):
    """Resident inputs of config 2 in ``dtype`` (generated in float32 on the
    host, converted on the device)."""
    g = np.random.default_rng(0)
    a32 = g.standard_normal((N, N), dtype=np.float32)
    row32 = g.uniform(0.5, 2.0, N).astype(np.float32)
    col32 = g.uniform(0.5, 2.0, (N, 1)).astype(np.float32)
    g32 = g.standard_normal((N, N), dtype=np.float32)

    def put(x):
        d = dev.from_numpy(x)
        return d if dtype == F32 else ops.to(d, dtype)

    a, row, col, grad = put(a32), put(row32), put(col32), put(g32)
    absa = ops.abs(a)
    loga = ops.add_scalar(absa, 1e-3)
    work = ops.clone(a)
    y = ops.sigmoid(a)
    return dict(a=a, row=row, col=col, grad=grad, absa=absa, loga=loga, work=work, y=y)


def config2_ops(ops, t):
    """(name, callable, bytes-per-element factor) for one pass of config 2."""
    a, row, col, grad, work = t["a"], t["row"], t["col"], t["grad"], t["work"]
    fwd, bwd = 2, 3
    return [
        ("add_row", lambda: ops.add(a, row), fwd), ("sub_row", lambda: ops.sub(a, row), fwd),
        ("mul_row", lambda: ops.mul(a, row), fwd), ("div_row", lambda: ops.div(a, row), fwd),
        ("add_col", lambda: ops.add(a, col), fwd), ("sub_col", lambda: ops.sub(a, col), fwd),
        ("mul_col", lambda: ops.mul(a, col), fwd), ("div_col", lambda: ops.div(a, col), fwd),
        ("add_", lambda: ops.add_(work, row), fwd), ("sub_", lambda: ops.sub_(work, row), fwd),
        ("mul_", lambda: ops.mul_(work, row), fwd), ("div_", lambda: ops.div_(work, row), fwd),
        ("add_scalar", lambda: ops.add_scalar(a, 2.0), fwd),
        ("sub_scalar", lambda: ops.sub_scalar(a, 2.0), fwd),
        ("mul_scalar", lambda: ops.mul_scalar(a, 3.0), fwd),
        ("div_scalar", lambda: ops.div_scalar(a, 4.0), fwd),
        ("exp", lambda: ops.exp(a), fwd), ("log", lambda: ops.log(t["loga"]), fwd),
        ("sqrt", lambda: ops.sqrt(t["absa"]), fwd), ("pow2", lambda: ops.pow_scalar(a, 2), fwd),
        ("relu", lambda: ops.relu(a), fwd), ("gelu", lambda: ops.gelu(a), fwd),
        ("sigmoid", lambda: ops.sigmoid(a), fwd),
        ("relu_backward", lambda: ops.threshold_backward(grad, a, 0), bwd),
        ("gelu_backward", lambda: ops.gelu_backward(grad, a), bwd),
        ("sigmoid_backward", lambda: ops.sigmoid_backward(grad, t["y"]), bwd),
    ]


def dominant_kernel(lib, ev, t, reps=50):
    """Average launch duration of the broadcasting binary kernel (fp32 add
    with a row-broadcast operand), called through the kernel-level C-ABI."""
    import ctypes as C
    a, row, out = t["a"], t["row"], t["out"]
    sizes = (C.c_int64 * 2)(N, N)
    sa = (C.c_int64 * 2)(N, 1)
    sb = (C.c_int64 * 2)(0, 1)

    def launch():
        st = lib.tp_amd_launch_binary(0, 0, F32, 2, sizes, a.data_ptr, sa, row.data_ptr, sb,
                                      out.data_ptr, sa, 1.0)
        assert st == 0

    for _ in range(5):
        launch()
    ms = ev.time_ms(launch, reps)
    algo = 2 * N * N * 4
    achieved = algo / (ms * 1e-3) / 1e9
    return {"kernel": "binary2d_kernel<float, full, row-broadcast> (add)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "cache": "warm: one input and one output reused on every launch (the Infinity Cache "
                     "keeps part of the 256 MiB input)",
            "traffic": DOMINANT_TRAFFIC_BYTES,
            "avg_us": round(ms * 1e3, 2), "algorithmic_bytes_per_launch": algo}


COLD_PAIRS = 4  # input/output pairs the cold measurement rotates over


def dominant_kernel_cold(lib, ops, ev, t, rounds=12):
    """The dominant kernel with its working set beyond the 256 MB Infinity
    Cache: COLD_PAIRS distinct [8192, 8192] float32 inputs and outputs (2 GiB
    in all), launched round-robin, so every launch reads an input and
    writes an output last touched COLD_PAIRS - 1 launches (1.5 GiB of other
    traffic) earlier.  Average launch duration over ``rounds`` rotations,
    from HIP events on the library's stream."""
    import ctypes as C
    a, row = t["a"], t["row"]
    inputs = [a] + [ops.add_scalar(a, float(k)) for k in range(1, COLD_PAIRS)]
    outputs = [ops.empty((N, N), F32) for _ in range(COLD_PAIRS)]
    sizes = (C.c_int64 * 2)(N, N)
    sa = (C.c_int64 * 2)(N, 1)
    sb = (C.c_int64 * 2)(0, 1)

    def rotation():
        for x, y in zip(inputs, outputs):
            st = lib.tp_amd_launch_binary(0, 0, F32, 2, sizes, x.data_ptr, sa, row.data_ptr, sb, y.data_ptr, sa,
                                          1.0)
            assert st == 0

    for _ in range(3):
        rotation()
    ms = ev.time_ms(rotation, rounds) / COLD_PAIRS
    algo = 2 * N * N * 4
    achieved = algo / (ms * 1e-3) / 1e9
    del inputs, outputs
    return {"kernel": "binary2d_kernel<float, full, row-broadcast> (add)",
            "cache": f"cold: {COLD_PAIRS} inputs and {COLD_PAIRS} outputs of 256 MiB rotated "
                     f"({COLD_PAIRS * 512} MiB working set, 256 MB Infinity Cache)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": COLD_TRAFFIC_BYTES,
            "avg_us": round(ms * 1e3, 2), "algorithmic_bytes_per_launch": algo}


def suite_config2(ops, ev, tensors):
    out = {}
    for dtype, t in tensors.items():
        for name, fn, factor in config2_ops(ops, t):
            for _ in range(2):
                fn()
            ms = ev.time_ms(fn, 10)
            gbs = factor * N * N * ESIZE[dtype] / (ms * 1e-3) / 1e9
            out[f"{name}_{NAME[dtype]}"] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1),
                                            "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)}
    return out


def suite_config3(ops, dev, ev):
    out = {}
    for shape, std in (((32768, 4096), 2.0), ((4096, 32000), 4.0)):
        x32 = np.random.default_rng(0).standard_normal(shape, dtype=np.float32) * np.float32(std)
        g32 = np.random.default_rng(1).standard_normal(shape, dtype=np.float32)
        for dtype in (F32, BF16):
            x, g = dev.from_numpy(x32), dev.from_numpy(g32)
            if dtype != F32:
                x, g = ops.to(x, dtype), ops.to(g, dtype)
            y = ops.softmax(x, -1)
            ly = ops.log_softmax(x, -1)
            n = shape[0] * shape[1] * ESIZE[dtype]
            tag = f"{shape[0]}x{shape[1]}_{NAME[dtype]}"
            cases = []
            for dim in (-1, 0):
                outb = (shape[0] if dim == -1 else shape[1]) * ESIZE[dtype]
                cases += [(f"sum_dim{dim}", lambda dim=dim: ops.sum_dim(x, dim), n + outb),
                          (f"mean_dim{dim}", lambda dim=dim: ops.mean_dim(x, dim), n + outb),
                          (f"amax_dim{dim}", lambda dim=dim: ops.amax(x, dim), n + outb),
                          (f"amin_dim{dim}", lambda dim=dim: ops.amin(x, dim), n + outb)]
            cases += [("softmax", lambda: ops.softmax(x, -1), 2 * n),
                      ("log_softmax", lambda: ops.log_softmax(x, -1), 2 * n),
                      ("softmax_backward", lambda: ops._softmax_backward_data(g, y, -1, dtype), 3 * n),
                      ("log_softmax_backward",
                       lambda: ops._log_softmax_backward_data(g, ly, -1, dtype), 3 * n)]
            for name, fn, nbytes in cases:
                for _ in range(2):
                    fn()
                ms = ev.time_ms(fn, 10)
                gbs = nbytes / (ms * 1e-3) / 1e9
                out[f"{name}_{tag}"] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1),
                                        "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)}
            del x, g, y, ly
    return out


def suite_gemm(ops, dev, ev):
    """Configs 4 and 5a: matrix products (TFLOP/s against the dtype's dense
    MFMA peak; bmm also against HBM)."""
    out = {}
    g = np.random.default_rng(0)

    def put(shape, dtype, scale):
        d = dev.from_numpy(g.standard_normal(shape, dtype=np.float32) * np.float32(scale))
        return d if dtype == F32 else ops.to(d, dtype)

    def record(name, fn, flops, dtype, nbytes=None):
        # five untimed calls: the shader clock is still settling over the
        # first few large products of a run
        for _ in range(5):
            fn()
        ms = ev.time_ms(fn, 5)
        tf = flops / (ms * 1e-3) / 1e12
        peak = MFMA_PEAK_TFLOPS[NAME[dtype]]
        entry = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1), "mfma_frac": round(tf / peak, 4)}
        if nbytes is not None:
            gbs = nbytes / (ms * 1e-3) / 1e9
            entry.update({"GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)})
        out[f"{name}_{NAME[dtype]}"] = entry

    for dtype in (BF16, F32):
        K = 4096
        a, b = put((K, K), dtype, K ** -0.25), put((K, K), dtype, K ** -0.25)
        bias = put((K,), dtype, 1.0)
        at = ops.contiguous(a.t())
        # the clock settles over the first products of a dtype (float32
        # 4096^3 runs ~15 % slower for its first ten or so): ten untimed
        # products before the dtype's first row
        for _ in range(10):
            ops.mm(a, b)
        record("mm_4096", lambda: ops.mm(a, b), 2 * K ** 3, dtype)
        record("addmm_4096", lambda: ops.addmm(bias, a, b), 2 * K ** 3, dtype)
        record("mm_4096_At", lambda: ops.mm(at.t(), b), 2 * K ** 3, dtype)
        del a, b, at
        x, w = put((8192, 4096), dtype, 4096 ** -0.25), put((11008, 4096), dtype, 4096 ** -0.25)
        lb = put((11008,), dtype, 1.0)
        record("linear_8192x4096x11008", lambda: ops.linear(x, w, lb), 2 * 8192 * 11008 * 4096, dtype)
        del x, w
    a, b = put((64, 512, 128), BF16, 128 ** -0.25), put((64, 128, 512), BF16, 128 ** -0.25)
    record("bmm_64x512x128x512", lambda: ops.bmm(a, b), 2 * 64 * 512 * 512 * 128, BF16,
           nbytes=(64 * 512 * 128 * 2 + 64 * 512 * 512) * 2)
    return out


def thin_cases(ops, dev, rows=(1, 16)):
    """Thin products of a decode step, each with its wide operand in several
    copies (rotated, so that the copies together exceed the 256 MB Infinity
    Cache): (name, launch, bytes moved a launch, copies).  ``rows``: the
    Linear layer's batch rows (64 rows of a 16-bit product take the split
    over K, not the thin kernel)."""
    g = np.random.default_rng(0)

    def put(shape, dtype, scale=1.0):
        d = dev.from_numpy(g.standard_normal(shape, dtype=np.float32) * np.float32(scale))
        return d if dtype == F32 else ops.to(d, dtype)

    def copies(w, n):
        return [w] + [ops.add_scalar(w, 0.001 * k) for k in range(1, n)]

    cases = []
    for dtype in (BF16, F32):
        e = ESIZE[dtype]
        w = copies(put((11008, 4096), dtype, 4096 ** -0.5), 4)
        for m in rows:
            x = put((m, 4096), dtype)
            cases.append((f"linear_{m}x4096x11008_{NAME[dtype]}", x, w, lambda x, w: ops.linear(x, w),
                          (11008 * 4096 + m * 4096 + m * 11008) * e))
        del w
    head = copies(put((50257, 4096), BF16, 4096 ** -0.5), 2)
    x = put((1, 4096), BF16)
    cases.append(("lm_head_logits_1x4096x50257_bf16", x, head, lambda x, w: ops.linear(x, w),
                  (50257 * 4096 + 4096 + 50257) * 2))
    dy = put((1, 50257), BF16)
    cases.append(("lm_head_dx_1x50257x4096_bf16", dy, head, lambda x, w: ops.mm(x, w),
                  (50257 * 4096 + 50257 + 4096) * 2))
    return cases


def suite_thin(ops, dev, ev):
    """Thin products (decode-step shapes): GB/s against HBM, the wide
    operand rotated over copies beyond the Infinity Cache."""
    out = {}
    for name, x, ws, fn, nbytes in thin_cases(ops, dev, rows=(1, 16, 64)):
        k = [0]

        def call(x=x, ws=ws, fn=fn):
            fn(x, ws[k[0] % len(ws)])
            k[0] += 1
        for _ in range(len(ws)):
            call()
        reps = 10 * len(ws)
        ms = ev.time_ms(call, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3),
                     "copies": len(ws)}
    return out


def suite_config5b(ops, dev, ev):
    """Config 5b: the fp32 MLP training step at full size (batch 8192, four
    Linear(4096, 4096) + ReLU layers, Linear(4096, 1000), log_softmax, NLL via
    mul + sum, backward, SGD), every operator through the C-ABI; TFLOP/s of
    the step's GEMM work against the fp32 MFMA peak."""
    wl = importlib.import_module("tensorplay-mlu_amd.workloads")
    batch, width, layers, classes = 8192, 4096, 4, 1000
    ws, bs = wl.MLP.host_init(width, layers, width, classes, seed=0)
    model = wl.MLP.to_device(ws, bs)
    del ws, bs
    g = np.random.default_rng(100)
    x = dev.from_numpy(g.standard_normal((batch, width), dtype=np.float32))
    labels = np.random.default_rng(101).integers(0, classes, batch)
    onehot = np.zeros((batch, classes), np.float32)
    onehot[np.arange(batch), labels] = 1.0
    onehot = dev.from_numpy(onehot)

    def step():
        wl.mlp_step(ops, model, x, onehot, 1e-3)

    step()
    ms = ev.time_ms(step, 3)
    flops = wl.mlp_step_flops(batch, width, layers, classes)
    tf = flops / (ms * 1e-3) / 1e12
    return {"mlp_step_fp32": {"ms": round(ms, 2), "TFLOP/s": round(tf, 1),
                              "mfma_frac": round(tf / MFMA_PEAK_TFLOPS["fp32"], 4),
                              "flops_per_step": flops}}


# The reference README's table (README.md:217-229): tensorplay-mlu on a
# Cambricon MLU590, median of 50 timed iterations, fp32 matmuls in TF32.
README_MS = {"mm_4096_fp32": 1.71, "mm_1024_fp32": 0.07, "add_4096sq_fp32": 0.38,
             "relu_4096sq_fp32": 0.14, "gelu_4096sq_fp32": 0.20, "softmax_4096sq_fp32": 0.20,
             "sum_all_4096sq_fp32": 0.08, "bmm_32x512x64x512_fp32": 0.07, "h2d_64MiB": 5.03,
             "d2h_64MiB": 5.6, "mlp_train_step_fp32": 0.50}


def suite_readme(ops, dev, ev, lib):
    """The reference README's benchmark rows on this GPU, measured the way the
    README states (median of 50 timed iterations after 5 untimed), beside the
    MLU590 time it publishes.  Device operators are timed with HIP events
    around each call; the 64 MiB host copies (pageable host memory, as a
    TensorPlay CPU tensor's) with the wall clock around the synchronous copy.
    fp32 matmuls here are full float32 (gfx950 has no TF32 matrix
    instruction); the README's ran TF32.  The MLP step is the README
    chart's "b256, 1024 -> 4096": Linear(1024, 4096) + ReLU, Linear(4096,
    1024), log_softmax, NLL through mul + sum with a one-hot, backward and SGD
    (the reference's benchmark script is not in its repository, so the loss
    is this build's choice), timed eagerly and as one recorded-graph replay."""
    import ctypes as C
    graph_mod = importlib.import_module("tensorplay-mlu_amd.graph")
    wl = importlib.import_module("tensorplay-mlu_amd.workloads")
    g = np.random.default_rng(0)
    out = {}

    def med(fn, iters=50):
        for _ in range(5):
            fn()
        return float(np.median([ev.time_ms(fn, 1) for _ in range(iters)]))

    def wall_med(fn, iters=50):
        for _ in range(5):
            fn()
        ts = []
        for _ in range(iters):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e3)
        return float(np.median(ts))

    def record(name, ms, **extra):
        ref = README_MS[name.split("@")[0]]
        out[name] = {"ms": round(ms, 4), "reference_mlu590_ms": ref, "ratio": round(ms / ref, 4), **extra}

    put = lambda shape: dev.from_numpy(g.standard_normal(shape, dtype=np.float32))
    for n in (4096, 1024):
        a, b = put((n, n)), put((n, n))
        record(f"mm_{n}_fp32", med(lambda: ops.mm(a, b)))
    x, y = put((4096, 4096)), put((4096, 4096))
    record("add_4096sq_fp32", med(lambda: ops.add(x, y)))
    record("relu_4096sq_fp32", med(lambda: ops.relu(x)))
    record("gelu_4096sq_fp32", med(lambda: ops.gelu(x)))
    record("softmax_4096sq_fp32", med(lambda: ops.softmax(x, -1)))
    record("sum_all_4096sq_fp32", med(lambda: ops.sum(x)))
    a3, b3 = put((32, 512, 64)), put((32, 64, 512))
    record("bmm_32x512x64x512_fp32", med(lambda: ops.bmm(a3, b3)))
    del a, b, x, y, a3, b3
    nbytes = 64 << 20
    host = np.ones(nbytes // 4, np.float32)
    back = np.empty_like(host)
    d = ops.empty((nbytes // 4,), F32)
    hp, bp = host.ctypes.data_as(C.c_void_p), back.ctypes.data_as(C.c_void_p)
    record("h2d_64MiB", wall_med(lambda: lib.tp_amd_copy_bytes(d.data_ptr, 0, hp, -1, nbytes)))
    record("d2h_64MiB", wall_med(lambda: lib.tp_amd_copy_bytes(bp, -1, d.data_ptr, 0, nbytes)))
    assert np.array_equal(host, back), "64 MiB round trip"
    del d
    ws, bs = wl.MLP.host_init(4096, 1, 1024, 1024, seed=0)
    model = wl.MLP.to_device(ws, bs)
    xb = put((256, 1024))
    onehot = np.zeros((256, 1024), np.float32)
    onehot[np.arange(256), g.integers(0, 1024, 256)] = 1.0
    oh = dev.from_numpy(onehot)
    step = lambda: wl.mlp_step(ops, model, xb, oh, 1e-3)
    record("mlp_train_step_fp32", med(step), mode="eager")
    graph = graph_mod.Graph()
    graph.capture(step)
    record("mlp_train_step_fp32@graph", med(graph.replay), mode="one recorded-graph replay")
    graph.reset()
    out["chart_rows"] = suite_chart(ops, dev, ev, med, put, graph_mod)
    return out


def suite_chart(ops, dev, ev, med, put, graph_mod):
    """The rows of the reference's benchmark chart (docs/images/
    benchmark-ratio.png) that carry only a ratio against torch_mlu and no
    time: float16 matmuls and memory-bound operators on 4096^2 (the README's
    shape for its float32 rows), the float32 -> float16 cast, and the
    launch-overhead row, add on 16 x 16.  Each gets this GPU's time and its
    rate against the roofline.  The 16 x 16 add is timed three ways: HIP
    events around one call, the host's wall time per call over 1000
    back-to-back asynchronous calls (what an eager loop pays to launch), and
    the same for replays of a recorded graph of that one add."""
    out = {}
    n = 4096
    e = 2

    def rate(name, ms, nbytes=None, flops=None):
        row = {"ms": round(ms, 4)}
        if nbytes is not None:
            gbs = nbytes / (ms * 1e-3) / 1e9
            row.update({"GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)})
        if flops is not None:
            tf = flops / (ms * 1e-3) / 1e12
            row.update({"TFLOP/s": round(tf, 1), "mfma_frac": round(tf / MFMA_PEAK_TFLOPS["fp16"], 4)})
        out[name] = row

    half = lambda shape: ops.to(put(shape), F16)
    for k in (1024, 4096):
        a, b, at = half((k, k)), half((k, k)), half((k, k))
        rate(f"mm_{k}_fp16", med(lambda: ops.mm(a, b)), flops=2 * k ** 3)
        rate(f"mm_tn_{k}_fp16", med(lambda: ops.mm(at.t(), b)), flops=2 * k ** 3)
        del a, b, at
    x, y, row = half((n, n)), half((n, n)), half((n,))
    nn = n * n
    rate("add_4096sq_fp16", med(lambda: ops.add(x, y)), 3 * nn * e)
    z = ops.add(x, y)
    rate("add__4096sq_fp16", med(lambda: ops.add_(z, y)), 3 * nn * e)
    rate("add_bcast_4096sq_fp16", med(lambda: ops.add(x, row)), 2 * nn * e)
    rate("relu_4096sq_fp16", med(lambda: ops.relu(x)), 2 * nn * e)
    rate("gelu_4096sq_fp16", med(lambda: ops.gelu(x)), 2 * nn * e)
    rate("exp_4096sq_fp16", med(lambda: ops.exp(x)), 2 * nn * e)
    rate("softmax_4096sq_fp16", med(lambda: ops.softmax(x, -1)), 2 * nn * e)
    rate("sum_dim_4096sq_fp16", med(lambda: ops.sum_dim(x, -1)), nn * e)
    rate("sum_all_4096sq_fp16", med(lambda: ops.sum(x)), nn * e)
    rate("mul_scalar_4096sq_fp16", med(lambda: ops.mul_scalar(x, 2.5)), 2 * nn * e)
    x32 = put((n, n))
    rate("cast_fp32_to_fp16_4096sq", med(lambda: ops.to(x32, F16)), nn * 6)
    del x, y, z, row, x32
    a, b = put((16, 16)), put((16, 16))
    out["add_16x16_fp32"] = {"ms": round(med(lambda: ops.add(a, b)), 4), "timing": "HIP events"}
    calls = 1000

    def per_call_us(fn, n=calls):
        for _ in range(20):
            fn()
        ev.lib.tp_amd_synchronize(0)
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        ev.lib.tp_amd_synchronize(0)
        return (time.perf_counter() - t0) / n * 1e6

    def eager_and_replay(fn, n=calls):
        eager = per_call_us(fn, n)
        graph = graph_mod.Graph()
        graph.capture(fn)
        replay = per_call_us(graph.replay, n)
        graph.reset()
        return eager, replay

    eager_us, replay_us = eager_and_replay(lambda: ops.add(a, b))
    out["add_16x16_fp32@wall"] = {"eager_us_per_call": round(eager_us, 2),
                                 "graph_replay_us_per_call": round(replay_us, 2),
                                 "replay_over_eager": round(replay_us / eager_us, 3),
                                 "timing": f"host wall time over {calls} back-to-back calls"}

    # One graph of 100 adds replayed, against the same 100 adds launched
    # eagerly: what a recorded graph saves per kernel once it holds many.
    def adds():
        for _ in range(100):
            ops.add(a, b)

    eager_us, replay_us = eager_and_replay(adds, 100)
    out["add_16x16_fp32_x100@wall"] = {"eager_us_per_add": round(eager_us / 100, 2),
                                      "graph_replay_us_per_add": round(replay_us / 100, 2),
                                      "replay_over_eager": round(replay_us / eager_us, 3),
                                      "timing": "host wall time over 100 back-to-back runs of 100 adds"}
    # Config 1, the README quickstart step on [256, 256]: mm, relu, softmax,
    # sum and their backward, eager against one recorded-graph replay.
    wl = importlib.import_module("tensorplay-mlu_amd.workloads")
    x1, w1 = put((256, 256)), put((256, 256))
    eager_us, replay_us = eager_and_replay(lambda: wl.quickstart_step(ops, x1, w1), 200)
    out["config1_quickstart_step@wall"] = {"eager_us": round(eager_us, 2),
                                          "graph_replay_us": round(replay_us, 2),
                                          "replay_over_eager": round(replay_us / eager_us, 3),
                                          "timing": "host wall time over 200 back-to-back steps"}
    return out


def suite_nn(ops, dev, ev):
    """The neural-network layers next to the training step (the reference's
    NNKernels.cpp): layer norm forward and backward over [8192, 4096] rows,
    dropout p = 0.1 and its backward on [8192, 4096], an embedding lookup of
    8192 indices into a [32000, 4096] table and its dense gradient, nll_loss
    over [8192, 32000] log-probabilities and its backward.  GB/s of
    algorithmic bytes (every input element read once, every output element
    written once; the backward of the embedding writes the whole table)
    against 8 TB/s."""
    out = {}
    g = np.random.default_rng(0)
    rows, D, V, C = 8192, 4096, 32000, 32000

    def put(shape, dtype, scale=1.0):
        d = dev.from_numpy(g.standard_normal(shape, dtype=np.float32) * np.float32(scale))
        return d if dtype == F32 else ops.to(d, dtype)

    def record(name, fn, nbytes, reps=10):
        for _ in range(2):
            fn()
        ms = ev.time_ms(fn, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)}

    idx = dev.from_numpy(g.integers(0, V, size=rows).astype(np.int64))
    tgt = dev.from_numpy(g.integers(0, C, size=rows).astype(np.int64))
    for dtype in (F32, BF16):
        e, tag = ESIZE[dtype], NAME[dtype]
        n = rows * D
        x, dy = put((rows, D), dtype, 2.0), put((rows, D), dtype)
        w, b = put((D,), dtype), put((D,), dtype)
        _, mean, rstd = ops.native_layer_norm(x, (D,), w, b)
        record(f"layer_norm_fwd_{rows}x{D}_{tag}", lambda: ops.native_layer_norm(x, (D,), w, b),
               2 * n * e + 8 * rows)
        record(f"layer_norm_bwd_{rows}x{D}_{tag}",
               lambda: ops.native_layer_norm_backward(dy, x, (D,), mean, rstd, w, b), 3 * n * e + 8 * rows)
        _, mask = ops.native_dropout(x, 0.1, True, 1)
        record(f"dropout_{rows}x{D}_{tag}", lambda: ops.native_dropout(x, 0.1, True, 7), n * (2 * e + 1))
        record(f"dropout_bwd_{rows}x{D}_{tag}", lambda: ops.native_dropout_backward(dy, mask, 1 / 0.9),
               n * (2 * e + 1))
        del x, mean, rstd, mask
        table = put((V, D), dtype)
        record(f"embedding_{rows}_from_{V}x{D}_{tag}", lambda: ops.embedding(table, idx),
               2 * n * e + 8 * rows)
        del table
        record(f"embedding_bwd_{rows}_to_{V}x{D}_{tag}",
               lambda: ops.embedding_dense_backward(dy, idx, V), n * e + V * D * e, reps=5)
        del dy, w, b
        logp = put((rows, C), dtype)
        y, total = ops.nll_loss(logp, tgt, None, 1)
        one = ops.to(dev.from_numpy(np.array(1.0, np.float32)), dtype)
        record(f"nll_loss_{rows}x{C}_{tag}", lambda: ops.nll_loss(logp, tgt, None, 1), rows * (e + 8))
        record(f"nll_loss_bwd_{rows}x{C}_{tag}",
               lambda: ops.nll_loss_backward(one, logp, tgt, None, 1, -100, total), rows * C * e + rows * 8)
        del logp, y, total
    return out


def cpu_baseline(min_seconds: float = 10.0, max_passes: int = 8):
    """The C oracle (CPU port, float64 arithmetic, OpenMP over the host's
    cores) running the whole config-2 step -- all 8192 rows, both dtypes --
    repeated until ``min_seconds`` have passed; GB/s of algorithmic bytes.
    Operand preparation (generation, dtype conversion) is not timed."""
    from oracle import binding as orc

    rows = N
    g = np.random.default_rng(0)
    a = g.standard_normal((rows, N), dtype=np.float32)
    row = g.uniform(0.5, 2.0, N).astype(np.float32)
    col = g.uniform(0.5, 2.0, (rows, 1)).astype(np.float32)
    grad = g.standard_normal((rows, N), dtype=np.float32)
    prepared = {}
    for dtype in (F32, BF16):
        A, R, Cc, G = (orc.from_float(v, dtype) for v in (a, row, col, grad))
        absa = orc.unary(5, dtype, A)
        prepared[dtype] = (A, R, Cc, G, absa, orc.affine(dtype, absa, 1.0, 1e-3))
    del a, grad

    def one_pass() -> int:
        total = 0
        for dtype, (A, R, Cc, G, absa, loga) in prepared.items():
            e = ESIZE[dtype] * rows * N
            for b in (R, Cc):
                for op, alpha in ((0, 1.0), (0, -1.0), (1, 1.0), (2, 1.0)):
                    orc.binary(op, dtype, A, b, alpha)
                    total += 2 * e
            work = A.copy()
            for op, alpha in ((0, 1.0), (0, -1.0), (1, 1.0), (2, 1.0)):
                orc.binary(op, dtype, work, R, alpha, out=work)
                total += 2 * e
            for al, be in ((1.0, 2.0), (1.0, -2.0), (3.0, 0.0), (0.25, 0.0)):
                orc.affine(dtype, A, al, be)
                total += 2 * e
            for op, x in ((0, A), (1, loga), (2, absa), (6, A), (8, A), (12, A), (9, A)):
                orc.unary(op, dtype, x)
                total += 2 * e
            y = orc.unary(9, dtype, A)
            for op, sv in ((0, A), (3, A), (1, y)):
                orc.activation_backward(op, dtype, G, sv)
                total += 3 * e
        return total

    total_bytes, passes, t0 = 0, 0, time.perf_counter()
    while passes < max_passes and (passes == 0 or time.perf_counter() - t0 < min_seconds):
        total_bytes += one_pass()
        passes += 1
    secs = time.perf_counter() - t0
    return {"value": round(total_bytes / secs / 1e9, 3), "unit": "GB/s",
            "cores": int(orc.lib().orc_num_threads()), "kind": "port",
            "seconds": round(secs, 2),
            "sample": f"the full config-2 step ({N}x{N}, 26 operators, fp32 and bf16) "
                      f"repeated {passes} times (repository C oracle, float64 arithmetic, "
                      "OpenMP; TensorPlay's CPU path is not installed)"}


def _torch_cpu(cores: int):
    """torch on the host CPU with the oracle's thread count, or None.

    torch stays on the CPU here: imported after the backend, it brings its
    own copy of the HIP and HSA runtimes into the process (its libraries ask
    for libamdhip64.so by file name from their own directory), and starting
    that second runtime on the same GPU is not safe."""
    try:
        import torch
    except ImportError:
        return None
    torch.set_num_threads(cores)
    return torch


def torch_cpu_mm(cores: int, seconds: float) -> dict:
    """A calibration line beside the oracle's GEMM figure: torch's CPU matmul
    (its BLAS, float32) on the whole 4096^3 mm, TFLOP/s; not TensorPlay's
    CPU path."""
    torch = _torch_cpu(cores)
    if torch is None:
        return {"error": "torch not importable"}
    g = torch.Generator().manual_seed(0)
    a = torch.randn(4096, 4096, generator=g)
    b = torch.randn(4096, 4096, generator=g)
    torch.mm(a, b)
    n, t0 = 0, time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        torch.mm(a, b)
        n += 1
    secs = time.perf_counter() - t0
    return {"value": float(f"{2 * 4096 ** 3 * n / secs / 1e12:.4g}"), "unit": "TFLOP/s", "cores": cores,
            "kind": "calibration", "sample": f"torch.mm fp32 4096^3 on the host CPU, {n} call(s)"}


def torch_cpu_config3(cores: int, seconds: float) -> dict:
    """A calibration line beside the oracle's config-3 figure: torch on the
    host CPU running X1's four reductions over dim -1 and 0 and softmax /
    log_softmax forward on the whole X1 [32768, 4096] fp32, GB/s of
    algorithmic bytes; not TensorPlay's CPU path."""
    torch = _torch_cpu(cores)
    if torch is None:
        return {"error": "torch not importable"}
    x = torch.randn(32768, 4096, generator=torch.Generator().manual_seed(0)) * 2.0
    n_bytes = x.numel() * 4

    def one():
        for dim in (-1, 0):
            x.sum(dim), x.mean(dim), x.amax(dim), x.amin(dim)
        torch.softmax(x, -1), torch.log_softmax(x, -1)
        return 8 * n_bytes + 2 * 2 * n_bytes

    work, n, t0 = 0, 0, time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        work += one()
        n += 1
    secs = time.perf_counter() - t0
    return {"value": float(f"{work / secs / 1e9:.4g}"), "unit": "GB/s", "cores": cores, "kind": "calibration",
            "sample": f"torch CPU: sum/mean/amax/amin over dim -1 and 0 and softmax/log_softmax forward on "
                      f"X1 [32768, 4096] fp32, {n} pass(es)"}


def torch_cpu_config2(cores: int, seconds: float) -> dict:
    """A calibration line beside the headline's CPU baseline: torch on the
    host CPU, with the oracle's thread count, running the config-2 step's 26
    operators on the whole [8192, 8192] operands in float32 and bfloat16
    storage, GB/s of the same algorithmic bytes; not TensorPlay's CPU path."""
    torch = _torch_cpu(cores)
    if torch is None:
        return {"error": "torch not importable"}
    g = torch.Generator().manual_seed(0)
    base = torch.randn(N, N, generator=g)
    row32, col32 = torch.rand(N, generator=g) * 1.5 + 0.5, torch.rand(N, 1, generator=g) * 1.5 + 0.5
    grad32 = torch.randn(N, N, generator=g)
    F = torch.nn.functional
    prepared = [(tuple(t.to(dt) for t in (base, row32, col32, grad32)), e)
                for dt, e in ((torch.float32, 4), (torch.bfloat16, 2))]
    del base, grad32

    def one_pass() -> int:
        total = 0
        for (a, row, col, grad), e in prepared:
            nb = N * N * e
            for b in (row, col):
                torch.add(a, b), torch.sub(a, b), torch.mul(a, b), torch.div(a, b)
                total += 8 * nb
            w = a.clone()
            w.add_(row), w.sub_(row), w.mul_(row), w.div_(row)
            total += 8 * nb
            a + 2.0, a - 2.0, a * 3.0, a * 0.25
            total += 8 * nb
            torch.exp(a), torch.log(a.abs() + 1e-3), torch.sqrt(a.abs()), torch.pow(a, 2)
            torch.relu(a), F.gelu(a), torch.sigmoid(a)
            total += 14 * nb
            y = torch.sigmoid(a)
            torch.where(a > 0, grad, torch.zeros_like(grad))
            torch.ops.aten.gelu_backward(grad, a)
            torch.ops.aten.sigmoid_backward(grad, y)
            total += 9 * nb
        return total

    work, n, t0 = 0, 0, time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        work += one_pass()
        n += 1
    secs = time.perf_counter() - t0
    return {"value": float(f"{work / secs / 1e9:.4g}"), "unit": "GB/s", "cores": cores, "kind": "calibration",
            "seconds": round(secs, 2),
            "sample": f"torch CPU: the config-2 step's 26 operators on [{N}, {N}] fp32 and bf16, {n} pass(es)"}


def cpu_suite(seconds_each: float = 3.0) -> dict:
    """CPU figures beside the suite's sections, in each section's unit: the C
    oracle (float64 arithmetic, OpenMP over the host's cores) on a bounded
    sample of the section's workload, repeated until ``seconds_each`` have
    passed (at least once).  Operand preparation is not timed."""
    from oracle import binding as orc

    cores = int(orc.lib().orc_num_threads())
    note = "repository C oracle, float64 arithmetic, OpenMP; TensorPlay's CPU path is not installed"
    g = np.random.default_rng(0)

    def timed(fn):
        work, passes, t0 = 0, 0, time.perf_counter()
        while passes == 0 or time.perf_counter() - t0 < seconds_each:
            work += fn()
            passes += 1
        return work, time.perf_counter() - t0, passes

    def entry(value, unit, secs, passes, sample):
        return {"value": float(f"{value:.4g}"), "unit": unit, "cores": cores, "kind": "port",
                "seconds": round(secs, 2), "sample": f"{sample}, {passes} pass(es) ({note})"}

    out = {}
    # Config 3: 1024 of X1's 32768 rows, fp32 and bf16.
    rows, D = 1024, 4096
    x32 = g.standard_normal((rows, D), dtype=np.float32) * np.float32(2.0)
    g32 = g.standard_normal((rows, D), dtype=np.float32)
    prep = {}
    for dt in (F32, BF16):
        X, G = orc.from_float(x32, dt), orc.from_float(g32, dt)
        prep[dt] = (X, G, orc.softmax(False, dt, X, rows, D, 1), orc.softmax(True, dt, X, rows, D, 1))

    def config3():
        total = 0
        for dt, (X, G, Y, LY) in prep.items():
            n = rows * D * ESIZE[dt]
            for op in (0, 1, 2, 3):  # sum, mean, amax, amin over dim -1, then dim 0
                orc.reduce(op, dt, X, rows, D, 1)
                orc.reduce(op, dt, X, 1, rows, D)
                total += 2 * n + (rows + D) * ESIZE[dt]
            for log in (False, True):
                orc.softmax(log, dt, X, rows, D, 1)
                orc.softmax_backward(log, dt, LY if log else Y, G, rows, D, 1)
                total += 5 * n
        return total

    work, secs, passes = timed(config3)
    out["config3"] = entry(work / secs / 1e9, "GB/s", secs, passes,
                           "sum/mean/amax/amin over dim -1 and 0, softmax and log_softmax forward "
                           f"and backward on {rows} of X1's 32768 rows [x 4096], fp32 and bf16")
    out["config3"]["torch_cpu_calibration"] = torch_cpu_config3(cores, seconds_each)
    del prep
    # Config 4: 64 rows of the 4096^3 products, fp32 and bf16 (fp32 accumulation).
    m, K = 64, 4096
    ops4 = {}
    for dt in (F32, BF16):
        a = orc.from_float(g.standard_normal((m, K), dtype=np.float32) * np.float32(K ** -0.25), dt)
        b = orc.from_float(g.standard_normal((K, K), dtype=np.float32) * np.float32(K ** -0.25), dt)
        ops4[dt] = (a, b)

    def config4():
        for dt, (a, b) in ops4.items():
            orc.gemm(dt, a, b)
        return 2 * (2 * m * K * K)

    work, secs, passes = timed(config4)
    out["config4"] = entry(work / secs / 1e12, "TFLOP/s", secs, passes,
                           f"mm {m}x{K}x{K} ({m} of the 4096 rows of config 4's mm), fp32 and bf16")
    out["config4"]["torch_cpu_calibration"] = torch_cpu_mm(cores, seconds_each)
    del ops4
    # Config 5b: the MLP training step on 32 of the batch's 8192 rows (four
    # Linear(4096, 4096) + ReLU, Linear(4096, 1000), log_softmax, NLL through
    # mul + sum with a one-hot, backward, SGD), every operator from the oracle.
    bsz, width, classes, lr = 32, 4096, 1000, 1e-3
    Ws = [g.standard_normal((width, width), dtype=np.float32) * np.float32(width ** -0.5) for _ in range(4)]
    Ws.append(g.standard_normal((classes, width), dtype=np.float32) * np.float32(width ** -0.5))
    bs = [np.zeros(w.shape[0], np.float32) for w in Ws]
    x = g.standard_normal((bsz, width), dtype=np.float32)
    onehot = np.zeros((bsz, classes), np.float32)
    onehot[np.arange(bsz), g.integers(0, classes, size=bsz)] = 1.0
    per_row = 2 * (4 * width * width + width * classes) * 2 + 2 * (3 * width * width + width * classes)

    def config5b():
        hs, zs = [x], []
        for li in range(4):
            zs.append(orc.gemm(F32, hs[-1], Ws[li], trans_b=True, beta=1.0, cin=bs[li]))
            hs.append(orc.unary(8, F32, zs[-1]))
        logits = orc.gemm(F32, hs[-1], Ws[4], trans_b=True, beta=1.0, cin=bs[4])
        lp = orc.softmax(True, F32, logits, bsz, classes, 1)
        orc.reduce(0, F32, orc.binary(1, F32, lp, onehot), 1, bsz * classes, 1)
        dlogits = orc.softmax_backward(True, F32, lp, orc.affine(F32, onehot, -1.0 / bsz, 0.0),
                                       bsz, classes, 1)
        grads = [None] * 5
        grads[4] = (orc.gemm(F32, dlogits, hs[4], trans_a=True), orc.reduce(0, F32, dlogits, 1, bsz, classes))
        da = orc.gemm(F32, dlogits, Ws[4])
        for li in range(3, -1, -1):
            dz = orc.activation_backward(0, F32, da, zs[li], 0.0)
            grads[li] = (orc.gemm(F32, dz, hs[li], trans_a=True), orc.reduce(0, F32, dz, 1, bsz, width))
            if li > 0:
                da = orc.gemm(F32, dz, Ws[li])
        for li in range(5):
            orc.binary(0, F32, Ws[li], grads[li][0], -lr, out=Ws[li])
            orc.binary(0, F32, bs[li], grads[li][1], -lr, out=bs[li])
        return per_row * bsz

    work, secs, passes = timed(config5b)
    out["config5b"] = entry(work / secs / 1e12, "TFLOP/s", secs, passes,
                            f"the fp32 MLP training step on {bsz} of the batch's 8192 rows "
                            "(GEMM flops of the sampled step over its time)")
    del Ws, bs
    # NN layers: layer norm forward and backward on 1024 of the 8192 rows.
    rows = 1024
    xs = g.standard_normal((rows, D), dtype=np.float32)
    dys = g.standard_normal((rows, D), dtype=np.float32)
    w = g.standard_normal(D, dtype=np.float32)
    bb = g.standard_normal(D, dtype=np.float32)
    _, mean, rstd = orc.layer_norm(F32, xs, D, w, bb)

    def nn():
        orc.layer_norm(F32, xs, D, w, bb)
        orc.layer_norm_backward(F32, dys, xs, D, mean, rstd, w)
        return 5 * rows * D * 4

    work, secs, passes = timed(nn)
    out["nn"] = entry(work / secs / 1e9, "GB/s", secs, passes,
                      f"layer norm forward and backward on {rows} of the 8192 rows [x {D}], fp32")
    return out


def profile_launches(what: str, lib, ops, dev) -> None:
    """Fixed launch sequences for counter and trace collection under
    rocprofv3 (``--profile``); no timing, no JSON line.

    traffic: ten launches of a copy-like kernel (affine y = 1 x + 0 on
             [8192, 8192] float32, 2 x 268,435,456 B) to calibrate the
             FETCH_SIZE / WRITE_SIZE counters, then ten of the dominant kernel;
    traffic_cold: the same calibration, then sixteen launches of the
             dominant kernel rotating over four inputs and four outputs
             (the cold measurement's sequence);
    gemm:    ten bf16 4096^3 products in each operand layout (A, B
             row-major; B transposed; A transposed; both transposed), the
             four layouts twice over (the second pass at a settled clock);
    gemm32:  the same in float32, five products a layout;
    linear:  ten config-4 bf16 linears, x [8192, 4096] @ W[11008, 4096]^T + b;
    vs_torch: bf16 4096^3 A @ B and A @ B^T and the config-4 linear, from
             this library and from torch (hipBLASLt) on the same GPU,
             interleaved: four rounds of ten calls a case each;
    mlp:     three config-5b training steps (fp32 MLP, batch 8192, four
             Linear(4096, 4096) + ReLU, Linear(4096, 1000), log_softmax, NLL
             through mul + sum, backward, SGD) after one untimed step;
    reduce:  config-3 X1 [32768, 4096], then X2 [4096, 32000]: sum and amax
             over dim -1 and 0, fp32 and bf16, five each;
    bmm:     ten launches of the copy-like kernel of ``traffic`` (counter
             calibration), then twenty config-5a products, bf16
             [64, 512, 128] x [64, 128, 512];
    reduce_all: whole-tensor sum and amax of 4096^2 in fp32, fp16 and bf16,
             then the config-5b loss sum over [8192, 1000] fp32, twenty each;
    softmax: config-3 softmax forward and backward on X1 [32768, 4096] and
             X2 [4096, 32000], fp32 and bf16, five each;
    nn:      the NN-layer suite's shapes, fp32 and bf16, five launches of
             each operator: layer norm forward and backward [8192, 4096],
             dropout p = 0.1 and its backward, embedding of 8192 indices into
             [32000, 4096] and its dense gradient, nll_loss over
             [8192, 32000] and its backward;
    vs_torch_thin: thin bf16 products of a decode step (Linear of 1 and
             16 rows, x @ W with W [4096, 11008], an LM head's logits and
             dX), this library and torch interleaved as in vs_torch, each
             rotating over its own copies of the wide operand;
    vs_torch_batch: bf16 products of a small batch (Linear of 32 and 64
             rows, x @ W with 64 rows and W [4096, 11008]), this library and
             torch interleaved as in vs_torch_thin;
    thin:    the thin products of the suite (decode-step Linear layers,
             an LM head's logits and dX), ten launches each, the wide
             operand rotated over its copies;
    odd:     products whose operands the matrix cores cannot read in place,
             repacked: ten bf16 mm 2047^3 and five bf16 [2048, 4096] x
             [4096, 50257]; then binary ops with transposed inputs, fp32 and
             bf16 4096^2, ten x.t() + y and ten x.t() * y.t() each."""
    import ctypes as C
    if what == "thin":
        for name, x, ws, fn, _ in thin_cases(ops, dev):
            for k in range(10):
                fn(x, ws[k % len(ws)])
        return
    if what == "traffic_cold":
        a = dev.from_numpy(np.full((N, N), 1.5, np.float32))
        row = dev.from_numpy(np.full((N,), 0.5, np.float32))
        out = ops.empty((N, N), F32)
        for _ in range(10):
            assert lib.tp_amd_launch_affine(0, F32, N * N, a.data_ptr, 1.0, 0.0, out.data_ptr) == 0
        inputs = [a] + [ops.add_scalar(a, float(k)) for k in range(1, COLD_PAIRS)]
        outputs = [out] + [ops.empty((N, N), F32) for _ in range(1, COLD_PAIRS)]
        sizes = (C.c_int64 * 2)(N, N)
        sa, sb = (C.c_int64 * 2)(N, 1), (C.c_int64 * 2)(0, 1)
        for _ in range(4):
            for x, y in zip(inputs, outputs):
                assert lib.tp_amd_launch_binary(0, 0, F32, 2, sizes, x.data_ptr, sa, row.data_ptr, sb,
                                                y.data_ptr, sa, 1.0) == 0
    elif what == "traffic":
        a = dev.from_numpy(np.full((N, N), 1.5, np.float32))
        row = dev.from_numpy(np.full((N,), 0.5, np.float32))
        out = ops.empty((N, N), F32)
        sizes = (C.c_int64 * 2)(N, N)
        sa, sb = (C.c_int64 * 2)(N, 1), (C.c_int64 * 2)(0, 1)
        for _ in range(10):
            assert lib.tp_amd_launch_affine(0, F32, N * N, a.data_ptr, 1.0, 0.0, out.data_ptr) == 0
        for _ in range(10):
            assert lib.tp_amd_launch_binary(0, 0, F32, 2, sizes, a.data_ptr, sa, row.data_ptr, sb,
                                            out.data_ptr, sa, 1.0) == 0
    elif what == "bmm":
        a = dev.from_numpy(np.full((N, N), 1.5, np.float32))
        out = ops.empty((N, N), F32)
        for _ in range(10):
            assert lib.tp_amd_launch_affine(0, F32, N * N, a.data_ptr, 1.0, 0.0, out.data_ptr) == 0
        del a, out
        g = np.random.default_rng(0)
        x = ops.to(dev.from_numpy(g.standard_normal((64, 512, 128), dtype=np.float32)), BF16)
        y = ops.to(dev.from_numpy(g.standard_normal((64, 128, 512), dtype=np.float32)), BF16)
        for _ in range(20):
            ops.bmm(x, y)
    elif what in ("gemm", "gemm32"):
        K = 4096
        dt, reps = (BF16, 10) if what == "gemm" else (F32, 5)
        g = np.random.default_rng(0)
        a = dev.from_numpy(g.standard_normal((K, K), dtype=np.float32))
        b = dev.from_numpy(g.standard_normal((K, K), dtype=np.float32))
        if dt != F32:
            a, b = ops.to(a, dt), ops.to(b, dt)
        c = ops.empty((K, K), dt)
        # two passes over the layouts: the shader clock settles during the
        # first (the same product runs ~15 % slower at the start of a run),
        # so the second pass compares the layouts at one clock
        for _ in range(2):
            for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
                for _ in range(reps):
                    assert lib.tp_amd_launch_gemm(0, dt, 1, K, K, K, 1.0, a.data_ptr, K, 0, ta,
                                                  b.data_ptr, K, 0, tb, 0.0, None, 0, 0, 0,
                                                  c.data_ptr, K, 0) == 0
    elif what == "linear":
        # config 4's linear: x [8192, 4096] @ W[11008, 4096]^T + b[11008], bf16
        g = np.random.default_rng(0)
        x = ops.to(dev.from_numpy(g.standard_normal((8192, 4096), dtype=np.float32) / 64), BF16)
        w = ops.to(dev.from_numpy(g.standard_normal((11008, 4096), dtype=np.float32) / 64), BF16)
        bias = ops.to(dev.from_numpy(g.standard_normal(11008, dtype=np.float32)), BF16)
        for _ in range(10):
            ops.linear(x, w, bias)
    elif what == "vs_torch":
        # The bf16 products of config 4 from this library and from torch on
        # the same GPU (hipBLASLt), interleaved: per round and case, ten
        # calls of one then ten of the other, the order swapped every round.
        import torch
        F = torch.nn.functional
        g = np.random.default_rng(0)

        def both(shape):
            a32 = g.standard_normal(shape, dtype=np.float32) * np.float32(shape[-1] ** -0.25)
            return ops.to(dev.from_numpy(a32), BF16), torch.from_numpy(a32).to("cuda").to(torch.bfloat16)

        a, ta = both((4096, 4096))
        b, tb = both((4096, 4096))
        x, tx = both((8192, 4096))
        w, tw = both((11008, 4096))
        bias, tbias = both((11008,))
        cases = [(lambda: ops.mm(a, b), lambda: torch.mm(ta, tb)),
                 (lambda: ops.mm(a, b.t()), lambda: torch.mm(ta, tb.t())),
                 (lambda: ops.linear(x, w, bias), lambda: F.linear(tx, tw, tbias))]

        def drain():
            assert lib.tp_amd_synchronize(0) == 0
            torch.cuda.synchronize()

        for rnd in range(4):
            for ours, theirs in cases:
                for fn in ((ours, theirs) if rnd % 2 == 0 else (theirs, ours)):
                    for _ in range(10):
                        fn()
                    drain()
    elif what in ("vs_torch_thin", "vs_torch_batch"):
        # Thin bf16 products of a decode step (or of a small batch) from this
        # library and from torch on the same GPU, interleaved as in vs_torch,
        # each library rotating over its own copies of the wide operand.
        import torch
        F = torch.nn.functional
        g = np.random.default_rng(0)

        def both(shape, copies=1):
            a32 = g.standard_normal(shape, dtype=np.float32) * np.float32(shape[-1] ** -0.5)
            ours = ops.to(dev.from_numpy(a32), BF16)
            theirs = torch.from_numpy(a32).to("cuda").to(torch.bfloat16)
            del a32
            return ([ours] + [ops.add_scalar(ours, 0.001 * k) for k in range(1, copies)],
                    [theirs] + [theirs + 0.001 * k for k in range(1, copies)])

        w, tw = both((11008, 4096), 4)
        wn, twn = both((4096, 11008), 4)
        x1, tx1 = both((1, 4096))
        x16, tx16 = both((16, 4096))
        head, thead = both((50257, 4096), 2)
        dy, tdy = both((1, 50257))
        k = [0]

        def rot(ws):
            k[0] += 1
            return ws[k[0] % len(ws)]
        cases = [(lambda: ops.linear(x1[0], rot(w)), lambda: F.linear(tx1[0], rot(tw))),
                 (lambda: ops.linear(x16[0], rot(w)), lambda: F.linear(tx16[0], rot(tw))),
                 (lambda: ops.mm(x1[0], rot(wn)), lambda: torch.mm(tx1[0], rot(twn))),
                 (lambda: ops.linear(x1[0], rot(head)), lambda: F.linear(tx1[0], rot(thead))),
                 (lambda: ops.mm(dy[0], rot(head)), lambda: torch.mm(tdy[0], rot(thead)))]
        if what == "vs_torch_batch":
            x32, tx32 = both((32, 4096))
            x64, tx64 = both((64, 4096))
            cases = [(lambda: ops.linear(x32[0], rot(w)), lambda: F.linear(tx32[0], rot(tw))),
                     (lambda: ops.linear(x64[0], rot(w)), lambda: F.linear(tx64[0], rot(tw))),
                     (lambda: ops.mm(x64[0], rot(wn)), lambda: torch.mm(tx64[0], rot(twn)))]

        def drain():
            assert lib.tp_amd_synchronize(0) == 0
            torch.cuda.synchronize()

        for rnd in range(4):
            for ours, theirs in cases:
                for fn in ((ours, theirs) if rnd % 2 == 0 else (theirs, ours)):
                    for _ in range(10):
                        fn()
                    drain()
    elif what == "reduce":
        g = np.random.default_rng(0)
        for shape in ((32768, 4096), (4096, 32000)):
            x32 = dev.from_numpy(g.standard_normal(shape, dtype=np.float32))
            for x in (x32, ops.to(x32, BF16)):
                for fn in (ops.sum_dim, ops.amax):
                    for dim in (-1, 0):
                        for _ in range(5):
                            fn(x, [dim])
            del x32, x
    elif what == "reduce_all":
        g = np.random.default_rng(0)
        x32 = dev.from_numpy(g.standard_normal((4096, 4096), dtype=np.float32))
        for x in (x32, ops.to(x32, F16), ops.to(x32, BF16)):
            for fn in (ops.sum, lambda t: ops.amax(t, [])):
                for _ in range(20):
                    fn(x)
        loss = dev.from_numpy(g.standard_normal((8192, 1000), dtype=np.float32))
        for _ in range(20):
            ops.sum(loss)
    elif what == "softmax":
        g = np.random.default_rng(0)
        for shape in ((32768, 4096), (4096, 32000)):
            x32 = dev.from_numpy(g.standard_normal(shape, dtype=np.float32) * np.float32(2.0))
            g32 = dev.from_numpy(g.standard_normal(shape, dtype=np.float32))
            for dtype in (F32, BF16):
                x, dy = (x32, g32) if dtype == F32 else (ops.to(x32, dtype), ops.to(g32, dtype))
                y = ops.softmax(x, -1)
                for _ in range(5):
                    ops.softmax(x, -1)
                    ops._softmax_backward_data(dy, y, -1, dtype)
                del x, dy, y
            del x32, g32
    elif what == "nn":
        g = np.random.default_rng(0)
        rows, D, V, C = 8192, 4096, 32000, 32000
        idx = dev.from_numpy(g.integers(0, V, size=rows).astype(np.int64))
        tgt = dev.from_numpy(g.integers(0, C, size=rows).astype(np.int64))
        for dtype in (F32, BF16):
            def put(shape):
                d = dev.from_numpy(g.standard_normal(shape, dtype=np.float32))
                return d if dtype == F32 else ops.to(d, dtype)
            x, dy, w, b = put((rows, D)), put((rows, D)), put((D,)), put((D,))
            _, mean, rstd = ops.native_layer_norm(x, (D,), w, b)
            _, mask = ops.native_dropout(x, 0.1, True, 1)
            table, logp = put((V, D)), put((rows, C))
            _, total = ops.nll_loss(logp, tgt, None, 1)
            one = ops.to(dev.from_numpy(np.array(1.0, np.float32)), dtype)
            for _ in range(5):
                ops.native_layer_norm(x, (D,), w, b)
                ops.native_layer_norm_backward(dy, x, (D,), mean, rstd, w, b)
                ops.native_dropout(x, 0.1, True, 7)
                ops.native_dropout_backward(dy, mask, 1 / 0.9)
                ops.embedding(table, idx)
                ops.embedding_dense_backward(dy, idx, V)
                ops.nll_loss(logp, tgt, None, 1)
                ops.nll_loss_backward(one, logp, tgt, None, 1, -100, total)
            del x, dy, w, b, mean, rstd, mask, table, logp, total
    elif what == "odd":
        g = np.random.default_rng(3)

        def put(shape, dtype):
            d = dev.from_numpy(g.standard_normal(shape, dtype=np.float32) * np.float32(0.05))
            return d if dtype == F32 else ops.to(d, dtype)
        a, b = put((2047, 2047), BF16), put((2047, 2047), BF16)
        for _ in range(10):
            ops.mm(a, b)
        h, w = put((2048, 4096), BF16), put((4096, 50257), BF16)
        for _ in range(5):
            ops.mm(h, w)
        del a, b, h, w
        for dtype in (F32, BF16):
            x, y = put((4096, 4096), dtype), put((4096, 4096), dtype)
            for _ in range(10):
                ops.add(x.t(), y)
            for _ in range(10):
                ops.mul(x.t(), y.t())
            del x, y
    elif what == "mlp":
        wl = importlib.import_module("tensorplay-mlu_amd.workloads")
        ws, bs = wl.MLP.host_init(4096, 4, 4096, 1000, seed=0)
        model = wl.MLP.to_device(ws, bs)
        del ws, bs
        g = np.random.default_rng(100)
        x = dev.from_numpy(g.standard_normal((8192, 4096), dtype=np.float32))
        onehot = np.zeros((8192, 1000), np.float32)
        onehot[np.arange(8192), g.integers(0, 1000, 8192)] = 1.0
        oh = dev.from_numpy(onehot)
        for _ in range(4):
            wl.mlp_step(ops, model, x, oh, 1e-3)
    else:
        raise SystemExit(f"unknown --profile {what}")
    assert lib.tp_amd_synchronize(0) == 0
    log(f"bench: profile launches '{what}' done")


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-suite", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--profile", choices=["traffic", "traffic_cold", "gemm", "gemm32", "linear", "vs_torch", "bmm",
                                         "reduce", "reduce_all", "softmax", "nn", "mlp", "odd", "thin",
                                         "vs_torch_thin", "vs_torch_batch"],
                   help="run a fixed launch sequence for rocprofv3 and exit")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        return 2

    if args.profile in ("vs_torch", "vs_torch_thin", "vs_torch_batch"):
        # torch's GPU path loads its own copy of the HIP runtime by a name
        # this library does not ask for; loaded first, it is the one copy in
        # the process, and this library binds to it by soname.  Loaded after
        # this library, the process would hold two runtimes on one GPU.
        import torch
        torch.cuda.init()
    lib = amd.load()
    ops = importlib.import_module("tensorplay-mlu_amd.ops")
    runtime = importlib.import_module("tensorplay-mlu_amd.runtime")
    dev = importlib.import_module("tensorplay-mlu_amd.tensor").DeviceTensor
    if not runtime.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    if args.profile:
        profile_launches(args.profile, lib, ops, dev)
        return 0

    log("bench: building config-2 inputs")
    tensors = {F32: build_config2(ops, dev, F32), BF16: build_config2(ops, dev, BF16)}
    tensors[F32]["out"] = ops.empty((N, N), F32)
    plan = [(fn, factor * N * N * ESIZE[d]) for d, t in tensors.items()
            for _, fn, factor in config2_ops(ops, t)]
    step_bytes = sum(b for _, b in plan)

    def step():
        for fn, _ in plan:
            fn()

    log(f"bench: warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    runtime.synchronize()
    ev = Events(lib)
    log(f"bench: timing {args.steps} steps")
    runtime.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    runtime.synchronize()
    secs = time.perf_counter() - t0
    value = step_bytes * args.steps / secs / 1e9

    log("bench: dominant kernel, warm and cold")
    roofline_warm = dominant_kernel(lib, ev, tensors[F32])
    roofline = dominant_kernel_cold(lib, ops, ev, tensors[F32])
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(secs / args.steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config2: broadcast elementwise, [8192,8192] fp32 and bf16 "
                               "storage, row [8192] and column [8192,1] broadcasts, 26 operators "
                               "per dtype (forward, in-place, scalar, unary, activation backward)",
                   "shape": [N, N], "storage_dtypes": ["fp32", "bf16"],
                   "bytes_per_step": step_bytes, "parallelism": "single GPU"},
        "roofline": roofline,
        "roofline_warm": roofline_warm,
    }
    if not args.no_suite:
        def section(name, fn):
            # A section that fails is reported as such; the headline line
            # above it still prints.
            log(f"bench: suite {name}")
            try:
                return fn()
            except Exception as exc:  # noqa: BLE001 - recorded in the JSON line
                log(f"bench: suite {name} failed: {exc!r}")
                return {"error": repr(exc)}

        suite = {"timing": "config2..nn: average of back-to-back calls between two HIP events on the "
                           "library's stream (10 calls after 2 untimed; GEMM 5 after 5 untimed; the MLP step 3 after 1); "
                           "readme_rows: median of 50 single-call HIP-event pairs after 5 untimed, the "
                           "reference README's method (host copies: wall clock)"}
        suite["config2"] = section("config 2", lambda: suite_config2(ops, ev, tensors))
        del tensors
        suite["config3"] = section("config 3", lambda: suite_config3(ops, dev, ev))
        suite["config4_5a"] = section("configs 4 and 5a", lambda: suite_gemm(ops, dev, ev))
        suite["thin"] = section("thin products", lambda: suite_thin(ops, dev, ev))
        suite["config5b"] = section("config 5b", lambda: suite_config5b(ops, dev, ev))
        suite["nn"] = section("NN layers", lambda: suite_nn(ops, dev, ev))
        suite["readme_rows"] = section("the reference README's rows", lambda: suite_readme(ops, dev, ev, lib))
        result["suite"] = suite
    if not args.no_cpu:
        log("bench: cpu baseline")
        result["cpu_baseline"] = cpu_baseline()
        log("bench: torch cpu calibration of the headline")
        try:
            result["cpu_baseline"]["torch_cpu_calibration"] = torch_cpu_config2(
                result["cpu_baseline"]["cores"], 5.0)
        except Exception as exc:  # noqa: BLE001 - recorded in the JSON line
            result["cpu_baseline"]["torch_cpu_calibration"] = {"error": repr(exc)}
        if not args.no_suite:
            log("bench: cpu samples of the suite")
            try:
                result["suite_cpu"] = cpu_suite()
            except Exception as exc:  # noqa: BLE001 - recorded in the JSON line
                result["suite_cpu"] = {"error": repr(exc)}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
