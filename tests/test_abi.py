"""The C-ABI library loads on a machine without a GPU and exports every
entry point ``include/*.h`` declares; the Python bindings cover all of
them.  No device work is issued."""

import ctypes
import importlib
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for header in ("tp_amd_runtime.h", "tp_amd_kernels.h", "tp_amd_ops.h"):
        text = open(os.path.join(ROOT, "include", header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(tp_(?:amd|mlu)_\w+)\s*\(",
                                text, flags=re.M))
    return names


def test_headers_declare_the_reference_surface():
    names = declared_functions()
    # the reference's Module.cpp entry points keep their names and arity
    for n in ("tp_mlu_init", "tp_mlu_device_count", "tp_mlu_memory_stats",
              "tp_mlu_reset_peak_memory_stats", "tp_mlu_empty_cache", "tp_mlu_last_error"):
        assert n in names
    assert len(names) >= 99


def test_library_exports_every_declared_symbol(amd):
    lib = ctypes.CDLL(amd.library_path())
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_every_declared_symbol():
    abi = importlib.import_module("tensorplay-mlu_amd._abi")
    assert declared_functions() == set(abi.PROTOTYPES)


def test_ops_mirror_the_72_registrations(amd):
    ops = importlib.import_module("tensorplay-mlu_amd.ops")
    assert len(ops.REGISTRATIONS) == 72
    assert all(callable(f) for f in ops.REGISTRATIONS.values())


def test_init_and_counts_without_a_device(amd):
    lib = amd.load()
    assert lib.tp_mlu_init() == 0
    assert lib.tp_mlu_device_count() >= 0
    stats = (ctypes.c_int64 * 4)()
    lib.tp_mlu_memory_stats(0, stats)  # no device: zeros, no crash
    if lib.tp_mlu_device_count() == 0:
        assert list(stats) == [0, 0, 0, 0]
        assert lib.tp_amd_set_device(0) == -1
        assert b"out of range" in lib.tp_mlu_last_error()
        assert lib.tp_amd_launch_affine(0, 0, 4, None, 1.0, 0.0, None) == -1


def test_oracle_builds_and_exports():
    from oracle import binding

    lib = binding.lib()
    for n in ("orc_binary", "orc_affine", "orc_unary", "orc_activation_backward", "orc_reduce",
              "orc_softmax", "orc_softmax_backward", "orc_gemm", "orc_gemm_entries", "orc_cast"):
        assert hasattr(lib, n)
    assert lib.orc_num_threads() >= 1


ADAPTER = os.path.join(ROOT, "tensorplay-mlu_amd", "csrc", "tensorplay")


def test_tensorplay_adapter_registers_the_72_operators():
    """The adapter's registration blocks name exactly the operators of the
    reference's five hot-path blocks and its NN block (the Python mirror
    lists the same)."""
    ops = importlib.import_module("tensorplay-mlu_amd.ops")
    text = open(os.path.join(ADAPTER, "Kernels.cpp")).read()
    names = re.findall(r'm\.impl\(\s*"([^"]+)"', text)
    assert len(names) == 72 and len(set(names)) == 72
    assert set(names) == set(ops.REGISTRATIONS)


def test_tensorplay_adapter_compiles():
    """Syntax check of the adapter (C++20, -Wall -Wextra -Werror) against
    declarations of the TensorPlay API as the reference uses it; TensorPlay's
    own headers are not on this machine."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        import pytest
        pytest.skip("g++ not available")
    for source in ("Kernels.cpp", "Backend.cpp", "Profiler.cpp"):
        cmd = [gxx, "-std=c++20", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
               "-I", os.path.join(ROOT, "tests", "native", "tensorplay_api"),
               "-I", os.path.join(ROOT, "include"), os.path.join(ADAPTER, source)]
        done = subprocess.run(cmd, capture_output=True, text=True)
        assert done.returncode == 0, done.stderr[-4000:]
