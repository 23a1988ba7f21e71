"""Host-side operator logic through the C-ABI, with no device work:
dtype promotion (Cnnl.cpp:178-192), broadcast shapes (Cnnl.cpp:194-205),
density (Cnnl.cpp:107-121), the native-dtype rule (Cnnl.h:24-27), element
sizes, and the decline paths that send an operator to the host
(BinaryKernels.cpp:92-101, UnaryKernels.cpp:23-25, ReduceKernels.cpp:86-91,
BlasKernels.cpp:244-248) -- each checked against hand-derived results."""

import ctypes as C
import os
import importlib

import numpy as np
import pytest

F32, F16, BF16, F64, I8, I16, I32, I64, U8, BOOL = range(10)


@pytest.fixture(scope="module")
def lib(amd):
    return amd.load()


@pytest.fixture(scope="module")
def tensor_mod(amd):
    return importlib.import_module("tensorplay-mlu_amd.tensor")


def bshape(lib, a, b):
    out = (C.c_int64 * 8)()
    nd = C.c_int()
    st = lib.tp_amd_broadcast_shape((C.c_int64 * max(len(a), 1))(*a), len(a),
                                    (C.c_int64 * max(len(b), 1))(*b), len(b), out, C.byref(nd))
    return st, list(out)[: nd.value]


@pytest.mark.parametrize("a,b", [((4, 1, 5), (3, 1)), ((8192, 8192), (8192,)),
                                 ((8192, 8192), (8192, 1)), ((), (3, 2)), ((1,), ()),
                                 ((2, 1, 4, 1), (3, 1, 5)), ((0, 3), (1, 3))])
def test_broadcast_shape_matches_numpy(lib, a, b):
    st, shape = bshape(lib, a, b)
    assert st == 0
    assert tuple(shape) == np.broadcast_shapes(a, b)


@pytest.mark.parametrize("a,b", [((4,), (3,)), ((2, 3), (3, 2)), ((5, 0), (5, 2))])
def test_broadcast_shape_rejects(lib, a, b):
    st, _ = bshape(lib, a, b)
    assert st == -1
    assert b"neither is 1" in lib.tp_mlu_last_error()


def test_binary_result_dtype(lib):
    r = lib.tp_amd_binary_result_dtype
    # same dtype
    assert r(BF16, 2, BF16, 2) == BF16
    # a 0-d operand of the same kind does not widen a dimensioned one
    assert r(BF16, 2, F32, 0) == BF16
    assert r(F32, 0, F16, 1) == F16
    assert r(I32, 1, I64, 0) == I32
    # a 0-d integer scalar keeps a float tensor's dtype
    assert r(F16, 3, I64, 0) == F16
    # a 0-d float scalar promotes an integer tensor
    assert r(I64, 1, F32, 0) == F32
    # both dimensioned: the usual promotion
    assert r(F16, 2, BF16, 2) == F32
    assert r(F32, 2, F64, 1) == F64
    assert r(I8, 1, U8, 1) == I16
    assert r(I32, 1, I64, 1) == I64
    assert r(BOOL, 1, I8, 1) == I8
    assert r(BOOL, 1, F16, 1) == F16


def test_native_float_and_element_sizes(lib):
    assert [lib.tp_amd_is_native_float(d) for d in range(10)] == [1, 1, 1] + [0] * 7
    assert [lib.tp_amd_element_size(d) for d in range(10)] == [4, 2, 2, 8, 1, 2, 4, 8, 1, 1]
    assert lib.tp_amd_element_size(42) == 0


def host_ref(amd, shape, strides, dtype=F32):
    abi = importlib.import_module("tensorplay-mlu_amd._abi")
    t = abi.Tensor()
    t.ndim = len(shape)
    for i, (s, st) in enumerate(zip(shape, strides)):
        t.sizes[i] = s
        t.strides[i] = st
    t.dtype = dtype
    t.device = -1
    t.data = 0x1000
    return t


@pytest.mark.parametrize("shape,strides,dense", [
    ((4, 6), (6, 1), True), ((4, 6), (1, 4), True), ((2, 3, 4), (1, 2, 6), True),
    ((4, 6), (12, 1), False), ((4, 6), (0, 1), False), ((1, 5), (99, 1), True),
    ((3, 1, 2), (2, 7, 1), True)])
def test_is_dense(amd, lib, shape, strides, dense):
    t = host_ref(amd, shape, strides)
    assert lib.tp_amd_is_dense(C.byref(t)) == int(dense)


def test_host_operands_are_declined(amd, lib, tensor_mod):
    ops = importlib.import_module("tensorplay-mlu_amd.ops")
    a = np.ones((3, 4), np.float32)
    for call in (lambda: ops.add(a, a), lambda: ops.mul(a, np.float32(2)),
                 lambda: ops.exp(a), lambda: ops.relu(a), lambda: ops.mm(a, a.T),
                 lambda: ops.sum(a), lambda: ops.softmax(a, -1), lambda: ops.mul_scalar(a, 2)):
        with pytest.raises(tensor_mod.DeclinedError):
            call()


def test_null_arguments_are_errors(lib):
    abi = importlib.import_module("tensorplay-mlu_amd._abi")
    out = abi.Tensor()
    assert lib.tp_amd_add(None, None, abi.scalar(1), C.byref(out)) == -1
    assert b"null tensor" in lib.tp_mlu_last_error()
    assert lib.tp_amd_exp(None, C.byref(out)) == -1


def test_profiler_without_a_device_or_tracing(amd):
    """Without a GPU a timer places no marker and reports no time, and
    kernel-level tracing (off unless the process starts with
    TP_AMD_DEVICE_TRACE=1) refuses to start with the reason."""
    if os.environ.get("TP_AMD_DEVICE_TRACE") == "1":
        pytest.skip("tracing requested for this process")
    prof = importlib.import_module("tensorplay-mlu_amd.profiler")
    runtime = importlib.import_module("tensorplay-mlu_amd.runtime")
    if runtime.device_count() == 0:
        t = prof.Timer(0)
        t.start()
        t.stop()
        assert t.elapsed_ms() is None
    assert not prof.Trace.available()
    assert "TP_AMD_DEVICE_TRACE" in prof.Trace.unavailable_reason()
    with pytest.raises(RuntimeError, match="TP_AMD_DEVICE_TRACE"):
        prof.Trace().start()
