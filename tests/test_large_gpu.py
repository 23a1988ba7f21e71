"""Tensors past 2^31 elements (8.6 GB of float32 each): element offsets,
packet counts and grid sizes are 64-bit through the elementwise, fill,
reduction and softmax kernels, and the ragged tail past the last whole
packet is reached; a batched product's batch offsets pass 2^31 elements.
Values are chosen so every expected result is exact."""

import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = 0


def test_elementwise_and_reductions_past_2_31_elements(dev, ops, amd):
    lib = amd.load()
    n = (1 << 31) + 4096 + 3
    a, b = ops.empty((n,), F32), ops.empty((n,), F32)
    ops.fill_(a, 1.0)
    ops.fill_(b, 2.0)
    c = ops.add(a, b, alpha=0.5)
    for lo, hi in ((0, 8), ((1 << 31) - 4, (1 << 31) + 4), (n - 8, n)):
        assert np.array_equal(c[lo:hi].numpy(), np.full(hi - lo, 2.0, np.float32)), (lo, hi)
    s = float(ops.sum(c).numpy())
    assert abs(s - 2.0 * n) <= 1e-6 * 2.0 * n, s
    ops.fill_(c[n - 1:], 7.0)
    assert float(ops.amax(c, []).numpy()) == 7.0
    del a, b, c
    rows, D = (1 << 20) + 7, 2048
    x = ops.empty((rows, D), F32)
    ops.fill_(x, 0.25)
    ops.fill_(x[rows - 1:], 1.0)
    assert np.array_equal(ops.sum_dim(x, [1])[rows - 3:].numpy(), np.float32([512.0, 512.0, 2048.0]))
    assert np.array_equal(ops.sum_dim(x, [0])[-4:].numpy(), np.full(4, 0.25 * (rows - 1) + 1.0, np.float32))
    y = ops.softmax(x, -1)
    assert np.array_equal(y[rows - 1:, -3:].numpy(), np.full((1, 3), 1.0 / D, np.float32))
    assert np.array_equal(ops.mul_scalar(x, 2.0)[rows - 1:, -3:].numpy(), np.full((1, 3), 2.0, np.float32))
    del x, y
    lib.tp_mlu_empty_cache()


def test_batched_product_past_2_31_elements(dev, ops, amd):
    """bmm of [40, 8192, 8192] bf16 operands (2.7e9 elements each): batch b
    of A is (b + 1) / 64 everywhere and B is 1, so C[b] is exactly
    128 (b + 1) -- batches whose offsets pass 2^31 elements included."""
    lib = amd.load()
    B, M = 40, 8192
    a, b = ops.empty((B, M, M), 2), ops.empty((B, M, M), 2)
    for i in range(B):
        ops.fill_(a[i], (i + 1) / 64.0)
    ops.fill_(b, 1.0)
    c = ops.bmm(a, b)
    for i in (0, 15, 16, 31, 39):
        for lo, hi in ((0, 4), (M - 4, M)):
            got = c[i, lo:hi, M - 4:].numpy()
            assert np.array_equal(got.view(np.uint16), np.full((4, 4), np.float32(128.0 * (i + 1)), np.float32)
                                  .view(np.uint32).__rshift__(16).astype(np.uint16)), (i, lo)
    del a, b, c
    lib.tp_mlu_empty_cache()
