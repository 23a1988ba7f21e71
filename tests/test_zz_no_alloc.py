"""The allocation-free reduction entry point, tp_amd_launch_reduce_noalloc,
against tp_amd_launch_reduce through the C-ABI.

Both run the same kernels in the same order, so their results must be
bit-identical; the split reductions' float32 partials come from a static
device array instead of the caching allocator, so the allocator's counters
must not move during the call.  Two calls in a row, the second smaller,
show that what the first left in the shared array does not leak into the
second."""

import ctypes

import numpy as np
import pytest

from _check import BF16, F32, assert_bitexact, assert_sum

pytestmark = pytest.mark.gpu

SUM, MEAN, AMAX, AMIN = 0, 1, 2, 3


def _stats(lib):
    out = (ctypes.c_int64 * 4)()
    lib.tp_mlu_memory_stats(0, out)
    return list(out)


# (outer, r, inner, dtype): a whole tensor, then a smaller one; a column
# reduction over 32768 rows (16 row chunks of partials), then a smaller one.
CASES = [
    [(1, 1 << 24, 1, F32), (1, 3 << 18, 1, F32)],
    [(1, 1 << 22, 1, BF16), (2, 1 << 16, 1, BF16)],
    [(1, 32768, 4096, F32), (1, 4096, 1024, F32)],
    [(1, 32768, 4096, BF16), (3, 2048, 384, BF16)],
]


@pytest.mark.parametrize("pair", CASES, ids=["rows-fp32", "rows-bf16", "cols-fp32", "cols-bf16"])
def test_noalloc_matches_allocating_entry(amd, dev, ops, orc, pair):
    lib = amd.load()
    noalloc = lib.tp_amd_launch_reduce_noalloc
    assert lib.tp_amd_reduce_noalloc_scratch_bytes() == 1 << 20
    for call, (outer, r, inner, dtype) in enumerate(pair):
        x = orc.from_float(np.random.default_rng(call).standard_normal((outer, r, inner))
                           .astype(np.float32) + np.float32(0.5), dtype)
        dx = dev.from_numpy(x, dtype=dtype)
        for op in (SUM, MEAN, AMAX, AMIN):
            want = orc.reduce(op, dtype, x, outer, r, inner)
            ref = ops.empty((outer * inner,), dtype)
            got = ops.empty((outer * inner,), dtype)
            assert lib.tp_amd_launch_reduce(0, op, dtype, outer, r, inner, dx.data_ptr,
                                            ref.data_ptr) == 0
            lib.tp_amd_synchronize(0)
            before = _stats(lib)
            rc = noalloc(0, op, dtype, outer, r, inner, dx.data_ptr, got.data_ptr)
            assert rc == 0, lib.tp_mlu_last_error()
            lib.tp_amd_synchronize(0)
            after = _stats(lib)
            assert after[:2] == before[:2], f"allocator counters moved: {before} -> {after}"
            what = f"call {call} op {op} {(outer, r, inner)}"
            assert_bitexact(got.numpy(), ref.numpy(), what)
            if op in (AMAX, AMIN):
                assert_bitexact(got.numpy(), want, what)
            else:
                mag = np.abs(orc.to_float(x, dtype).astype(np.float64)).sum(axis=1).reshape(-1)
                assert_sum(got.numpy(), want, dtype, what, r if op == MEAN else 1,
                           mag / r if op == MEAN else mag, r)


@pytest.mark.parametrize("outer,r,inner,dtype", [(1, 1 << 24, 1, F32), (1, 32768, 4096, F32),
                                                 (3, 2048, 384, BF16), (4096, 32000, 1, F32),
                                                 (7, 8192, 256, F32)],
                         ids=["whole-fp32", "cols-fp32", "cols-bf16", "rows-unsplit", "cols-7x256"])
def test_partials_query_matches_the_launch(amd, dev, ops, orc, outer, r, inner, dtype):
    """tp_amd_reduce_partial_bytes at this GPU's CU count is the workspace
    the allocating entry takes (the allocator's peak over the call, requests
    rounded to 512 B), and the allocation-free entry accepts every shape
    whose figure fits its static array -- on a 256-CU MI355X every shape
    does (tests/test_reduce_plan.py) -- with the same bits."""
    lib = amd.load()
    runtime = __import__("importlib").import_module("tensorplay-mlu_amd.runtime")
    cus = runtime.compute_units(0)
    want = lib.tp_amd_reduce_partial_bytes(cus, dtype, outer, r, inner)
    assert 0 <= want <= lib.tp_amd_reduce_noalloc_scratch_bytes()
    x = orc.from_float(np.random.default_rng(9).standard_normal((outer, r, inner)).astype(np.float32), dtype)
    dx = dev.from_numpy(x, dtype=dtype)
    ref = ops.empty((outer * inner,), dtype)
    got = ops.empty((outer * inner,), dtype)
    lib.tp_amd_synchronize(0)
    # no idle cached block may serve the workspace (the cache reuses a block
    # up to 1.25x the request and counts the block's size)
    lib.tp_mlu_empty_cache()
    lib.tp_mlu_reset_peak_memory_stats(0)
    before = _stats(lib)
    assert lib.tp_amd_launch_reduce(0, SUM, dtype, outer, r, inner, dx.data_ptr, ref.data_ptr) == 0
    lib.tp_amd_synchronize(0)
    after = _stats(lib)
    assert after[2] - before[0] == (want + 511) // 512 * 512, (before, after, want)
    assert lib.tp_amd_launch_reduce_noalloc(0, SUM, dtype, outer, r, inner, dx.data_ptr, got.data_ptr) == 0
    lib.tp_amd_synchronize(0)
    assert_bitexact(got.numpy(), ref.numpy(), f"{(outer, r, inner)}")
