"""The parity checkers themselves (CPU): each per-element bound admits a
correct float32 computation and rejects a result that is wrong on a single
non-maximal entry per row -- where the norm-wise rule of the reference's
tests (max |got - want| <= tol * 10 * max |want|) still passes.

The oracle supplies the reference values; the "kernels" here are numpy
float32 restatements (the positive controls) and the oracle's own output
with one entry per row perturbed (the negative controls)."""

import numpy as np
import pytest

from _check import (BF16, F32, as_float, assert_normwise, assert_softmax, assert_softmax_backward, assert_sum,
                    storage_ulp)


def _x(shape, std, seed=0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def _softmax32(x, log):
    d = x - x.max(axis=-1, keepdims=True)
    e = np.exp(d)
    s = e.sum(axis=-1, keepdims=True, dtype=np.float32)
    return (d - np.log(s)) if log else e * (np.float32(1) / s)


def _perturb_small(y, rel):
    """One entry per row -- the row's smallest, never its maximum --
    scaled by (1 + rel)."""
    out = y.copy()
    rows = np.arange(y.shape[0])
    cols = np.argmin(np.abs(y), axis=1)
    out[rows, cols] = out[rows, cols] * np.float32(1 + rel)
    return out


def _rejects(fn, *args):
    with pytest.raises(AssertionError):
        fn(*args)


@pytest.mark.parametrize("log", [False, True], ids=["softmax", "log_softmax"])
def test_softmax_bound_admits_float32_and_rejects_one_entry(orc, log):
    x = _x((64, 4096), 4.0)
    want = orc.softmax(log, F32, x, 64, 4096, 1)
    assert_softmax(_softmax32(x, log), want, F32, log, "float32 restatement")
    # log_softmax's smallest-magnitude entry is the row maximum's; perturb
    # the most negative one instead
    bad = _perturb_small(want, 0.01) if not log else want.copy()
    if log:
        cols = np.argmin(want, axis=1)
        bad[np.arange(64), cols] *= np.float32(1.01)
    _rejects(assert_softmax, bad, want, F32, log, "perturbed")
    if not log:
        assert_normwise(bad, want, F32, 1, "the norm-wise rule misses it")


def test_softmax_backward_bound(orc):
    x = _x((32, 8192), 2.0, 1)
    dy = _x((32, 8192), 1.0, 2)
    for log in (False, True):
        y = orc.softmax(log, F32, x, 32, 8192, 1)
        want = orc.softmax_backward(log, F32, y, dy, 32, 8192, 1)
        if log:
            s = dy.sum(axis=-1, keepdims=True, dtype=np.float32)
            got = dy - np.exp(y) * s
        else:
            s = (dy * y).sum(axis=-1, keepdims=True, dtype=np.float32)
            got = y * (dy - s)
        assert_softmax_backward(got, want, F32, log, y, dy, 32, 8192, 1, f"float32 restatement log={log}")
        # perturb, per row, an entry with a small output weight but a sizeable
        # upstream gradient
        bad = want.copy()
        score = np.where(np.abs(dy) > 0.5, np.abs(y if not log else np.exp(y)), np.inf)
        cols = np.argmin(score, axis=1)
        bad[np.arange(32), cols] *= np.float32(1.01)
        _rejects(assert_softmax_backward, bad, want, F32, log, y, dy, 32, 8192, 1, "perturbed")


def test_bf16_softmax_within_one_ulp(orc):
    x = orc.from_float(_x((16, 4096), 2.0, 3), BF16)
    want = orc.softmax(False, BF16, x, 16, 4096, 1)
    got = orc.from_float(_softmax32(as_float(x, BF16).astype(np.float32), False), BF16)
    assert_softmax(got, want, BF16, False, "float32 then rounded")
    bad = want.copy()
    wf = as_float(want, BF16)
    cols = np.argmin(wf, axis=1)
    bad[np.arange(16), cols] += np.uint16(2)  # two codes up: two ulps (positive values)
    _rejects(assert_softmax, bad, want, BF16, False, "two ulps off")


def test_bf16_sum_bound(orc):
    """Positive data, where sum|x| = |sum x|: the per-element bound is about
    one ulp, a result three codes off fails, and the float32 sum rounded
    once passes."""
    a = np.random.default_rng(4).uniform(0.5, 2.0, (64, 4096)).astype(np.float32)
    x = orc.from_float(a, BF16)
    xf = as_float(x, BF16).astype(np.float64)
    want = orc.reduce(0, BF16, x, 64, 4096, 1)
    mag = np.abs(xf).sum(axis=1)
    got = orc.from_float(xf.astype(np.float32).sum(axis=1, dtype=np.float32), BF16)
    assert_sum(got, want, BF16, "float32 sum", 1, mag, 4096)
    bad = want.copy()
    bad[5] += np.uint16(3)
    _rejects(assert_sum, bad, want, BF16, "three codes off", 1, mag, 4096)


def test_storage_ulp():
    w = np.array([1.0, 1.5, 2.0, -3.0, 0.0, 2.0 ** -130], np.float64)
    assert np.array_equal(storage_ulp(w, BF16), [2.0 ** -7, 2.0 ** -7, 2.0 ** -6, 2.0 ** -6, 2.0 ** -133,
                                                  2.0 ** -133])
