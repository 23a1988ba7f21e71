"""Comparison helpers with the tolerances the parity bar states.

* bit-exact: copies, casts, fills, relu, threshold_backward, amax/amin, and
  the single-operation float arithmetic (add/sub with alpha 1, mul, div,
  neg, abs): a float32 result of one correctly rounded operation equals
  the oracle's double result rounded to float32 (double has more than
  2 * 24 + 2 bits, so rounding twice is harmless), and the narrow dtypes
  then round that same float32 the same way.
* float32 elementwise transcendental results: |got - want| <= 1e-5 |want| + 1e-6
  (rtol 1e-5; the absolute floor covers results within 1e-6 of zero, where
  the device library's absolute error dominates).
* bfloat16 / float16 elementwise results: within one unit in the last place
  of the storage dtype (the float32 results may straddle a rounding
  midpoint differently).
* reductions and softmax: the reference test's norm-wise rule
  (tests/test_mlu.py:25-34): max |got - want| <= tol * 10 * max(max |want|, 1)
  * scale, tol = 1e-5 float32, 2e-3 float16, 2e-2 bfloat16 -- a per-element
  relative bound cannot hold for sums that cancel under a different
  summation order.
"""

from __future__ import annotations

import numpy as np

from oracle import binding as orc

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16
NORM_TOL = {F32: 1e-5, F16: 2e-3, BF16: 2e-2}


def as_float(x: np.ndarray, dtype: int) -> np.ndarray:
    return orc.to_float(x, dtype)


def assert_bitexact(got: np.ndarray, want: np.ndarray, what: str = "") -> None:
    assert got.shape == want.shape, (what, got.shape, want.shape)
    g = np.ascontiguousarray(got).view(np.uint8)
    w = np.ascontiguousarray(want).view(np.uint8)
    if not np.array_equal(g, w):
        bad = np.flatnonzero(np.ascontiguousarray(got).reshape(-1) != np.ascontiguousarray(want).reshape(-1))
        i = int(bad[0]) if bad.size else -1
        raise AssertionError(f"{what}: {bad.size} elements differ; first at {i}: "
                             f"got {got.reshape(-1)[i]!r} want {want.reshape(-1)[i]!r}")


def ulp_distance(got: np.ndarray, want: np.ndarray, dtype: int) -> np.ndarray:
    """Distance in units of the last place of the storage dtype (signed
    magnitudes mapped onto a monotone integer line)."""
    if dtype == F32:
        g = got.view(np.int32).astype(np.int64)
        w = want.view(np.int32).astype(np.int64)
        sign = np.int64(1 << 31)
    else:
        g = got.view(np.int16).astype(np.int64)
        w = want.view(np.int16).astype(np.int64)
        sign = np.int64(1 << 15)
    g = np.where(g < 0, -(g + sign), g)
    w = np.where(w < 0, -(w + sign), w)
    return np.abs(g - w)


def assert_elementwise(got: np.ndarray, want: np.ndarray, dtype: int, what: str = "",
                       max_ulp: int | None = None) -> None:
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if max_ulp is not None:
        d = ulp_distance(np.ascontiguousarray(got), np.ascontiguousarray(want), dtype)
        worst = int(d.max()) if d.size else 0
        assert worst <= max_ulp, f"{what}: {worst} ulp apart (allowed {max_ulp})"
        return
    g, w = as_float(got, dtype), as_float(want, dtype)
    if dtype == F32:
        bound = 1e-5 * np.abs(w) + 1e-6
        err = np.abs(g - w)
        bad = err > bound
        assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond rtol 1e-5; worst "
                               f"rel {float(np.max(err / (np.abs(w) + 1e-30))):.3g}")
    else:
        d = ulp_distance(np.ascontiguousarray(got), np.ascontiguousarray(want), dtype)
        worst = int(d.max()) if d.size else 0
        assert worst <= 1, f"{what}: {worst} ulp apart in the storage dtype"


def assert_normwise(got: np.ndarray, want: np.ndarray, dtype: int, scale: float = 1.0,
                    what: str = "") -> float:
    g, w = as_float(got, dtype), as_float(want, dtype)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    if g.size == 0:
        return 0.0
    err = float(np.max(np.abs(g - w)))
    ref = max(float(np.max(np.abs(w))), 1.0) * scale
    tol = NORM_TOL[dtype] * ref * 10
    assert err <= tol, f"{what}: max error {err} > tolerance {tol}"
    return err


def assert_sum(got: np.ndarray, want: np.ndarray, dtype: int, what: str = "", count: int = 1) -> float:
    """Sums and means: the kernels add in float32 and round once to the
    storage dtype, the oracle adds in float64 and rounds once, so the
    reference's norm-wise rule holds at scale 1.  A mean is compared on its
    sum's scale (both sides times ``count``, the number of reduced elements),
    where a 16-bit mean of zero-mean data is not lost under the rule's floor
    of 1.  The data must make the check able to fail: the tolerance has to
    sit below max |want|, so a result of zeros (or any result off by the
    whole answer) is caught."""
    g = as_float(got, dtype).astype(np.float64) * count
    w = as_float(want, dtype).astype(np.float64) * count
    assert g.shape == w.shape, (what, g.shape, w.shape)
    if w.size == 0:
        return 0.0
    peak = float(np.max(np.abs(w)))
    tol = NORM_TOL[dtype] * max(peak, 1.0) * 10
    assert np.isfinite(peak) and tol < peak, (
        f"{what}: tolerance {tol} >= max |want| {peak}; a zero result would pass -- use data "
        "with larger sums")
    err = float(np.max(np.abs(g - w)))
    assert err <= tol, f"{what}: max error {err} > tolerance {tol}"
    return err
