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
* softmax and log_softmax, forward and backward: per element
  (assert_softmax, assert_softmax_backward), with the bounds one float32
  pass over the row admits: softmax |got - want| <= 1e-5 |want| (+1e-30),
  log_softmax <= 1e-5 max(|want|, 1), the backward scaled by the terms
  that enter each element (see the functions); 16-bit storage adds one
  unit in the last place of the storage dtype.  A result that is right
  only on each row's largest entries fails.
* float32 sums and means: the reference test's norm-wise rule
  (tests/test_mlu.py:25-34): max |got - want| <= tol * 10 * max(max |want|, 1)
  with tol = 1e-5 -- a per-element relative bound cannot hold for sums that
  cancel under a different summation order.
* 16-bit sums and means: per element, n 2^-24 sum|x| + one storage ulp
  (float32 accumulation in any order of n terms, then one rounding on each
  side), and also the norm-wise rule (tol 2e-3 float16, 2e-2 bfloat16),
  which is the tighter of the two for very long reductions.
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


def assert_sum(got: np.ndarray, want: np.ndarray, dtype: int, what: str = "", count: int = 1,
               abs_sum: np.ndarray | None = None, terms: int | None = None) -> float:
    """Sums and means: the kernels add in float32 and round once to the
    storage dtype, the oracle adds in float64 and rounds once, so the
    reference's norm-wise rule holds at scale 1.  A mean is compared on its
    sum's scale (both sides times ``count``, the number of reduced elements),
    where a 16-bit mean of zero-mean data is not lost under the rule's floor
    of 1.  The data must make the check able to fail: the tolerance has to
    sit below max |want|, so a result of zeros (or any result off by the
    whole answer) is caught.

    16-bit results must also pass per element: |got - want| <= terms
    2^-24 abs_sum + one storage ulp of want (abs_sum: the sum of |x| over
    each output's terms, float64, want's shape; for a mean, the mean of
    |x| with terms = count)."""
    if dtype != F32:
        assert abs_sum is not None and terms is not None, f"{what}: 16-bit sums need abs_sum and terms"
        bound = (terms + 2) * 2.0 ** -24 * np.asarray(abs_sum, np.float64)
        assert_pointwise(got, want, dtype, bound, what + " (per element)")
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


def storage_ulp(want: np.ndarray, dtype: int) -> np.ndarray:
    """One unit in the last place of the 16-bit storage dtype at |want|
    (the subnormal spacing at and below the smallest normal)."""
    mant, emin = (7, -126) if dtype == BF16 else (10, -14)
    a = np.abs(np.asarray(want, np.float64))
    safe = np.where(np.isfinite(a) & (a > 0), a, 1.0)
    e = np.where(np.isfinite(a) & (a > 0), np.floor(np.log2(safe)), emin)
    e = np.maximum(e, emin)
    return np.ldexp(1.0, (e - mant).astype(np.int64))


def assert_pointwise(got: np.ndarray, want: np.ndarray, dtype: int, bound, what: str = "") -> None:
    """|got - want| <= bound element for element (bound broadcast to want's
    shape; 16-bit dtypes add one storage ulp of want).  Infinities must match
    in place and sign, NaN in place."""
    g = as_float(got, dtype).astype(np.float64)
    w = as_float(want, dtype).astype(np.float64)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    nan_g, nan_w = np.isnan(g), np.isnan(w)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN in {int(nan_g.sum())} places, expected {int(nan_w.sum())}"
    inf_w = np.isinf(w)
    assert np.array_equal(np.isinf(g), inf_w) and np.array_equal(g[inf_w], w[inf_w]), f"{what}: infinities differ"
    b = np.broadcast_to(np.asarray(bound, np.float64), w.shape)
    if dtype != F32:
        b = b + storage_ulp(w, dtype)
    fin = np.isfinite(w)
    with np.errstate(invalid="ignore"):
        err = np.where(fin, np.abs(g - w), 0.0)
    bad = err > b
    if bad.any():
        i = int(np.flatnonzero(bad.reshape(-1))[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements beyond the bound; first at {i}: "
                             f"got {g.reshape(-1)[i]!r} want {w.reshape(-1)[i]!r} bound {b.reshape(-1)[i]!r}")


def _rows(x: np.ndarray, dtype: int, outer: int, size: int, inner: int) -> np.ndarray:
    return as_float(x, dtype).astype(np.float64).reshape(outer, size, inner)


def assert_softmax(got: np.ndarray, want: np.ndarray, dtype: int, log: bool, what: str = "") -> None:
    """softmax: |got - want| <= 1e-5 |want| + 1e-30; log_softmax: <= 1e-5
    max(|want|, 1).  One float32 pass forms d = x - max (error u|d|), 2^(d
    log2 e) (|d| u plus the exp unit's few ulps), the row sum (relative error
    of its depth times u) and one reciprocal or log, all well inside 1e-5
    relative for |d| below 100; 16-bit storage adds one ulp (the float32
    value and the oracle's may round to neighbouring codes)."""
    w = np.abs(as_float(want, dtype).astype(np.float64))
    bound = 1e-5 * np.maximum(w, 1.0) if log else 1e-5 * w + 1e-30
    assert_pointwise(got, want, dtype, 0.0 if dtype != F32 else bound, what)


def assert_softmax_backward(got: np.ndarray, want: np.ndarray, dtype: int, log: bool, y: np.ndarray,
                            dy: np.ndarray, outer: int, size: int, inner: int, what: str = "") -> None:
    """Per element, with the row terms that enter it (sums over the softmax
    axis, float64): softmax dx = y (dy - s), s = sum(dy y), within
    1e-5 |y| (|dy| + |s| + sum|dy y|); log_softmax dx = dy - e^y s, s =
    sum(dy), within 1e-5 (|dy| + e^y (|s| + sum|dy|)).  The sum|.| term is
    the float32 error of s in any order; 16-bit storage adds one ulp."""
    yv, gv = _rows(y, dtype, outer, size, inner), _rows(dy, dtype, outer, size, inner)
    if log:
        s = gv.sum(axis=1, keepdims=True)
        a = np.abs(gv).sum(axis=1, keepdims=True)
        bound = 1e-5 * (np.abs(gv) + np.exp(yv) * (np.abs(s) + a)) + 1e-30
    else:
        s = (gv * yv).sum(axis=1, keepdims=True)
        a = np.abs(gv * yv).sum(axis=1, keepdims=True)
        bound = 1e-5 * np.abs(yv) * (np.abs(gv) + np.abs(s) + a) + 1e-30
    assert_pointwise(got, want, dtype, bound.reshape(np.shape(want)), what)
