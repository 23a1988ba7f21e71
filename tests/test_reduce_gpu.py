"""Reductions and softmax on the GPU against the CPU oracle: the
reference's cases (tests/test_mlu.py:303-350) and config 3 of the benchmark
at full size.  amax/amin are bit-exact; float32 sums and means use the
reference's norm-wise rule, 16-bit ones also a per-element bound, and
softmax and its backward per-element bounds (tests/_check.py)."""

import numpy as np
import pytest

from _check import (BF16, F16, F32, as_float, assert_bitexact, assert_softmax, assert_softmax_backward,
                    assert_sum)

pytestmark = pytest.mark.gpu

DTYPES = [F32, F16, BF16]
SUM, MEAN, AMAX, AMIN = 0, 1, 2, 3


def sample(orc, shape, dtype, seed=0, std=1.0, mean=0.0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * np.float32(std)
    return orc.from_float(x + np.float32(mean), dtype)


def oracle_reduce(orc, op, dtype, x, dims, keepdim=False):
    """Reduce over ``dims`` one run at a time with the oracle (float32
    intermediates when the runs are not adjacent)."""
    nd = x.ndim
    dims = sorted(d % nd for d in (dims if dims else range(nd)))
    shape = list(x.shape)
    runs = []
    for d in dims:
        if runs and runs[-1][1] == d - 1:
            runs[-1][1] = d
        else:
            runs.append([d, d])
    cur, cur_dtype = x, dtype
    if len(runs) > 1:
        cur, cur_dtype = orc.to_float(x, dtype).astype(np.float32), F32
    for first, last in reversed(runs):
        outer = int(np.prod(shape[:first]))
        r = int(np.prod(shape[first:last + 1]))
        inner = int(np.prod(shape[last + 1:]))
        cur = orc.reduce(op, cur_dtype, cur, outer, r, inner)
        for d in range(first, last + 1):
            shape[d] = 1
        cur = cur.reshape(shape)
    if len(runs) > 1:
        cur = orc.from_float(cur, dtype)
    if not keepdim:
        cur = cur.reshape([s for i, s in enumerate(x.shape) if i not in dims])
    return cur


def check_sum(got, want, dtype, what, a, dims, mean=False, keepdim=False, mask=None):
    """assert_sum with the per-element terms of a reduction of ``a`` over
    ``dims`` (None or [] = all): the count of terms and the sum (or, for a
    mean, the mean) of |x| per output; ``mask`` selects outputs."""
    nd = a.ndim
    axes = tuple(sorted(d % nd for d in (dims if dims else range(nd))))
    n = int(np.prod([a.shape[d] for d in axes])) if axes else 1
    x = np.abs(as_float(a, dtype).astype(np.float64)).sum(axis=axes, keepdims=keepdim)
    x = x / n if mean else x
    if mask is not None:
        x = x[mask]
    return assert_sum(got, want, dtype, what, n if mean else 1, x, n)


@pytest.mark.parametrize("dtype", DTYPES)
def test_reductions(dev, ops, orc, dtype):
    # a mean of 2 keeps every sum and mean well clear of the tolerance
    a = sample(orc, (6, 7, 8), dtype, mean=2.0)
    d = dev.from_numpy(a, dtype=dtype)
    check_sum(ops.sum(d).numpy(), oracle_reduce(orc, SUM, dtype, a, None), dtype, "sum", a, None)
    check_sum(ops.sum_dim(d, 1).numpy(), oracle_reduce(orc, SUM, dtype, a, [1]), dtype, "sum dim 1", a, [1])
    got = ops.sum_dim(d, (0, 2), keepdim=True).numpy()
    assert got.shape == (1, 7, 1)
    check_sum(got, oracle_reduce(orc, SUM, dtype, a, [0, 2], True), dtype, "sum (0, 2)", a, [0, 2],
              keepdim=True)
    check_sum(ops.mean(d).numpy(), oracle_reduce(orc, MEAN, dtype, a, None), dtype, "mean", a, None, True)
    check_sum(ops.mean_dim(d, -1).numpy(), oracle_reduce(orc, MEAN, dtype, a, [2]), dtype,
              "mean dim -1", a, [2], True)
    for op, fn in ((AMAX, ops.amax), (AMIN, ops.amin)):
        for dims in ([0], [1], [-1], [0, 2], []):
            assert_bitexact(fn(d, dims).numpy(), oracle_reduce(orc, op, dtype, a, dims),
                            f"amax/amin {dims}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(5, 2048, 384), (2, 8192, 3), (3, 700, 1000)],
                         ids=["outer5-packets", "outer2-scalar", "outer3-ragged"])
def test_column_reduction_row_chunks(dev, ops, orc, dtype, shape):
    """Reductions over a middle axis long enough to be split into row chunks,
    whose partials the last block of each column range folds: several outer
    indices, a width that takes 16-byte packets, one that does not, and rows
    that do not divide evenly.  Each reduction runs twice, so an arrival
    counter left non-zero by the first launch would corrupt the second."""
    a = sample(orc, shape, dtype, 3, mean=1.0)
    a[0, 5, 1] = orc.from_float(np.array([np.nan], np.float32), dtype)[0]
    d = dev.from_numpy(a, dtype=dtype)
    for op, fn in ((SUM, ops.sum_dim), (MEAN, ops.mean_dim), (AMAX, ops.amax), (AMIN, ops.amin)):
        want = oracle_reduce(orc, op, dtype, a, [1])
        for rep in range(2):
            got = fn(d, [1]).numpy()
            if op in (AMAX, AMIN):
                assert_bitexact(got, want, f"op {op} run {rep}")
            else:
                assert np.array_equal(np.isnan(orc.to_float(got, dtype)), np.isnan(orc.to_float(want, dtype)))
                ok = ~np.isnan(orc.to_float(want, dtype))
                check_sum(got[ok], want[ok], dtype, f"op {op} run {rep}", a, [1], op == MEAN, mask=ok)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1 << 24,), ((1 << 24) + 3,), (3, 1000003), (7, 65536)],
                         ids=["2^24", "2^24+3-scalar", "3-rows-ragged", "7-rows"])
def test_few_long_rows_folded_in_one_launch(dev, ops, orc, dtype, shape):
    """Few long rows (a whole-tensor reduction, a loss over all logits) are
    split into one-block segments, and the last block of each row folds the
    row's partials in the same launch: a whole 2^24-element tensor with
    16-byte packets, a ragged length read element by element, three and
    seven rows.  Every reduction runs twice, so an arrival counter left
    non-zero by the first launch would corrupt the second; amax/amin also see
    a NaN, which they skip."""
    # float16 sums of 2^24 elements stay below its largest finite value
    a = sample(orc, shape, dtype, 4, mean=0.002 if dtype == F16 else 0.5)
    d = dev.from_numpy(a, dtype=dtype)
    dims = None if len(shape) == 1 else [-1]
    for op, fn in ((SUM, ops.sum), (MEAN, ops.mean)):
        want = oracle_reduce(orc, op, dtype, a, dims)
        for rep in range(2):
            got = (fn(d) if dims is None else (ops.sum_dim if op == SUM else ops.mean_dim)(d, dims)).numpy()
            check_sum(got, want, dtype, f"op {op} {shape} run {rep}", a, dims, op == MEAN)
    b = a.copy()
    b.reshape(-1)[shape[-1] // 3] = orc.from_float(np.array([np.nan], np.float32), dtype)[0]
    db = dev.from_numpy(b, dtype=dtype)
    for op, fn in ((AMAX, ops.amax), (AMIN, ops.amin)):
        want = oracle_reduce(orc, op, dtype, b, dims)
        for rep in range(2):
            got = fn(db, [] if dims is None else dims).numpy()
            assert_bitexact(got, want, f"op {op} {shape} run {rep}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_long_reductions(dev, ops, orc, dtype):
    # float16 sums of 131072 elements stay below its largest finite value
    m = 0.25 if dtype == F16 else 1.0
    for shape in ((2, 4096), (2, 65536), (16, 8192), (3, 32768), (4096, 2)):
        a = sample(orc, shape, dtype, mean=m)
        d = dev.from_numpy(a, dtype=dtype)
        check_sum(ops.sum(d).numpy(), oracle_reduce(orc, SUM, dtype, a, None), dtype, f"sum {shape}", a, None)
        check_sum(ops.mean(d).numpy(), oracle_reduce(orc, MEAN, dtype, a, None), dtype, f"mean {shape}",
                  a, None, True)
        check_sum(ops.sum_dim(d, 1).numpy(), oracle_reduce(orc, SUM, dtype, a, [1]), dtype,
                  f"sum dim 1 {shape}", a, [1])
        check_sum(ops.mean_dim(d, 0).numpy(), oracle_reduce(orc, MEAN, dtype, a, [0]), dtype,
                  f"mean dim 0 {shape}", a, [0], True)
        assert_bitexact(ops.amax(d, 0).numpy(), oracle_reduce(orc, AMAX, dtype, a, [0]), "amax 0")
    a = sample(orc, (65537,), dtype, mean=m)
    d = dev.from_numpy(a, dtype=dtype)
    check_sum(ops.sum(d).numpy(), oracle_reduce(orc, SUM, dtype, a, None), dtype, "sum 65537", a, None)
    assert_bitexact(ops.amin(d).numpy(), oracle_reduce(orc, AMIN, dtype, a, None), "amin all")
    a = sample(orc, (2, 4096, 2), dtype, mean=m)
    d = dev.from_numpy(a, dtype=dtype)
    check_sum(ops.sum_dim(d, 1).numpy(), oracle_reduce(orc, SUM, dtype, a, [1]), dtype, "sum mid", a, [1])
    check_sum(ops.mean_dim(d, 1).numpy(), oracle_reduce(orc, MEAN, dtype, a, [1]), dtype, "mean mid", a, [1],
              True)
    a = sample(orc, (16, 8192), dtype)
    d = dev.from_numpy(a, dtype=dtype)
    assert_bitexact(ops.amax(d, -1).numpy(), oracle_reduce(orc, AMAX, dtype, a, [-1]), "amax -1")
    assert_bitexact(ops.amin(d, -1).numpy(), oracle_reduce(orc, AMIN, dtype, a, [-1]), "amin -1")


def test_reduction_edge_cases(dev, ops, orc):
    # signed zeros and NaN: amax/amin skip NaN and order -0 below +0
    x = np.array([[0.0, -0.0, np.nan], [-0.0, -0.0, np.nan], [np.nan, np.nan, np.nan],
                  [1.0, np.nan, -2.0]], np.float32)
    d = dev.from_numpy(x)
    for op, fn in ((AMAX, ops.amax), (AMIN, ops.amin)):
        got = fn(d, [1]).numpy()
        want = orc.reduce(op, F32, x, 4, 3, 1)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        assert_bitexact(got[ok], want[ok], "signed zero / NaN")
    # an empty reduced axis gives zeros (ReduceKernels.cpp:72-73)
    e = dev.from_numpy(np.zeros((3, 0), np.float32))
    assert_bitexact(ops.sum_dim(e, 1).numpy(), np.zeros(3, np.float32), "empty sum")
    # a 0-d tensor reduces to itself
    s = dev.from_numpy(np.array(2.5, np.float32))
    assert ops.item(ops.sum(s)) == 2.5


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", [0, 1])
def test_amax_amin_nan_and_signed_zero_vectorised(dev, ops, orc, dtype, dim):
    """The packet paths of both reduction kernels (rows and columns) with NaN,
    all-NaN, signed-zero and all-negative lines mixed into random data."""
    g = np.random.default_rng(11)
    x = g.standard_normal((96, 4096)).astype(np.float32)
    x[3, 17] = np.nan                       # one NaN among numbers
    x[5, :] = np.nan                        # all NaN
    x[7, :] = -0.0                          # only -0
    x[9, :] = 0.0
    x[9, ::2] = -0.0                        # -0 and +0 mixed
    x[11, :] = -np.abs(x[11, :]) - 1.0      # all negative
    x[13, g.integers(0, 4096, 64)] = np.nan
    x[:, 21] = np.nan                       # a NaN column
    x[:, 23] = -0.0
    x[:, 25] = 0.0
    x[::3, 25] = -0.0
    x[:, 27] = np.nan
    x[40, 27] = -5.0                        # a single number in a NaN column
    a = orc.from_float(x, dtype)
    d = dev.from_numpy(a, dtype=dtype)
    for op, fn in ((AMAX, ops.amax), (AMIN, ops.amin)):
        got = fn(d, [dim]).numpy()
        want = oracle_reduce(orc, op, dtype, a, [dim])
        gf, wf = orc.to_float(got, dtype), orc.to_float(want, dtype)
        assert np.array_equal(np.isnan(gf), np.isnan(wf)), (op, dim)
        ok = ~np.isnan(wf)
        assert_bitexact(got[ok], want[ok], f"op {op} dim {dim}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_reductions_of_permuted_views(dev, ops, orc, dtype):
    """A transposed or permuted view of a dense tensor is reduced where it
    lies, its dims in memory order; the result comes back in logical order
    (reordered when its kept dims lie out of order).  Sums at the sum
    tolerance, amax / amin bit-exact."""
    a = sample(orc, (64, 96), dtype, 11)
    d = dev.from_numpy(a, dtype=dtype)
    at = np.ascontiguousarray(a.T)
    for dims in ([0], [1], None):
        check_sum(ops.sum_dim(d.t(), dims or []).numpy() if dims else ops.sum(d.t()).numpy(),
                  oracle_reduce(orc, SUM, dtype, at, dims), dtype, f"sum of .t() over {dims}", at, dims)
    assert_bitexact(ops.amax(d.t(), [0]).numpy(), oracle_reduce(orc, AMAX, dtype, at, [0]), "amax of .t()")
    b = sample(orc, (6, 40, 24), dtype, 12)
    db = dev.from_numpy(b, dtype=dtype)
    perm = db._view([24, 6, 40], [1, 960, 24])      # b.transpose(2, 0, 1), no copy
    bp = np.ascontiguousarray(np.transpose(b, (2, 0, 1)))
    check_sum(ops.sum_dim(perm, [1]).numpy(), oracle_reduce(orc, SUM, dtype, bp, [1]), dtype,
              "sum over dim 1 of a permutation (kept dims reordered)", bp, [1])
    got = ops.sum_dim(perm, [0, 2], keepdim=True).numpy()
    check_sum(got, oracle_reduce(orc, SUM, dtype, bp, [0, 2], True), dtype, "sum (0, 2) of a permutation",
              bp, [0, 2], keepdim=True)
    assert_bitexact(ops.amin(perm, [2]).numpy(), oracle_reduce(orc, AMIN, dtype, bp, [2]), "amin of a permutation")


def special_rows():
    """Rows of 37 normal values with every ordered pair of special values
    placed in two slots (signed zeros, infinities, NaN, the float32 and
    float16 extremes, float32 subnormals), and rows made only of NaN, -inf,
    +inf, -0 or +0."""
    sp = np.float32([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-40, -1e-40,
                     65504.0, -65504.0, 2.5])
    rng = np.random.default_rng(0)
    rows = []
    for u in sp:
        for v in sp:
            r = rng.standard_normal(37).astype(np.float32)
            r[5], r[17] = u, v
            rows.append(r)
    rows += [np.full(37, c, np.float32) for c in (np.nan, -np.inf, np.inf, -0.0, 0.0)]
    return np.stack(rows)


def same_special(got, want, dtype, what, exact, tol=None):
    """NaN where the oracle has NaN, infinities equal; the rest equal with
    the sign of zero (exact) or within ``tol`` (per element)."""
    g, w = as_float(got, dtype).reshape(-1), as_float(want, dtype).reshape(-1)
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(g), nan), f"{what}: NaN in other places"
    inf = np.isinf(w)
    assert np.array_equal(g[inf], w[inf]), f"{what}: infinities differ"
    fin = ~nan & ~inf
    if exact:
        assert np.array_equal(g[fin], w[fin]) and np.array_equal(np.signbit(g[fin]), np.signbit(w[fin])), what
    else:
        bad = np.abs(g[fin] - w[fin]) > tol.reshape(-1)[fin]
        assert not bad.any(), f"{what}: {int(bad.sum())} beyond the bound"


@pytest.mark.parametrize("dtype", DTYPES)
def test_reductions_and_softmax_special_values(dev, ops, orc, dtype):
    """Reductions over rows and over columns, and softmax / log_softmax over
    either axis, of lines holding special values: NaN, infinities and signed
    zeros as the oracle has them (amax/amin bit-exact), sums within the
    float32 error of their terms.  A mean whose float32 sum overflows (two
    3.4e38 terms) is left out: the device sums in float32 and gives +-inf,
    the oracle in float64 a finite mean."""
    with np.errstate(over="ignore"):
        a = orc.from_float(special_rows(), dtype)
    R, C = a.shape
    x = as_float(a, dtype).astype(np.float64)
    with np.errstate(invalid="ignore"):
        exact = x.sum(axis=1)
        ab = np.nan_to_num(np.abs(x).sum(axis=1), posinf=0.0)
        over = np.abs(exact) > 3.4028234e38
    d = dev.from_numpy(a, dtype=dtype)
    sum_tol = 1e-2 * np.maximum(np.abs(np.nan_to_num(exact, posinf=0, neginf=0)), 1.0) + 4e-6 * ab
    same_special(ops.sum_dim(d, [1]).numpy(), orc.reduce(SUM, dtype, a, R, C, 1), dtype, "sum rows", False, sum_tol)
    mean = ops.mean_dim(d, [1]).numpy()
    want = orc.reduce(MEAN, dtype, a, R, C, 1)
    same_special(mean[~over], want[~over], dtype, "mean rows", False, sum_tol[~over] / C)
    for op, fn in ((AMAX, ops.amax), (AMIN, ops.amin)):
        same_special(fn(d, [1]).numpy(), orc.reduce(op, dtype, a, R, C, 1), dtype, f"op {op} rows", True)
    at = np.ascontiguousarray(a.T)
    dt = dev.from_numpy(at, dtype=dtype)
    same_special(ops.sum_dim(dt, [0]).numpy(), orc.reduce(SUM, dtype, at, 1, C, R), dtype, "sum columns", False,
                 sum_tol)
    for op, fn in ((AMAX, ops.amax), (AMIN, ops.amin)):
        same_special(fn(dt, [0]).numpy(), orc.reduce(op, dtype, at, 1, C, R), dtype, f"op {op} columns", True)
    for log in (False, True):
        fn = ops.log_softmax if log else ops.softmax
        for arr, dd, dim, lines in ((a, d, -1, (R, C, 1)), (at, dt, 0, (1, C, R))):
            got = fn(dd, dim).numpy()
            want = orc.softmax(log, dtype, arr, *lines)
            w = np.abs(as_float(want, dtype).astype(np.float64))
            tol = (1e-5 * np.maximum(w, 1.0) if log else 1e-5 * w + 1e-30) + (0 if dtype == F32 else 2 * w * 2.0 ** -8)
            same_special(got, want, dtype, f"softmax log={log} dim={dim}", False, tol)


# Shapes for softmax over dim 0 / 1 (inner > 1): one column tile of one
# slice; several tiles; few tiles over a long D, split into slices whose
# partials a second launch folds; an odd inner size; enough tiles for one
# fused launch.
SOFTMAX_SHAPES = [(5, 6, 7), (3, 90, 130), (300, 2, 130), (700, 3, 37), (64, 1000, 64)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", [0, 1, -1])
@pytest.mark.parametrize("shape", SOFTMAX_SHAPES, ids=["5x6x7", "3x90x130", "300x2x130", "700x3x37",
                                                       "64x1000x64"])
def test_softmax_and_log_softmax(dev, ops, orc, dtype, dim, shape):
    a = sample(orc, shape, dtype)
    if shape == (300, 2, 130):
        # -inf over half a column: over dim 0, whole slices of it hold only -inf
        a[:150, 1, 5] = orc.from_float(np.full(150, -np.inf, np.float32), dtype)
    d = dev.from_numpy(a, dtype=dtype)
    k = dim % 3
    outer, size, inner = int(np.prod(a.shape[:k])), a.shape[k], int(np.prod(a.shape[k + 1:]))
    for log, fn in ((False, ops.softmax), (True, ops.log_softmax)):
        y = fn(d, dim)
        want = orc.softmax(log, dtype, a, outer, size, inner)
        # log_softmax of -inf is -inf: the checker matches infinities in
        # place and sign, the finite entries per element
        yh = y.numpy()
        assert_softmax(yh, want, dtype, log, f"softmax log={log}")
        g = sample(orc, a.shape, dtype, 9)
        back = ops._log_softmax_backward_data if log else ops._softmax_backward_data
        got = back(dev.from_numpy(g, dtype=dtype), y, dim, dtype).numpy()
        assert_softmax_backward(got, orc.softmax_backward(log, dtype, yh, g, outer, size, inner), dtype, log,
                                yh, g, outer, size, inner, f"softmax backward log={log}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape,dim", [((3, 130), 0), ((2, 5, 70), 1), ((4, 300, 130), 0)],
                         ids=["3x130-dim0", "2x5x70-dim1", "4x300x130-dim0"])
def test_softmax_nan_over_a_leading_axis(dev, ops, orc, dtype, shape, dim):
    """A NaN makes its whole softmax line NaN, also over a leading axis
    where a wave's batch of rows can hold nothing but that NaN, masked rows
    and -inf: forward and backward, against the oracle (NaN in the same
    places, the rest per element)."""
    a = sample(orc, shape, dtype, 21)
    nan = orc.from_float(np.array([np.nan], np.float32), dtype)[0]
    ninf = orc.from_float(np.array([-np.inf], np.float32), dtype)[0]
    idx = [0] * len(shape)
    a[tuple(idx)] = nan                        # row 0 of column 0
    idx[-1] = 7
    a[tuple(idx)] = nan                        # a second column: NaN, the rest -inf
    sl = [slice(None)] * len(shape)
    sl[-1] = 7
    col = a[tuple(sl)]
    sel = [slice(None)] * col.ndim
    sel[dim] = slice(1, None)
    col[tuple(sel)] = ninf
    a[tuple(sl)] = col
    d = dev.from_numpy(a, dtype=dtype)
    k = dim % len(shape)
    outer, size, inner = int(np.prod(shape[:k])), shape[k], int(np.prod(shape[k + 1:]))
    g = sample(orc, shape, dtype, 22)
    for log in (False, True):
        y = (ops.log_softmax if log else ops.softmax)(d, dim)
        yh = y.numpy()
        want = orc.softmax(log, dtype, a, outer, size, inner)
        assert np.isnan(as_float(want, dtype)).sum() >= 2 * size
        assert_softmax(yh, want, dtype, log, f"forward log={log}")
        back = ops._log_softmax_backward_data if log else ops._softmax_backward_data
        got = back(dev.from_numpy(g, dtype=dtype), y, dim, dtype).numpy()
        assert_softmax_backward(got, orc.softmax_backward(log, dtype, yh, g, outer, size, inner), dtype, log,
                                yh, g, outer, size, inner, f"backward log={log}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape,dim", [((64, 1000), -1), ((40, 16400), -1), ((6, 70000), -1),
                                       ((300, 130), 0), ((5, 300, 70), 1)],
                         ids=["rows-1000", "rows-16400", "rows-70000", "300x130-dim0", "5x300x70-dim1"])
def test_softmax_subnormal_tails(dev, ops, orc, dtype, shape, dim):
    """Lines spanning 110 below their maximum: entries 88-103 below it have
    subnormal softmax values (float32's, and bfloat16's with the same
    exponent range), which every kernel must produce rather than 0 -- the
    bfloat16 bound is one ulp -- and log_softmax's backward takes e^y of
    them.  Row kernels (register-resident, walked by one block per CU, two
    reads) and column kernels."""
    x = np.random.default_rng(31).uniform(-110.0, 0.0, shape).astype(np.float32)
    a = orc.from_float(x, dtype)
    d = dev.from_numpy(a, dtype=dtype)
    k = dim % len(shape)
    outer, size, inner = int(np.prod(shape[:k])), shape[k], int(np.prod(shape[k + 1:]))
    g = sample(orc, shape, dtype, 32)
    for log in (False, True):
        y = (ops.log_softmax if log else ops.softmax)(d, dim)
        yh = y.numpy()
        want = orc.softmax(log, dtype, a, outer, size, inner)
        if not log:
            tiny = (as_float(want, dtype) > 0) & (as_float(want, dtype) < 1.17549435e-38)
            assert tiny.sum() > 0, "the data must produce subnormal softmax values"
        assert_softmax(yh, want, dtype, log, f"forward log={log}")
        back = ops._log_softmax_backward_data if log else ops._softmax_backward_data
        got = back(dev.from_numpy(g, dtype=dtype), y, dim, dtype).numpy()
        assert_softmax_backward(got, orc.softmax_backward(log, dtype, yh, g, outer, size, inner), dtype, log,
                                yh, g, outer, size, inner, f"backward log={log}")


@pytest.mark.parametrize("D", [1, 7, 64, 256, 1000, 1024, 4096, 4100, 16384, 32000, 65536, 70000])
def test_softmax_row_lengths(dev, ops, orc, D):
    # every register-resident configuration and the two-read fallback
    rows = max(1, min(64, (1 << 22) // D))
    for dtype in (F32, BF16):
        a = sample(orc, (rows, D), dtype, 1, 3.0)
        d = dev.from_numpy(a, dtype=dtype)
        for log in (False, True):
            y = (ops.log_softmax if log else ops.softmax)(d, -1)
            yh = y.numpy()
            assert_softmax(yh, orc.softmax(log, dtype, a, rows, D, 1), dtype, log, f"D={D} log={log}")
            g = sample(orc, (rows, D), dtype, 2)
            back = ops._log_softmax_backward_data if log else ops._softmax_backward_data
            got = back(dev.from_numpy(g, dtype=dtype), y, -1, dtype).numpy()
            assert_softmax_backward(got, orc.softmax_backward(log, dtype, yh, g, rows, D, 1), dtype, log,
                                    yh, g, rows, D, 1, f"backward D={D} log={log}")


@pytest.mark.parametrize("rows,D,dtype", [(600, 8200, F32), (1000, 20000, F32), (257, 32000, F32),
                                          (600, 16400, BF16), (513, 30000, BF16)])
def test_softmax_rows_walked_by_one_block_per_cu(dev, ops, orc, rows, D, dtype):
    """Rows needing a 16-wave block are walked by a grid of one block per CU
    with the next row prefetched: more rows than CUs, odd row counts."""
    a = sample(orc, (rows, D), dtype, 5, 3.0)
    d = dev.from_numpy(a, dtype=dtype)
    for log in (False, True):
        y = (ops.log_softmax if log else ops.softmax)(d, -1)
        assert_softmax(y.numpy(), orc.softmax(log, dtype, a, rows, D, 1), dtype, log,
                       f"rows={rows} D={D} log={log}")


def test_softmax_declines(dev, ops, orc):
    tensor = __import__("importlib").import_module("tensorplay-mlu_amd.tensor")
    a = dev.from_numpy(sample(orc, (4, 5), F32))
    with pytest.raises(tensor.DeclinedError):
        ops._softmax(a, -1, True)  # half_to_float goes to the host (:202)
    y = ops.softmax(a, -1)
    with pytest.raises(tensor.DeclinedError):
        ops._softmax_backward_data(a, y, -1, BF16)


# ---- benchmark config 3 at full size ---------------------------------------------


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape,std", [((32768, 4096), 2.0), ((4096, 32000), 4.0)],
                         ids=["32768x4096", "4096x32000"])
def test_config3_full_size(dev, ops, orc, dtype, shape, std):
    a = sample(orc, shape, dtype, 0, std)
    d = dev.from_numpy(a, dtype=dtype)
    R, C = shape
    for dim, (outer, r, inner) in ((-1, (R, C, 1)), (0, (1, R, C))):
        check_sum(ops.sum_dim(d, dim).numpy(), orc.reduce(SUM, dtype, a, outer, r, inner),
                  dtype, f"sum dim {dim}", a, [dim])
        check_sum(ops.mean_dim(d, dim).numpy(), orc.reduce(MEAN, dtype, a, outer, r, inner),
                  dtype, f"mean dim {dim}", a, [dim], True)
        assert_bitexact(ops.amax(d, dim).numpy(), orc.reduce(AMAX, dtype, a, outer, r, inner),
                        f"amax dim {dim}")
        assert_bitexact(ops.amin(d, dim).numpy(), orc.reduce(AMIN, dtype, a, outer, r, inner),
                        f"amin dim {dim}")
    g = sample(orc, shape, dtype, 1)
    dg = dev.from_numpy(g, dtype=dtype)
    for log in (False, True):
        y = (ops.log_softmax if log else ops.softmax)(d, -1)
        yh = y.numpy()
        assert_softmax(yh, orc.softmax(log, dtype, a, R, C, 1), dtype, log, f"softmax log={log}")
        back = ops._log_softmax_backward_data if log else ops._softmax_backward_data
        assert_softmax_backward(back(dg, y, -1, dtype).numpy(), orc.softmax_backward(log, dtype, yh, g, R, C, 1),
                                dtype, log, yh, g, R, C, 1, f"softmax backward log={log}")
