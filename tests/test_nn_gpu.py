"""Neural-network layers on the GPU against the CPU oracle, through the
operator C-ABI (tp_amd_native_layer_norm, tp_amd_native_dropout,
tp_amd_embedding, tp_amd_nll_loss and their backwards; the reference's
NNKernels.cpp:57-395).

Tolerances: the dropout mask and the embedding lookup are bit-exact (a
mask decided by exact integer comparison, a row copy); the other results
are float sums whose order differs from the oracle's, so they use the
norm-wise rule of tests/_check.py (max |got - want| <= tol * 10 *
max(max |want|, 1), tol 1e-5 float32, 2e-3 float16, 2e-2 bfloat16); the
kept dropout values are within 1e-5 relative (float32) or one unit in the
last place (16-bit).
"""

import importlib

import numpy as np
import pytest

from _check import (BF16, F16, F32, as_float, assert_bitexact, assert_elementwise, assert_normwise,
                    assert_pointwise)

pytestmark = pytest.mark.gpu

DTYPES = [F32, F16, BF16]
IDS = ["fp32", "fp16", "bf16"]


def tensor_mod():
    return importlib.import_module("tensorplay-mlu_amd.tensor")


def sample(orc, shape, dtype, seed=0, std=1.0, shift=0.0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    return orc.from_float(x * np.float32(std) + np.float32(shift), dtype)


# ---- layer norm ------------------------------------------------------------------

LN_CASES = [
    ((4, 16), (16,)),            # the reference test's case (tests/test_mlu.py:951)
    ((3, 5, 24), (5, 24)),       # two normalized dimensions
    ((300, 1024), (1024,)),      # packet rows, one wave
    ((64, 4096), (4096,)),       # several waves per row
    ((9, 1001), (1001,)),        # width not a whole number of packets
    ((37, 12288), (12288,)),     # sixteen waves a row, the widest register layouts
    ((2, 40000), (40000,)),      # a row longer than the register-resident kernel holds
    ((300, 9000), (9000,)),      # the backward's generic dW/dB pass over four row slices
]
LN_IDS = ["4x16", "3x5x24", "300x1024", "64x4096", "9x1001", "37x12288", "2x40000", "300x9000"]


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("shape,norm", LN_CASES, ids=LN_IDS)
def test_layer_norm_forward(dev, ops, orc, dtype, shape, norm):
    D = int(np.prod(norm))
    x = sample(orc, shape, dtype, 1, 2.0, 0.5)
    w = sample(orc, norm, dtype, 2)
    b = sample(orc, norm, dtype, 3)
    for affine in (True, False):
        args = (dev.from_numpy(w, dtype=dtype), dev.from_numpy(b, dtype=dtype)) if affine else (None, None)
        y, mean, rstd = ops.native_layer_norm(dev.from_numpy(x, dtype=dtype), norm, *args, eps=1e-5)
        wy, wm, wr = orc.layer_norm(dtype, x, D, w if affine else None, b if affine else None, 1e-5)
        assert y.shape == shape and mean.shape == (x.size // D,) and rstd.shape == mean.shape
        what = f"{shape} affine={affine}"
        assert_normwise(y.numpy(), wy, dtype, 1, "y " + what)
        assert_normwise(mean.numpy(), wm, F32, 1, "mean " + what)
        assert_normwise(rstd.numpy(), wr, F32, 1, "rstd " + what)


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("shape,norm", LN_CASES, ids=LN_IDS)
def test_layer_norm_backward(dev, ops, orc, dtype, shape, norm):
    D = int(np.prod(norm))
    rows = int(np.prod(shape)) // D
    x = sample(orc, shape, dtype, 4, 1.5, -0.25)
    w = sample(orc, norm, dtype, 5)
    b = sample(orc, norm, dtype, 6)
    dy = sample(orc, shape, dtype, 7)
    dx_, w_, b_ = (dev.from_numpy(a, dtype=dtype) for a in (x, w, b))
    _, mean, rstd = ops.native_layer_norm(dx_, norm, w_, b_, eps=1e-5)
    m, r = mean.numpy(), rstd.numpy()
    gx, gw, gb = ops.native_layer_norm_backward(dev.from_numpy(dy, dtype=dtype), dx_, norm, mean,
                                                rstd, w_, b_)
    ox, ow, ob = orc.layer_norm_backward(dtype, dy, x, D, m, r, w)
    assert gx.shape == shape and gw.shape == tuple(norm) and gb.shape == tuple(norm)
    assert_normwise(gx.numpy(), ox, dtype, 1, "dx")
    # dW and dB sum over the rows
    scale = max(1.0, np.sqrt(rows))
    assert_normwise(gw.numpy().reshape(-1), ow, dtype, scale, "dweight")
    assert_normwise(gb.numpy().reshape(-1), ob, dtype, scale, "dbias")
    # without a weight, and with outputs masked off
    gx2, gw2, gb2 = ops.native_layer_norm_backward(dev.from_numpy(dy, dtype=dtype), dx_, norm, mean,
                                                   rstd, None, None, (True, False, True))
    assert gw2 is None
    ox2, _, ob2 = orc.layer_norm_backward(dtype, dy, x, D, m, r, None)
    assert_normwise(gx2.numpy(), ox2, dtype, 1, "dx without weight")
    assert_normwise(gb2.numpy().reshape(-1), ob2, dtype, scale, "dbias without weight")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
def test_layer_norm_bench_shape(dev, ops, orc, dtype):
    """[8192, 4096], the shape bench.py times: every CU holds a block of the
    backward's rows kernel, so the fold adds 256 partial rows a column (its
    full 16-load batches), which the smaller cases above never reach."""
    shape, norm, D = (8192, 4096), (4096,), 4096
    x = sample(orc, shape, dtype, 11, 1.5, -0.25)
    w = sample(orc, norm, dtype, 12)
    b = sample(orc, norm, dtype, 13)
    dy = sample(orc, shape, dtype, 14)
    dx_, w_, b_ = (dev.from_numpy(a, dtype=dtype) for a in (x, w, b))
    y, mean, rstd = ops.native_layer_norm(dx_, norm, w_, b_, eps=1e-5)
    wy, _, _ = orc.layer_norm(dtype, x, D, w, b, 1e-5)
    assert_normwise(y.numpy(), wy, dtype, 1, "y")
    m, r = mean.numpy(), rstd.numpy()
    gx, gw, gb = ops.native_layer_norm_backward(dev.from_numpy(dy, dtype=dtype), dx_, norm, mean,
                                                rstd, w_, b_)
    ox, ow, ob = orc.layer_norm_backward(dtype, dy, x, D, m, r, w)
    assert_normwise(gx.numpy(), ox, dtype, 1, "dx")
    scale = float(np.sqrt(shape[0]))
    assert_normwise(gw.numpy(), ow, dtype, scale, "dweight")
    assert_normwise(gb.numpy(), ob, dtype, scale, "dbias")
    # Per column: a float32 sum of `rows` terms is within (rows + 2) u sum|term|
    # of the exact sum (u = 2^-24), plus 3 u per term for xhat and the product.
    xf = as_float(x, dtype).astype(np.float64)
    dyf = as_float(dy, dtype).astype(np.float64)
    xhat = (xf - m.astype(np.float64)[:, None]) * r.astype(np.float64)[:, None]
    u, rows = 2.0 ** -24, shape[0]
    assert_pointwise(gw.numpy(), ow, dtype, (rows + 5) * u * np.abs(dyf * xhat).sum(axis=0), "dweight per column")
    assert_pointwise(gb.numpy(), ob, dtype, (rows + 2) * u * np.abs(dyf).sum(axis=0), "dbias per column")


def test_layer_norm_strided_input_and_declines(dev, ops, orc):
    a = sample(orc, (48, 32), F32, 8)
    t = dev.from_numpy(a).t()  # [32, 48] view, not contiguous
    y, mean, rstd = ops.native_layer_norm(t, (48,))
    wy, _, _ = orc.layer_norm(F32, np.ascontiguousarray(a.T), 48)
    assert_normwise(y.numpy(), wy, F32, 1, "transposed input")
    DeclinedError = tensor_mod().DeclinedError
    with pytest.raises(DeclinedError):
        ops.native_layer_norm(dev.from_numpy(a), (48, 32))  # no outer dimension (:64)
    with pytest.raises(DeclinedError):
        ops.native_layer_norm(dev.from_numpy(a), (31,))  # shape mismatch (:67-68)
    with pytest.raises(DeclinedError):
        ops.native_layer_norm(dev.from_numpy(a.astype(np.float64)), (32,))  # not a native float


# ---- dropout ---------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_dropout_matches_the_philox_stream(dev, ops, orc, dtype, p):
    n = (1 << 20) + 3
    x = sample(orc, (n,), dtype, 9)
    seed = 0x5DEECE66D1234567
    out, mask = ops.native_dropout(dev.from_numpy(x, dtype=dtype), p, True, seed)
    wout, wmask = orc.dropout(dtype, x, p, seed, 0)
    got_mask = mask.numpy()
    assert got_mask.dtype == np.bool_
    assert_bitexact(got_mask.astype(np.uint8), wmask, f"mask p={p}")
    got = out.numpy()
    keep = wmask.astype(bool)
    assert_elementwise(got[keep], wout[keep], dtype, f"kept p={p}")
    assert not got[~keep].view(np.uint8).any(), "dropped elements must be +0"


def test_dropout_shapes_modes_and_backward(dev, ops, orc):
    a = sample(orc, (37, 29), F32, 10)
    d = dev.from_numpy(a)
    # not training: the input unchanged, every element kept
    out, mask = ops.native_dropout(d, 0.3, False, 1)
    assert_bitexact(out.numpy(), a, "eval")
    assert mask.numpy().all()
    # p == 1 drops everything
    out, mask = ops.native_dropout(d, 1.0, True, 1)
    assert not out.numpy().any() and not mask.numpy().any()
    # a strided view keeps its shape; the stream follows the logical order
    t = d.t()
    out, mask = ops.native_dropout(t, 0.5, None, 77)
    wout, wmask = orc.dropout(F32, np.ascontiguousarray(a.T), 0.5, 77, 0)
    assert out.shape == (29, 37) and mask.shape == (29, 37)
    assert_bitexact(mask.numpy().astype(np.uint8), wmask, "strided mask")
    # backward: grad * mask * scale
    g = sample(orc, (29, 37), F32, 11)
    for dtype in DTYPES:
        gd = orc.from_float(orc.to_float(g, F32), dtype)
        got = ops.native_dropout_backward(dev.from_numpy(gd, dtype=dtype), mask, 2.0).numpy()
        want = orc.dropout_backward(dtype, gd, wmask, 2.0)
        assert_bitexact(got, want, f"dropout backward dtype {dtype}")


# ---- embedding -------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("dim", [768, 13], ids=["packets", "scalar"])
@pytest.mark.parametrize("itype", [np.int64, np.int32], ids=["i64", "i32"])
def test_embedding_lookup(dev, ops, orc, dtype, dim, itype):
    V = 1000
    w = sample(orc, (V, dim), dtype, 12)
    idx = np.random.default_rng(13).integers(0, V, size=(4, 33)).astype(itype)
    got = ops.embedding(dev.from_numpy(w, dtype=dtype), dev.from_numpy(idx)).numpy()
    assert got.shape == (4, 33, dim)
    assert_bitexact(got, orc.embedding(dtype, w, idx), "lookup")


def test_embedding_out_of_range_rows_are_nan(dev, ops, orc):
    w = sample(orc, (10, 64), F32, 14)
    idx = np.array([2, 10, -1, 9], np.int64)
    got = ops.embedding(dev.from_numpy(w), dev.from_numpy(idx)).numpy()
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all()
    assert_bitexact(got[[0, 3]], w[[2, 9]], "valid rows")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("pad,freq", [(-1, False), (3, False), (3, True)],
                         ids=["plain", "padding", "padding-freq"])
def test_embedding_dense_backward(dev, ops, orc, dtype, pad, freq):
    V, D = 50, 64
    idx = np.random.default_rng(15).integers(0, V, size=(8, 33)).astype(np.int64)
    idx[0, :5] = 3
    dy = sample(orc, (8, 33, D), dtype, 16)
    got = ops.embedding_dense_backward(dev.from_numpy(dy, dtype=dtype), dev.from_numpy(idx), V,
                                       pad, freq).numpy()
    want = orc.embedding_backward(dtype, dy, idx, V, pad, freq)
    assert got.shape == (V, D)
    counts = np.bincount(idx.reshape(-1), minlength=V)
    assert_normwise(got, want, dtype, float(np.sqrt(counts.max())), "embedding backward")
    if pad >= 0:
        assert not orc.to_float(got[pad:pad + 1], dtype).any(), "padding row must stay zero"


# (V, n, index dtype): 313 blocks of 128 rows read 3000 int32 indices each
# (3.7 MB, the range plan), or 70000 int64 indices each (175 MB, above the
# plan's 128 MiB cap: count, scan and fill over the whole table)
PLAN_CASES = [(40000, 3000, np.int32), (40000, 70000, np.int64)]


@pytest.mark.parametrize("V,n,itype", PLAN_CASES, ids=["range-plan", "count-scan-fill"])
def test_embedding_dense_backward_large_table(dev, ops, orc, V, n, itype):
    """A large table (40 samples on the last row, padding row 5 with samples
    of its own): the oracle's gradient, the padding row zero, and the same
    bits on a second run."""
    D = 8
    idx = np.random.default_rng(21).integers(0, V, size=n).astype(itype)
    idx[:40] = V - 1
    idx[40:60] = 5
    dy = sample(orc, (n, D), F32, 22)
    g, i = dev.from_numpy(dy), dev.from_numpy(idx)
    got = ops.embedding_dense_backward(g, i, V, 5, False).numpy()
    assert_bitexact(ops.embedding_dense_backward(g, i, V, 5, False).numpy(), got, "repeat")
    want = orc.embedding_backward(F32, dy, idx.astype(np.int64), V, 5, False)
    assert got.shape == (V, D)
    counts = np.bincount(idx.astype(np.int64), minlength=V)
    assert_normwise(got, want, F32, float(np.sqrt(counts.max())), f"embedding backward V={V} n={n}")
    assert not got[5].any(), "padding row must stay zero"


def sample_order_sum(orc, dtype, dy, idx, V, pad, freq):
    """Each row's float32 sum of its samples' dy rows in increasing sample
    order, starting from 0 (np.add.at adds in index order), times the
    float32 1 / count with scale_grad_by_freq, stored in `dtype`."""
    keep = (idx >= 0) & (idx < V) & (idx != pad)
    acc = np.zeros((V, dy.shape[1]), np.float32)
    np.add.at(acc, idx[keep].astype(np.int64), orc.to_float(dy, dtype)[keep])
    if freq:
        c = np.bincount(idx[keep].astype(np.int64), minlength=V).astype(np.float32)
        scale = np.float32(1) / np.maximum(c, np.float32(1))
        acc = acc * scale[:, None]
    return orc.from_float(acc, dtype)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("V,n,itype", [(5000, 8192, np.int64), (3000, 12000, np.int32),
                                       (100, 300000, np.int32), (40000, 70000, np.int64)],
                         ids=["range-plan-int64", "range-plan-int32", "range-plan-13-regions",
                              "count-scan-fill"])
def test_embedding_dense_backward_sums_in_sample_order(dev, ops, orc, dtype, V, n, itype):
    """Both plans list each row's samples in increasing order and the row is
    their float32 sum from 0 in that order: bit-exact against that sum, with
    a 500-sample row, a padding index with samples, out-of-range indices
    (skipped) and both scalings.  The range plan spreads its blocks over 16
    list regions, fewer when 16 x n entries would pass 2^22: 100 one-row
    blocks over 300000 int32 indices (120 MB of index reads, under the plan's
    128 MiB cap) use 13."""
    rng = np.random.default_rng(26)
    D = 64 if n <= 8192 else 8
    idx = rng.integers(0, V, size=n).astype(itype)
    idx[rng.permutation(n)[:500]] = 3
    idx[7:19] = 11
    idx[100] = V
    idx[200] = -1
    dy = sample(orc, (n, D), dtype, 27)
    g, i = dev.from_numpy(dy, dtype=dtype), dev.from_numpy(idx)
    for freq in (False, True):
        got = ops.embedding_dense_backward(g, i, V, 11, freq).numpy()
        assert_bitexact(got, sample_order_sum(orc, dtype, dy, idx, V, 11, freq), f"freq={freq}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
def test_embedding_dense_backward_heavy_rows(dev, ops, orc, dtype):
    """A row taking more samples than the per-row LDS ordering holds (5000
    of 6000 samples on row 7), ragged widths, int32 indices; two runs give
    the same bits (each row sums its samples in sample order)."""
    rng = np.random.default_rng(24)
    V = 40
    idx = rng.integers(0, V, size=6000).astype(np.int32)
    idx[rng.permutation(6000)[:5000]] = 7
    for D in (96, 5):
        dy = sample(orc, (6000, D), dtype, 25)
        g, i = dev.from_numpy(dy, dtype=dtype), dev.from_numpy(idx)
        got = ops.embedding_dense_backward(g, i, V, -1, True).numpy()
        again = ops.embedding_dense_backward(g, i, V, -1, True).numpy()
        assert_bitexact(again, got, f"repeat D={D}")
        want = orc.embedding_backward(dtype, dy, idx, V, -1, True)
        assert_normwise(got, want, dtype, 1, f"heavy rows D={D}")
        got = ops.embedding_dense_backward(g, i, V, -1, False).numpy()
        want = orc.embedding_backward(dtype, dy, idx, V, -1, False)
        assert_normwise(got, want, dtype, float(np.sqrt(5000)), f"heavy rows unscaled D={D}")


def test_embedding_declines_sparse(dev, ops, orc):
    w = dev.from_numpy(sample(orc, (10, 8), F32, 17))
    i = dev.from_numpy(np.array([1, 2], np.int64))
    with pytest.raises(tensor_mod().DeclinedError):
        ops.embedding(w, i, sparse=True)


# ---- negative log-likelihood ------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("reduction", [0, 1, 2], ids=["none", "mean", "sum"])
@pytest.mark.parametrize("weighted", [False, True], ids=["unweighted", "weighted"])
def test_nll_loss(dev, ops, orc, dtype, reduction, weighted):
    n, c = 1000, 37
    x = sample(orc, (n, c), dtype, 18)
    rng = np.random.default_rng(19)
    t = rng.integers(0, c, size=n).astype(np.int64)
    t[::17] = 5  # a custom ignore_index below
    w = orc.from_float(rng.random(c).astype(np.float32) + 0.5, dtype) if weighted else None
    dx_, dt_ = dev.from_numpy(x, dtype=dtype), dev.from_numpy(t)
    dw_ = dev.from_numpy(w, dtype=dtype) if weighted else None
    y, total = ops.nll_loss(dx_, dt_, dw_, reduction, 5)
    wy, wtotal = orc.nll_loss(dtype, x, t, w, reduction, 5)
    assert y.shape == wy.shape and total.shape == ()
    assert_normwise(y.numpy(), wy, dtype, float(np.sqrt(n)) if reduction == 2 else 1, "loss")
    assert_normwise(total.numpy(), wtotal, dtype, 1, "total weight")
    g = sample(orc, (n,) if reduction == 0 else (), dtype, 20)
    got = ops.nll_loss_backward(dev.from_numpy(g, dtype=dtype), dx_, dt_, dw_, reduction, 5,
                                total).numpy()
    want = orc.nll_loss_backward(dtype, g, (n, c), t, total.numpy(), w, reduction, 5)
    assert_elementwise(got, want, dtype, "nll backward")


def test_nll_loss_int32_targets_and_bad_target(dev, ops, orc):
    x = sample(orc, (64, 10), F32, 21)
    t = np.arange(64, dtype=np.int32) % 10
    y, total = ops.nll_loss(dev.from_numpy(x), dev.from_numpy(t), None, 2, -100)
    assert_normwise(y.numpy(), orc.nll_loss(F32, x, t, None, 2)[0], F32, 8, "int32 targets")
    assert float(total.numpy()) == 64.0
    t[7] = 10  # outside [0, C), not ignore_index
    y, _ = ops.nll_loss(dev.from_numpy(x), dev.from_numpy(t), None, 0, -100)
    got = y.numpy()
    assert np.isnan(got[7]) and not np.isnan(np.delete(got, 7)).any()
    dx = ops.nll_loss_backward(dev.from_numpy(np.ones(64, np.float32)), dev.from_numpy(x),
                               dev.from_numpy(t), None, 0, -100,
                               dev.from_numpy(np.zeros((), np.float32))).numpy()
    assert np.isnan(dx[7]).all() and not np.isnan(np.delete(dx, 7, axis=0)).any()


def test_nll_loss_large_batch(dev, ops, orc):
    n, c = 2048, 32000
    x = sample(orc, (n, c), F32, 22)
    t = np.random.default_rng(23).integers(0, c, size=n).astype(np.int64)
    dx_, dt_ = dev.from_numpy(x), dev.from_numpy(t)
    y, total = ops.nll_loss(dx_, dt_, None, 1, -100)
    assert_normwise(y.numpy(), orc.nll_loss(F32, x, t, None, 1)[0], F32, 1, "mean loss")
    g = np.array(0.75, np.float32)
    got = ops.nll_loss_backward(dev.from_numpy(g), dx_, dt_, None, 1, -100, total).numpy()
    want = orc.nll_loss_backward(F32, g, (n, c), t, total.numpy(), None, 1, -100)
    assert_elementwise(got, want, F32, "large nll backward")


@pytest.mark.parametrize("reduction", [1, 2], ids=["mean", "sum"])
def test_nll_loss_many_blocks_folded_in_one_launch(dev, ops, orc, reduction):
    """300001 samples: 1172 blocks, more than the last block's 256 threads,
    so each folding thread adds several partials.  Two calls in a row give
    the same bits (the arrival counter is reset, the fold order is fixed)."""
    n, c = 300001, 7
    x = sample(orc, (n, c), F32, 24)
    t = np.random.default_rng(25).integers(0, c, size=n).astype(np.int64)
    t[::11] = 3  # ignore_index
    dx_, dt_ = dev.from_numpy(x), dev.from_numpy(t)
    outs = [ops.nll_loss(dx_, dt_, None, reduction, 3) for _ in range(2)]
    wy, wtotal = orc.nll_loss(F32, x, t, None, reduction, 3)
    y0, total0 = (v.numpy() for v in outs[0])
    y1, total1 = (v.numpy() for v in outs[1])
    assert y0.tobytes() == y1.tobytes() and total0.tobytes() == total1.tobytes()
    assert_normwise(y0, wy, F32, float(np.sqrt(n)) if reduction == 2 else 1, "loss")
    assert float(total0) == float(wtotal) == float(np.count_nonzero(t != 3))


# ---- empty inputs ----------------------------------------------------------------


def test_empty_inputs_follow_the_reference(dev, ops, orc):
    """Empty operands take the reference's paths (NNKernels.cpp): layer norm
    and its backward decline an empty input (:73, :122), as does nll_loss
    and its backward (nll_native needs numel > 0, :315-320); dropout and
    its backward return empty results (:181, :228); an embedding lookup of
    no indices is [0, D] (:252); the gradient of a table from no samples
    is a zero table, and of an empty table an empty one (:279)."""
    DeclinedError = tensor_mod().DeclinedError
    x0 = dev.from_numpy(np.zeros((0, 64), np.float32))
    with pytest.raises(DeclinedError):
        ops.native_layer_norm(x0, (64,))
    st = dev.from_numpy(np.zeros(0, np.float32))
    with pytest.raises(DeclinedError):
        ops.native_layer_norm_backward(x0, x0, (64,), st, st)
    out, mask = ops.native_dropout(x0, 0.5, True, seed=3)
    assert out.shape == (0, 64) and mask.shape == (0, 64)
    assert ops.native_dropout_backward(x0, mask, 2.0).shape == (0, 64)
    w = dev.from_numpy(sample(orc, (10, 8), F32, 40))
    none = dev.from_numpy(np.zeros(0, np.int64))
    assert ops.embedding(w, none).shape == (0, 8)
    g0 = dev.from_numpy(np.zeros((0, 8), np.float32))
    for V in (10, 3000):   # the range plan with no samples
        got = ops.embedding_dense_backward(g0, none, V).numpy()
        assert got.shape == (V, 8) and not got.any()
    assert ops.embedding_dense_backward(g0, none, 0).shape == (0, 8)
    with pytest.raises(DeclinedError):
        ops.nll_loss(dev.from_numpy(np.zeros((0, 5), np.float32)), none, None, 1)
    with pytest.raises(DeclinedError):
        ops.nll_loss_backward(dev.from_numpy(np.array(1.0, np.float32)),
                              dev.from_numpy(np.zeros((0, 5), np.float32)), none, None, 1, -100,
                              dev.from_numpy(np.array(0.0, np.float32)))
    # a real call after the empty ones still gives the oracle's answer
    idx = np.array([1, 4, 4, 9], np.int64)
    dy = sample(orc, (4, 8), F32, 41)
    got = ops.embedding_dense_backward(dev.from_numpy(dy), dev.from_numpy(idx), 3000).numpy()
    assert_bitexact(got, sample_order_sum(orc, F32, dy, idx, 3000, -1, False), "after empty calls")


def same_nonfinite(got, want, dtype, what, rel):
    """NaN and infinities where the oracle has them; the finite rest within
    ``rel`` of max(|want|, 1)."""
    g, w = as_float(got, dtype).reshape(-1), as_float(want, dtype).reshape(-1)
    assert np.array_equal(np.isnan(g), np.isnan(w)), f"{what}: NaN in other places"
    inf = np.isinf(w)
    assert np.array_equal(np.isinf(g), inf) and np.array_equal(g[inf], w[inf]), f"{what}: infinities differ"
    fin = np.isfinite(w)
    assert np.all(np.abs(g[fin] - w[fin]) <= rel * np.maximum(np.abs(w[fin]), 1.0)), f"{what}: finite values differ"


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_special_values(dev, ops, orc, dtype):
    """NaN, infinities and constant rows through layer norm and its
    backward (a NaN or infinite element makes its row NaN, a constant row
    normalises to the bias), dropout (the mask is the same; a kept NaN stays
    NaN) and nll_loss (a -inf or NaN target log-probability), against the
    oracle."""
    rng = np.random.default_rng(1)
    D = 256
    x = rng.standard_normal((8, D)).astype(np.float32)
    x[1, 3], x[2, 7], x[4, 9] = np.nan, np.inf, -np.inf
    x[3, :], x[5, :] = 5.0, 0.0
    X = orc.from_float(x, dtype)
    w = sample(orc, (D,), dtype, 2)
    b = sample(orc, (D,), dtype, 3)
    dX, dw, db = (dev.from_numpy(a, dtype=dtype) for a in (X, w, b))
    y, mean, rstd = ops.native_layer_norm(dX, (D,), dw, db)
    wy, wm, wr = orc.layer_norm(dtype, X, D, w, b, 1e-5)
    tol = 1e-5 if dtype == F32 else 1e-2
    same_nonfinite(y.numpy(), wy, dtype, "layer norm y", tol)
    same_nonfinite(mean.numpy(), wm, F32, "layer norm mean", 1e-5)
    same_nonfinite(rstd.numpy(), wr, F32, "layer norm rstd", 1e-5)
    dy = sample(orc, (8, D), dtype, 4)
    gx, gw, gb = ops.native_layer_norm_backward(dev.from_numpy(dy, dtype=dtype), dX, (D,), mean, rstd, dw, db)
    ox, ow, ob = orc.layer_norm_backward(dtype, dy, X, D, mean.numpy(), rstd.numpy(), w)
    same_nonfinite(gx.numpy(), ox, dtype, "layer norm dx", 10 * tol)
    same_nonfinite(gw.numpy(), ow, dtype, "layer norm dweight", 10 * tol)
    same_nonfinite(gb.numpy(), ob, dtype, "layer norm dbias", 10 * tol)
    xs = np.tile(np.float32([np.nan, np.inf, -np.inf, -0.0, 0.0, 1.0, -2.0, 3e4]), 4096)
    XS = orc.from_float(xs, dtype)
    out, mask = ops.native_dropout(dev.from_numpy(XS, dtype=dtype), 0.3, True, seed=7)
    wo, wmask = orc.dropout(dtype, XS, 0.3, 7)
    assert np.array_equal(mask.numpy().astype(np.uint8), wmask), "dropout mask"
    same_nonfinite(out.numpy(), wo, dtype, "dropout", 0.0)
    lp = rng.standard_normal((16, 50)).astype(np.float32)
    lp[2, 4], lp[3, 5], lp[6, 1] = -np.inf, np.nan, np.inf
    t = np.array([4, 4, 4, 5, 0, 1, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10], np.int64)
    LP = orc.from_float(lp, dtype)
    for red in (0, 1, 2):
        got, _ = ops.nll_loss(dev.from_numpy(LP, dtype=dtype), dev.from_numpy(t), None, red)
        want, _ = orc.nll_loss(dtype, LP, t, None, red)
        same_nonfinite(got.numpy(), want, dtype, f"nll_loss reduction {red}", tol)

