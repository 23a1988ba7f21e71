"""Pins the oracle's neural-network layers (oracle/oracle.c: orc_layer_norm,
orc_philox4x32_10, orc_dropout, orc_embedding, orc_nll_loss and their
backwards) before they are trusted as the checker.

Expected values come from code that is not the oracle's: torch's CPU
float64 operators and autograd (an independent library implementation),
numpy indexing and one-hot products, central finite differences, the
Random123 known-answer vectors for Philox4x32-10, and closed forms chosen
so that a plausible slip -- unbiased instead of biased variance, eps outside
the square root, a dropped weight, the wrong Philox word or key half,
scaling by p instead of 1 / (1 - p), counting the padding row, dividing the
mean by N instead of the total weight -- fails at least one check.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _check import ulp_distance

F32, F16, BF16, F64 = 0, 1, 2, 3


def t64(a):
    return torch.from_numpy(np.asarray(a, np.float64))


# ---- layer norm ------------------------------------------------------------------

@pytest.mark.parametrize("norm", [(24,), (5, 24)])
def test_layer_norm_against_torch_float64(orc, norm):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 5, 24)) * 2.0 + 0.5
    D = int(np.prod(norm))
    w = rng.standard_normal(norm)
    b = rng.standard_normal(norm)
    y, mean, rstd = orc.layer_norm(F64, x, D, w, b, eps=1e-3)
    ty, tmean, trstd = torch.native_layer_norm(t64(x), list(norm), t64(w), t64(b), 1e-3)
    np.testing.assert_allclose(y, ty.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mean, tmean.numpy().reshape(-1), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(rstd, trstd.numpy().reshape(-1), rtol=1e-12)
    # without the affine parameters
    y0, _, _ = orc.layer_norm(F64, x, D, None, None, eps=1e-3)
    np.testing.assert_allclose(y0, F.layer_norm(t64(x), list(norm), eps=1e-3).numpy(),
                               rtol=1e-12, atol=1e-12)


def test_layer_norm_float32_rounds_once(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 40)).astype(np.float32)
    w = rng.standard_normal(40).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    y, mean, rstd = orc.layer_norm(F32, x, 40, w, b)
    want = F.layer_norm(t64(x), [40], t64(w), t64(b), 1e-5).numpy().astype(np.float32)
    assert int(ulp_distance(y, want, F32).max()) == 0
    assert mean.dtype == np.float32 and rstd.dtype == np.float32
    # 16-bit storage keeps float32 statistics
    xb = orc.to_bf16(x)
    _, mb, rb = orc.layer_norm(BF16, xb, 40)
    assert mb.dtype == np.float32 and rb.dtype == np.float32
    xf = orc.from_bf16(xb).astype(np.float64)
    np.testing.assert_allclose(mb, xf.mean(1), rtol=1e-6, atol=1e-7)


def test_layer_norm_invariants(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 33))
    # eps = 0: invariant under a positive scale and a shift of each row
    y, _, _ = orc.layer_norm(F64, x, 33, eps=0.0)
    y2, _, _ = orc.layer_norm(F64, 3.0 * x + 7.0, 33, eps=0.0)
    np.testing.assert_allclose(y2, y, atol=1e-12)
    # unit weight: each row has mean 0 and biased variance 1
    np.testing.assert_allclose(y.mean(1), 0.0, atol=1e-13)
    np.testing.assert_allclose((y ** 2).mean(1), 1.0, rtol=1e-12)
    # a constant row: y = b, mean = the constant, rstd = 1 / sqrt(eps)
    c = np.full((2, 8), 4.25)
    b = np.arange(8.0)
    yc, mc, rc = orc.layer_norm(F64, c, 8, np.ones(8), b, eps=0.25)
    np.testing.assert_array_equal(yc, np.broadcast_to(b, (2, 8)))
    np.testing.assert_array_equal(mc, [4.25, 4.25])
    np.testing.assert_array_equal(rc, [2.0, 2.0])
    # two values: mean and biased variance by hand
    _, m2, r2 = orc.layer_norm(F64, np.array([[1.0, 3.0]]), 2, eps=0.0)
    assert m2[0] == 2.0 and r2[0] == 1.0


def test_layer_norm_backward_against_torch_autograd(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((9, 31)) * 1.5 - 0.25
    w = rng.standard_normal(31)
    b = rng.standard_normal(31)
    dy = rng.standard_normal((9, 31))
    _, mean, rstd = orc.layer_norm(F64, x, 31, w, b, eps=1e-4)
    dx, dw, db = orc.layer_norm_backward(F64, dy, x, 31, mean, rstd, w)
    tx, tw, tb = t64(x).requires_grad_(), t64(w).requires_grad_(), t64(b).requires_grad_()
    F.layer_norm(tx, [31], tw, tb, 1e-4).backward(t64(dy))
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-12, atol=1e-12)
    # outputs not asked for are not produced
    dx2, dw2, db2 = orc.layer_norm_backward(F64, dy, x, 31, mean, rstd, w, mask=(True, False, False))
    assert dw2 is None and db2 is None
    np.testing.assert_array_equal(dx2, dx)


def test_layer_norm_backward_finite_differences(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 12))
    w = rng.standard_normal(12)
    b = rng.standard_normal(12)
    dy = rng.standard_normal((3, 12))
    _, mean, rstd = orc.layer_norm(F64, x, 12, w, b, eps=1e-2)
    dx, dw, db = orc.layer_norm_backward(F64, dy, x, 12, mean, rstd, w)

    def loss(xv, wv, bv):
        return float((orc.layer_norm(F64, xv, 12, wv, bv, eps=1e-2)[0] * dy).sum())

    h = 1e-6
    for _ in range(3):
        vx, vw, vb = rng.standard_normal(x.shape), rng.standard_normal(12), rng.standard_normal(12)
        fd = (loss(x + h * vx, w + h * vw, b + h * vb) - loss(x - h * vx, w - h * vw, b - h * vb)) / (2 * h)
        an = float((dx * vx).sum() + (dw * vw).sum() + (db * vb).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an))


# ---- Philox4x32-10 and dropout ------------------------------------------------------

# Random123 known-answer vectors for philox4x32 with 10 rounds:
# (counter words, key words) -> output words.
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(orc, ctr, key, want):
    assert tuple(int(v) for v in orc.philox4x32_10(ctr, key)) == want


def test_dropout_first_block_by_hand(orc):
    # seed 0, offset 0: elements 0..3 take the words of the first vector.
    words = PHILOX_KAT[0][2]
    x = np.array([1.0, -2.0, 3.0, 0.5, 7.0])
    for p in (0.25, 0.5, 0.75):
        out, mask = orc.dropout(F64, x, p, seed=0, offset=0)
        want = [(wd >> 8) * 2.0 ** -24 >= p for wd in words]
        np.testing.assert_array_equal(mask[:4], want)
        np.testing.assert_array_equal(out[:4], np.where(want, x[:4] / (1 - p), 0.0))


def test_dropout_stream_layout(orc):
    # element e: word e % 4 of counter (e / 4, 0, offset lo, offset hi) under
    # key (seed lo, seed hi)
    seed, offset = 0x299F31D0A4093822, 0x0370734413198A2E
    n = 4 * 5 + 3
    _, mask = orc.dropout(F64, np.ones(n), 0.5, seed, offset)
    for e in range(n):
        w = orc.philox4x32_10((e // 4, 0, offset & 0xFFFFFFFF, offset >> 32),
                              (seed & 0xFFFFFFFF, seed >> 32))[e % 4]
        assert mask[e] == ((int(w) >> 8) * 2.0 ** -24 >= 0.5)
    # the high half of the seed is part of the key
    _, m0 = orc.dropout(F64, np.ones(64), 0.5, seed, 0)
    _, m1 = orc.dropout(F64, np.ones(64), 0.5, seed & 0xFFFFFFFF, 0)
    assert (m0 != m1).any()


def test_dropout_statistics_and_scale(orc):
    rng = np.random.default_rng(6)
    n = 1 << 20
    x = rng.standard_normal(n).astype(np.float32)
    for p in (0.1, 0.5, 0.9):
        out, mask = orc.dropout(F32, x, p, seed=1234, offset=0)
        keep = mask.astype(bool)
        frac = keep.mean()
        assert abs(frac - (1 - p)) < 5 * np.sqrt(p * (1 - p) / n)
        np.testing.assert_array_equal(out[~keep], 0.0)
        want = (x[keep].astype(np.float64) / (1 - p)).astype(np.float32)
        assert int(ulp_distance(out[keep], want, F32).max()) == 0
    # p = 0 keeps everything unchanged
    out, mask = orc.dropout(F32, x, 0.0, seed=5)
    assert mask.all()
    np.testing.assert_array_equal(out, x)
    # another seed, another mask
    _, m2 = orc.dropout(F32, x, 0.5, seed=1235)
    _, m1 = orc.dropout(F32, x, 0.5, seed=1234)
    assert 0.45 < (m1 != m2).mean() < 0.55


def test_dropout_backward(orc):
    rng = np.random.default_rng(7)
    g = rng.standard_normal(1001)
    m = (rng.random(1001) < 0.6).astype(np.uint8)
    np.testing.assert_array_equal(orc.dropout_backward(F64, g, m, 2.5), g * m * 2.5)


# ---- embedding -------------------------------------------------------------------------

@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_embedding_is_row_indexing(orc, itype):
    rng = np.random.default_rng(8)
    w = rng.standard_normal((50, 12)).astype(np.float32)
    idx = rng.integers(0, 50, size=(4, 7)).astype(itype)
    out = orc.embedding(F32, w, idx)
    np.testing.assert_array_equal(out, w[idx])
    wb = orc.to_bf16(w)
    np.testing.assert_array_equal(orc.embedding(BF16, wb, idx), wb[idx])
    # an index outside the table gives a NaN row
    bad = np.array([3, 50, -1, 7], itype)
    o = orc.embedding(F32, w, bad)
    assert np.isnan(o[1]).all() and np.isnan(o[2]).all()
    np.testing.assert_array_equal(o[[0, 3]], w[[3, 7]])


@pytest.mark.parametrize("pad,freq", [(-1, False), (3, False), (-1, True), (3, True)])
def test_embedding_backward_against_torch_autograd(orc, pad, freq):
    rng = np.random.default_rng(9)
    V, D = 20, 6
    idx = rng.integers(0, V, size=(5, 9)).astype(np.int64)
    idx[0, :4] = 3  # repeated and padding indices
    dy = rng.standard_normal((5, 9, D))
    got = orc.embedding_backward(F64, dy, idx, V, pad, freq)
    tw = torch.zeros(V, D, dtype=torch.float64, requires_grad=True)
    F.embedding(torch.from_numpy(idx), tw, padding_idx=pad if pad >= 0 else None,
                scale_grad_by_freq=freq).backward(t64(dy))
    np.testing.assert_allclose(got, tw.grad.numpy(), rtol=1e-12, atol=1e-12)
    if not freq:
        # the one-hot product, padding column removed
        onehot = np.zeros((idx.size, V))
        onehot[np.arange(idx.size), idx.reshape(-1)] = 1.0
        if pad >= 0:
            onehot[:, pad] = 0.0
        np.testing.assert_allclose(got, onehot.T @ dy.reshape(-1, D), rtol=1e-12, atol=1e-12)


def test_embedding_backward_skips_out_of_range(orc):
    dy = np.ones((3, 2))
    got = orc.embedding_backward(F64, dy, np.array([1, 9, -2], np.int32), 4)
    np.testing.assert_array_equal(got, [[0, 0], [1, 1], [0, 0], [0, 0]])


# ---- negative log-likelihood ----------------------------------------------------------

@pytest.mark.parametrize("reduction", [0, 1, 2])
@pytest.mark.parametrize("weighted", [False, True])
def test_nll_loss_against_torch(orc, reduction, weighted):
    rng = np.random.default_rng(10)
    n, c = 37, 11
    x = rng.standard_normal((n, c))
    t = rng.integers(0, c, size=n).astype(np.int64)
    t[[2, 5, 30]] = -100
    w = rng.random(c) + 0.5 if weighted else None
    y, total = orc.nll_loss(F64, x, t, w, reduction, -100)
    red = ["none", "mean", "sum"][reduction]
    ty = F.nll_loss(t64(x), torch.from_numpy(t), None if w is None else t64(w),
                    ignore_index=-100, reduction=red)
    np.testing.assert_allclose(y, ty.numpy(), rtol=1e-12, atol=1e-12)
    valid = t != -100
    wt = (w[t[valid]] if weighted else np.ones(valid.sum())).sum()
    assert float(total) == (0.0 if reduction == 0 else pytest.approx(wt, rel=1e-12))
    # backward against autograd
    tx = t64(x).requires_grad_()
    g = rng.standard_normal(n) if reduction == 0 else np.array(1.7)
    F.nll_loss(tx, torch.from_numpy(t), None if w is None else t64(w), ignore_index=-100,
               reduction=red).backward(t64(g))
    dx = orc.nll_loss_backward(F64, g, (n, c), t, np.array(wt), w, reduction, -100)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_nll_loss_closed_forms(orc):
    x = np.array([[0.5, -1.0, 2.0], [3.0, 0.25, -4.0]])
    t = np.array([2, 0], np.int32)
    y, total = orc.nll_loss(F64, x, t, None, 2)
    assert float(y) == -(2.0 + 3.0) and float(total) == 2.0
    y, _ = orc.nll_loss(F64, x, t, None, 1)
    assert float(y) == -(2.0 + 3.0) / 2
    # weights divide the mean by the total weight, not by N
    w = np.array([4.0, 1.0, 0.5])
    y, total = orc.nll_loss(F64, x, t, w, 1)
    assert float(total) == 4.5 and float(y) == -(0.5 * 2.0 + 4.0 * 3.0) / 4.5
    # every target ignored: the mean is 0 / 0
    y, total = orc.nll_loss(F64, x, np.array([-100, -100], np.int64), None, 1)
    assert np.isnan(y) and float(total) == 0.0
    # a target outside [0, C) that is not ignore_index: NaN
    y, _ = orc.nll_loss(F64, x, np.array([5, 0], np.int64), None, 0)
    assert np.isnan(y[0]) and y[1] == -3.0
