"""Thin products (at most 64 rows or 64 columns of C) on the GPU against the
float64 product of the same stored operands: the decode-step shapes of a
Linear layer, a matrix-vector product and an LM head, which run on their
own kernel (stream-K over column tiles, 16 x 16 MFMAs, partials of tiles
shared between blocks added in block order).

Bars as for every product (north_star): float32 within 2e-3, bfloat16 and
float16 within 1e-2 as max |got - want| / max |want|.  Operands are stored
with NaN padding past their logical extent, so a read outside the operand
shows as NaN.
"""

import numpy as np
import pytest

from _check import BF16, F16, F32

pytestmark = pytest.mark.gpu

BAR = {F32: 2e-3, BF16: 1e-2, F16: 1e-2}
IDS = {F32: "fp32", BF16: "bf16", F16: "fp16"}


def _padded(orc, shape, pad, dtype, seed):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * np.float32(0.5)
    store = np.full(shape[:-1] + (shape[-1] + pad,), np.nan, np.float32)
    store[..., :shape[-1]] = x
    return orc.from_float(store, dtype)


def _run(lib, dev, orc, dtype, bt, m, n, k, ta, tb, *, pad=8, alpha=1.0, beta=0.0, cin_kind="none",
         shared_b=False, reps=1, seed=0):
    """C = alpha op(A) op(B) + beta Cin through tp_amd_launch_gemm; returns
    (outputs of each rep, float64 expectation)."""
    a = _padded(orc, (bt, k, m) if ta else (bt, m, k), pad, dtype, seed + 1)
    b = _padded(orc, (1 if shared_b else bt, n, k) if tb else (1 if shared_b else bt, k, n), pad, dtype,
                seed + 2)
    lda, ldb = a.shape[-1], b.shape[-1]
    A = orc.to_float(a, dtype).astype(np.float64)[..., :(m if ta else k)]
    B = orc.to_float(b, dtype).astype(np.float64)[..., :(k if tb else n)]
    A = np.swapaxes(A, -1, -2) if ta else A
    B = np.swapaxes(B, -1, -2) if tb else B
    want = alpha * np.matmul(A, B)
    if cin_kind == "none":
        cin, rs, cs, sb = None, 0, 0, 0
    elif cin_kind == "bias-row":
        cin, rs, cs, sb = _padded(orc, (n,), 0, dtype, seed + 3), 0, 1, 0
        want = want + beta * orc.to_float(cin, dtype)
    else:
        cin, rs, cs, sb = _padded(orc, (bt, m, n), 0, dtype, seed + 3), n, 1, m * n
        want = want + beta * orc.to_float(cin, dtype)
    da, db = dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)
    dc = dev.from_numpy(cin, dtype=dtype) if cin is not None else None
    outs = []
    for _ in range(reps):
        out = dev.empty((bt, m, n), dtype=dtype)
        st = lib.tp_amd_launch_gemm(0, dtype, bt, m, n, k, alpha, da.data_ptr, lda, a.shape[-2] * lda, int(ta),
                                    db.data_ptr, ldb, 0 if shared_b else b.shape[-2] * ldb, int(tb), beta,
                                    dc.data_ptr if dc is not None else 0, rs, cs, sb, out.data_ptr, n, m * n)
        assert st == 0, lib.tp_mlu_last_error()
        outs.append(out.numpy())
    return outs, want


def _check(orc, got, want, dtype, what):
    g = orc.to_float(got, dtype)
    assert not np.isnan(g).any(), f"{what}: NaN padding reached the product"
    e = float(np.max(np.abs(g - want)) / max(np.max(np.abs(want)), 1e-30))
    assert e <= BAR[dtype], f"{what}: relative error {e:.3g} > {BAR[dtype]}"


# (m, n, k): thin rows, then the same shapes with the thin side as columns.
# They cover tiles split between blocks (long K), one step per block (short K
# over many tiles), ragged column tiles, 16 and 32 thin rows and one more
# (two MFMA row groups), and a K that is not a whole number of steps.  The
# wide operand is at least 1 MiB (8 MiB past 16 thin rows), the sizes from
# which products take the thin kernel; the last shape is below that and
# checks the tiled kernels still take it.
THIN = [(1, 1000, 4096), (5, 4104, 136), (16, 520, 1024), (17, 4104, 1024), (32, 8200, 512), (32, 512, 8200),
        (3, 264, 2056), (3, 17, 2056)]


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: IDS[d])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("m,n,k", THIN + [(n, m, k) for (m, n, k) in THIN],
                         ids=[f"{m}x{n}x{k}" for (m, n, k) in THIN] + [f"{n}x{m}x{k}" for (m, n, k) in THIN])
def test_thin_layouts(amd, dev, orc, dtype, ta, tb, m, n, k):
    lib = amd.load()
    (got,), want = _run(lib, dev, orc, dtype, 1, m, n, k, ta, tb)
    _check(orc, got[0], want[0], dtype, f"thin {m}x{n}x{k} ta={ta} tb={tb}")


# 33 to 64 thin rows (row groups of 64): W K-major and float32 W N-major;
# 16-bit W N-major past 32 rows, and anything past 64, goes to the tiled
# kernels.  Checked in the four layouts like the shapes above.
WIDE = [(40, 4104, 1024), (64, 2056, 2048), (65, 1032, 4096), (100, 4104, 1024)]


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: IDS[d])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("m,n,k", WIDE + [(n, m, k) for (m, n, k) in WIDE],
                         ids=[f"{m}x{n}x{k}" for (m, n, k) in WIDE] + [f"{n}x{m}x{k}" for (m, n, k) in WIDE])
def test_thin_up_to_128_rows(amd, dev, orc, dtype, ta, tb, m, n, k):
    lib = amd.load()
    (got,), want = _run(lib, dev, orc, dtype, 1, m, n, k, ta, tb)
    _check(orc, got[0], want[0], dtype, f"thin {m}x{n}x{k} ta={ta} tb={tb}")


# 16-bit products of more than 16 thin rows leave the thin kernel for the
# split over K when that gives every CU a block (8200 wide columns with K =
# 4096: 65 tiles of 128 times seven slices of 640, the last 256; 10248
# columns and 24 rows: 81 tiles times six slices).  K = 4100 has a last
# slice of 260 after a copy of the K-major operands.  float32 products of
# 33-64 rows against at least 128 tiles of 64 columns take the split on
# 64 x 64 tiles (8200 columns; K = 4100 does not split and stays thin).
SPLIT = [(40, 8200, 4096), (64, 8200, 4096), (48, 8200, 4100), (24, 10248, 4096)]


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: IDS[d])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("m,n,k", SPLIT + [(n, m, k) for (m, n, k) in SPLIT],
                         ids=[f"{m}x{n}x{k}" for (m, n, k) in SPLIT] + [f"{n}x{m}x{k}" for (m, n, k) in SPLIT])
def test_thin_rows_past_32_split(amd, dev, orc, dtype, ta, tb, m, n, k):
    lib = amd.load()
    outs, want = _run(lib, dev, orc, dtype, 1, m, n, k, ta, tb, alpha=0.5, beta=2.0, cin_kind="bias-row",
                      reps=2)
    assert np.array_equal(outs[0], outs[1]), "two runs differ"
    _check(orc, outs[0][0], want[0], dtype, f"split {m}x{n}x{k} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: IDS[d])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, True)], ids=["NN", "NT", "TT"])
@pytest.mark.parametrize("cin_kind", ["bias-row", "full"])
@pytest.mark.parametrize("m,n,k", [(1, 1000, 1024), (24, 1040, 4096), (1032, 9, 512), (96, 2056, 2048)])
def test_thin_epilogue_batched(amd, dev, orc, dtype, ta, tb, cin_kind, m, n, k):
    """alpha = 0.5 and beta = 2 with a per-column bias or a full Cin, a
    batch of 3 (its B shared by the batch, stride 0, in the bias case), and
    two runs giving the same bits (partials added in block order)."""
    lib = amd.load()
    shared = cin_kind == "bias-row"
    outs, want = _run(lib, dev, orc, dtype, 3, m, n, k, ta, tb, alpha=0.5, beta=2.0, cin_kind=cin_kind,
                      shared_b=shared, reps=2)
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8)), "thin product not deterministic"
    _check(orc, outs[0], want, dtype, f"thin batched {m}x{n}x{k} {cin_kind}")


@pytest.mark.parametrize("dtype", [F32, BF16, F16], ids=lambda d: IDS[d])
def test_thin_vector_forms(dev, ops, orc, dtype):
    """matmul of a vector by a matrix and of a matrix by a vector, linear of
    one row, addmm with one row and a bias (the ops that reach thin
    products), against float64."""
    g = np.random.default_rng(5)
    mk = lambda *s: orc.from_float(g.standard_normal(s).astype(np.float32), dtype)  # noqa: E731
    d = lambda x: dev.from_numpy(x, dtype=dtype)  # noqa: E731
    f = lambda x: orc.to_float(x, dtype).astype(np.float64)  # noqa: E731
    v, w, x = mk(1536), mk(1536, 2048), mk(2048, 1536)
    _check(orc, ops.matmul(d(v), d(w)).numpy(), f(v) @ f(w), dtype, "vector @ matrix")
    _check(orc, ops.matmul(d(x), d(v)).numpy(), f(x) @ f(v), dtype, "matrix @ vector")
    xr, wl, bias = mk(1, 1536), mk(3000, 1536), mk(3000)
    _check(orc, ops.linear(d(xr), d(wl), d(bias)).numpy(), f(xr) @ f(wl).T + f(bias), dtype, "linear one row")
    got = ops.addmm(d(bias), d(xr), d(wl).t(), beta=0.5, alpha=2.0).numpy()
    _check(orc, got, 0.5 * f(bias) + 2.0 * (f(xr) @ f(wl).T), dtype, "addmm one row")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: IDS[d])
def test_thin_decode_shapes(dev, ops, orc, dtype):
    """The decode step of config 4's Linear (x [1, 4096] W [11008, 4096]^T),
    an LM head's logits (x [4, 4096] W [50257, 4096]^T) and its dX
    (dY [1, 50257] W [50257, 4096], an odd K)."""
    g = np.random.default_rng(7)
    mk = lambda *s: orc.from_float(g.standard_normal(s).astype(np.float32), dtype)  # noqa: E731
    d = lambda x: dev.from_numpy(x, dtype=dtype)  # noqa: E731
    f = lambda x: orc.to_float(x, dtype).astype(np.float64)  # noqa: E731
    x, w = mk(1, 4096), mk(11008, 4096)
    _check(orc, ops.linear(d(x), d(w)).numpy(), f(x) @ f(w).T, dtype, "decode linear")
    del w
    head = mk(50257, 4096)
    dh = d(head)
    x4 = mk(4, 4096)
    _check(orc, ops.linear(d(x4), dh).numpy(), f(x4) @ f(head).T, dtype, "LM head logits")
    dy = mk(1, 50257)
    _check(orc, ops.mm(d(dy), dh).numpy(), f(dy) @ f(head), dtype, "LM head dX")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: IDS[d])
@pytest.mark.parametrize("tb", [False, True], ids=["W-N-major", "W-K-major"])
def test_thin_nan_and_inf(dev, ops, orc, dtype, tb):
    """A NaN or infinity in one thin row or one wide column reaches exactly
    the entries IEEE arithmetic gives it, and no others (padding lanes
    multiply zeros)."""
    m, n, k = 7, 2000, 264
    rng = np.random.default_rng(3)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    a[2, 5], a[4, 9] = np.nan, np.inf
    b[9, 11] = 0.0
    b[40, 50] = -np.inf
    A, B = orc.from_float(a, dtype), orc.from_float(b, dtype)
    dA, dB = dev.from_numpy(A, dtype=dtype), dev.from_numpy(B, dtype=dtype)
    if tb:
        dB = dev.from_numpy(np.ascontiguousarray(B.T), dtype=dtype).t()
    got = orc.to_float(ops.mm(dA, dB).numpy(), dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        want = orc.to_float(A, dtype).astype(np.float64) @ orc.to_float(B, dtype).astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want)), "NaN in other places"
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf), "infinities in other places"
    assert np.array_equal(got[inf], want[inf]), "signs of the infinities"


@pytest.mark.parametrize("dtype", [F32, BF16], ids=lambda d: IDS[d])
def test_thin_after_repack(dev, ops, orc, dtype):
    """x [3, 2048] @ W [2048, 1001]: W row-major with an odd leading
    dimension, which no kernel reads in 16-byte packets, is copied K-major
    and then multiplied by the thin kernel; against float64."""
    g = np.random.default_rng(11)
    x = orc.from_float(g.standard_normal((3, 2048)).astype(np.float32), dtype)
    w = orc.from_float(g.standard_normal((2048, 1001)).astype(np.float32), dtype)
    got = ops.mm(dev.from_numpy(x, dtype=dtype), dev.from_numpy(w, dtype=dtype)).numpy()
    want = orc.to_float(x, dtype).astype(np.float64) @ orc.to_float(w, dtype).astype(np.float64)
    _check(orc, got, want, dtype, "thin product of a repacked operand")


def test_thin_random_shapes(amd, dev, orc):
    """Forty seeded random thin products: dtype, layout, thin side, row count
    (1-64), K (with and without a partial last step; odd when W is N-major),
    N ragged against the column tiles, batch (1-3, W shared or not), alpha,
    beta and the Cin form all drawn at random; each against float64 at the
    dtype's bar, and every one run twice for the same bits."""
    lib = amd.load()
    rng = np.random.default_rng(2024)
    for case in range(40):
        dtype = [F32, BF16, F16][rng.integers(3)]
        v = 8 if dtype != F32 else 4
        ta, tb = bool(rng.integers(2)), bool(rng.integers(2))
        thin = int(rng.integers(1, 65))
        wide = int(rng.integers(1, 40)) * 64 + int(rng.integers(0, 64))
        k = int(rng.integers(2, 40)) * 64 + (int(rng.integers(0, 64)) // v) * v
        if rng.integers(2):
            m, n = thin, wide
        else:
            m, n = wide, thin
        w_kmajor = tb if m <= n else not ta
        if not w_kmajor:
            k += int(rng.integers(1, v))  # a K that is not a whole number of packets
        bt = int(rng.integers(1, 4))
        alpha = float(rng.choice([1.0, 0.5, -2.0]))
        kind = ["none", "bias-row", "full"][rng.integers(3)]
        beta = 0.0 if kind == "none" else float(rng.choice([1.0, 2.0]))
        shared = kind != "full" and bool(rng.integers(2))
        what = (f"case {case}: {IDS[dtype]} {bt}x{m}x{n}x{k} ta={ta} tb={tb} alpha={alpha} "
                f"{kind} beta={beta} shared={shared}")
        outs, want = _run(lib, dev, orc, dtype, bt, m, n, k, ta, tb, alpha=alpha, beta=beta, cin_kind=kind,
                          shared_b=shared, reps=2, seed=case)
        assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8)), f"{what}: not deterministic"
        _check(orc, outs[0], want, dtype, what)
