"""Matrix products on the GPU against the CPU oracle: the reference's cases
(tests/test_mlu.py:238-300) and configs 4 and 5a of the benchmark at full
size.

Bars (north_star): float32 products within 2e-3 and bfloat16 / float16
products (float32 accumulation) within 1e-2, both as max |got - want| /
max |want| against the float64 product of the same stored inputs.  Full-size
products are checked on 4096 sampled entries computed exactly by the oracle
and, over the whole matrix, with Freivalds' test C x = A (B x) in float64.
"""

import numpy as np
import pytest

from _check import BF16, F16, F32

pytestmark = pytest.mark.gpu

DTYPES = [F32, BF16, F16]
BAR = {F32: 2e-3, BF16: 1e-2, F16: 1e-2}


def sample(orc, shape, dtype, seed, scale=1.0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * np.float32(scale)
    return orc.from_float(x, dtype)


def rel_err(orc, got, want, dtype):
    g = orc.to_float(got, dtype)
    w = orc.to_float(want, dtype) if want.dtype != np.float64 else want
    return float(np.max(np.abs(g - w)) / max(np.max(np.abs(w)), 1e-30))


def check(orc, got, want, dtype, what):
    e = rel_err(orc, got, want, dtype)
    assert e <= BAR[dtype], f"{what}: relative error {e:.3g} > {BAR[dtype]}"
    return e


def exact(orc, a, b, dtype, ta=False, tb=False):
    """float64 product of the stored operands (op = transpose when t*)."""
    A = orc.to_float(a, dtype)
    B = orc.to_float(b, dtype)
    A = np.swapaxes(A, -1, -2) if ta else A
    B = np.swapaxes(B, -1, -2) if tb else B
    return A @ B


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,k,n", [(37, 19, 23), (128, 64, 96), (200, 72, 136), (256, 256, 256),
                                   (64, 520, 24), (8, 16, 8)])
def test_mm_transposes(dev, ops, orc, dtype, ta, tb, m, k, n):
    a = sample(orc, (k, m) if ta else (m, k), dtype, 1)
    b = sample(orc, (n, k) if tb else (k, n), dtype, 3)
    da = dev.from_numpy(a, dtype=dtype)
    db = dev.from_numpy(b, dtype=dtype)
    got = ops.mm(da.t() if ta else da, db.t() if tb else db).numpy()
    want = orc.gemm(dtype, a, b, ta, tb)
    assert got.shape == (m, n)
    check(orc, got, want, dtype, f"mm ta={ta} tb={tb}")
    check(orc, got, exact(orc, a, b, dtype, ta, tb), dtype, "mm vs float64")


@pytest.mark.parametrize("dtype", DTYPES)
def test_addmm_bmm_matmul(dev, ops, orc, dtype):
    bias, a, b = sample(orc, (23,), dtype, 0), sample(orc, (37, 19), dtype, 1), sample(orc, (19, 23), dtype, 2)
    d = lambda x: dev.from_numpy(x, dtype=dtype)  # noqa: E731
    got = ops.addmm(d(bias), d(a), d(b), beta=0.5, alpha=2.0).numpy()
    check(orc, got, orc.gemm(dtype, a, b, alpha=2.0, beta=0.5, cin=bias), dtype, "addmm")
    want64 = 0.5 * orc.to_float(bias, dtype) + 2.0 * exact(orc, a, b, dtype)
    check(orc, got, want64, dtype, "addmm vs float64")
    x, y = sample(orc, (4, 9, 6), dtype, 4), sample(orc, (4, 6, 5), dtype, 5)
    check(orc, ops.bmm(d(x), d(y)).numpy(), orc.gemm(dtype, x, y), dtype, "bmm")
    w = sample(orc, (6, 5), dtype, 6)
    got = ops.matmul(d(x), d(w)).numpy()
    assert got.shape == (4, 9, 5)
    check(orc, got, exact(orc, x, w, dtype), dtype, "matmul 3d @ 2d")
    v = sample(orc, (2, 1, 6, 3), dtype, 7)
    got = ops.matmul(d(x), d(v)).numpy()
    assert got.shape == (2, 4, 9, 3)
    check(orc, got, exact(orc, x, v, dtype), dtype, "matmul broadcast batch")
    u = sample(orc, (6,), dtype, 8)
    got = ops.matmul(d(x), d(u)).numpy()
    assert got.shape == (4, 9)
    check(orc, got, exact(orc, x, u, dtype), dtype, "matmul 3d @ 1d")
    got = ops.matmul(d(u), d(w)).numpy()
    assert got.shape == (5,)
    check(orc, got, exact(orc, u, w, dtype), dtype, "matmul 1d @ 2d")


@pytest.mark.parametrize("dtype", DTYPES)
def test_linear(dev, ops, orc, dtype):
    x, w, b = sample(orc, (3, 5, 64), dtype, 0), sample(orc, (48, 64), dtype, 1), sample(orc, (48,), dtype, 2)
    d = lambda t: dev.from_numpy(t, dtype=dtype)  # noqa: E731
    want = exact(orc, x, w, dtype, tb=True)
    got = ops.linear(d(x), d(w), d(b)).numpy()
    assert got.shape == (3, 5, 48)
    check(orc, got, want + orc.to_float(b, dtype), dtype, "linear with bias")
    check(orc, ops.linear(d(x), d(w)).numpy(), want, dtype, "linear")
    got = ops.linear(d(x)[0, 0], d(w), d(b)).numpy()
    assert got.shape == (48,)
    check(orc, got, want[0, 0] + orc.to_float(b, dtype), dtype, "linear 1-d input")


@pytest.mark.parametrize("dtype", DTYPES)
def test_bmm_shapes(dev, ops, orc, dtype):
    for (bt, m, k, n) in ((32, 512, 64, 512), (1, 256, 4096, 1024), (3, 1, 7, 5)):
        a = sample(orc, (bt, m, k), dtype, 1, k ** -0.5)
        b = sample(orc, (bt, k, n), dtype, 2)
        got = ops.bmm(dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)).numpy()
        check(orc, got, exact(orc, a, b, dtype), dtype, f"bmm {bt}x{m}x{k}x{n}")
    a, b = sample(orc, (4, 9, 6), dtype, 3), sample(orc, (4, 5, 6), dtype, 4)
    got = ops.bmm(dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype).transpose(1, 2)).numpy()
    check(orc, got, exact(orc, a, b, dtype, tb=True), dtype, "bmm transposed operand")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k,n", [(2, 1024, 1024), (128, 1024, 256), (256, 4096, 1024),
                                   (1024, 4096, 128)])
def test_mm_shapes(dev, ops, orc, dtype, m, k, n):
    a, b = sample(orc, (m, k), dtype, 1), sample(orc, (k, n), dtype, 2)
    got = ops.mm(dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)).numpy()
    check(orc, got, exact(orc, a, b, dtype), dtype, f"mm {m}x{k}x{n}")


def test_k_zero_and_empty(dev, ops, orc):
    a = dev.from_numpy(np.zeros((4, 0), np.float32))
    b = dev.from_numpy(np.zeros((0, 3), np.float32))
    assert np.array_equal(ops.mm(a, b).numpy(), np.zeros((4, 3), np.float32))
    bias = dev.from_numpy(np.arange(3, dtype=np.float32))
    got = ops.addmm(bias, a, b, beta=2.0).numpy()
    assert np.array_equal(got, np.broadcast_to(np.arange(3, dtype=np.float32) * 2, (4, 3)))


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "bf16", "fp16"])
def test_product_planner_layouts(dev, ops, orc, dtype):
    """Layouts the product planner reads where they lie, or copies, with NaN
    in every stored element outside the views (a read outside the view
    shows up as NaN in the result)."""
    d = lambda t: dev.from_numpy(t, dtype=dtype)  # noqa: E731
    f = lambda t: orc.to_float(t, dtype)  # noqa: E731

    def no_nan(got, what):
        assert not np.isnan(f(got)).any(), f"{what}: read outside the view"

    # mm on column slices: leading dimensions wider than the rows.
    a = _padded(orc, (70, 40), 9, dtype, 1)
    b = _padded(orc, (40, 33), 7, dtype, 2)
    got = ops.mm(d(a)[:, :40], d(b)[:, :33]).numpy()
    no_nan(got, "mm column slices")
    check(orc, got, f(a)[:, :40] @ f(b)[:, :33], dtype, "mm column slices")
    # bmm over every other matrix of a stack (batch stride 2 m k).
    x = sample(orc, (8, 16, 24), dtype, 3)
    y = sample(orc, (8, 24, 12), dtype, 4)
    got = ops.bmm(d(x)[::2], d(y)[1::2]).numpy()
    check(orc, got, f(x)[::2] @ f(y)[1::2], dtype, "bmm strided batch")
    # [B, M, K] stored as transposes against a shared [K, N]: the batch does
    # not fold into the rows, the shared side is read with batch stride 0.
    xt = sample(orc, (5, 24, 16), dtype, 5)
    w = _padded(orc, (24, 20), 4, dtype, 6)
    got = ops.matmul(d(xt).transpose(1, 2), d(w)[:, :20]).numpy()
    assert got.shape == (5, 16, 20)
    no_nan(got, "matmul unfoldable batch")
    check(orc, got, np.swapaxes(f(xt), 1, 2) @ f(w)[:, :20], dtype, "matmul unfoldable batch")
    # [1, M, K] against [B, K, N] (left side shared), and [K] against [B, K, N].
    l1 = sample(orc, (1, 16, 24), dtype, 7)
    got = ops.matmul(d(l1), d(y)).numpy()
    assert got.shape == (8, 16, 12)
    check(orc, got, f(l1) @ f(y), dtype, "matmul shared left side")
    v = sample(orc, (24,), dtype, 8)
    got = ops.matmul(d(v), d(y)).numpy()
    assert got.shape == (8, 12)
    check(orc, got, f(v) @ f(y), dtype, "matmul vector @ stack")
    # Batch axes that do not merge into one stride ([2, 3] from a permuted
    # [3, 2] stack): copied dense first.
    s = sample(orc, (3, 2, 16, 24), dtype, 9)
    got = ops.matmul(d(s).permute(1, 0, 2, 3), d(y)[:6].view(2, 3, 24, 12)).numpy()
    want = np.swapaxes(f(s), 0, 1) @ f(y)[:6].reshape(2, 3, 24, 12)
    check(orc, got, want, dtype, "matmul unmergeable batch")
    # linear on a permuted 3-D input with bias, and with an input whose rows
    # are a column slice.
    xin = sample(orc, (6, 4, 32), dtype, 10)
    wt = sample(orc, (10, 32), dtype, 11)
    bias = sample(orc, (10,), dtype, 12)
    got = ops.linear(d(xin).permute(1, 0, 2), d(wt), d(bias)).numpy()
    assert got.shape == (4, 6, 10)
    want = np.swapaxes(f(xin), 0, 1) @ f(wt).T + f(bias)
    check(orc, got, want, dtype, "linear permuted input")
    xs = _padded(orc, (12, 32), 6, dtype, 13)
    got = ops.linear(d(xs)[:, :32], d(wt), d(bias)).numpy()
    no_nan(got, "linear column-slice input")
    check(orc, got, f(xs)[:, :32] @ f(wt).T + f(bias), dtype, "linear column-slice input")


def test_planner_empty_sums(dev, ops, orc):
    """An inner size of 0 gives zeros, or beta * bias; linear keeps the
    input's rows; addmm with beta = 0 never reads (or shape-checks) the
    bias."""
    z = lambda *s: dev.from_numpy(np.zeros(s, np.float32))  # noqa: E731
    bias = np.array([1.0, -2.0, 3.0], np.float32)
    got = ops.linear(z(4, 0), z(3, 0), dev.from_numpy(bias)).numpy()
    assert np.array_equal(got, np.broadcast_to(bias, (4, 3)))
    assert np.array_equal(ops.linear(z(2, 5, 0), z(3, 0)).numpy(), np.zeros((2, 5, 3), np.float32))
    assert np.array_equal(ops.matmul(z(2, 4, 0), z(0, 3)).numpy(), np.zeros((2, 4, 3), np.float32))
    a = np.random.default_rng(0).standard_normal((4, 6)).astype(np.float32)
    b = np.random.default_rng(1).standard_normal((6, 3)).astype(np.float32)
    odd_bias = dev.from_numpy(np.full((7,), np.nan, np.float32))
    got = ops.addmm(odd_bias, dev.from_numpy(a), dev.from_numpy(b), beta=0.0, alpha=2.0).numpy()
    check(orc, got, 2.0 * (a.astype(np.float64) @ b), F32, "addmm beta 0")


# ---- full-size configs ------------------------------------------------------------


def sampled_entries(orc, got, a, b, dtype, ta=False, tb=False, alpha=1.0, beta=0.0, cin=None,
                    count=4096, seed=0):
    m, n = got.shape[-2:]
    g = np.random.default_rng(seed)
    idx = np.stack([np.zeros(count, np.int64), g.integers(0, m, count), g.integers(0, n, count)], 1)
    want = orc.gemm_entries(dtype, a, b, idx, ta, tb, alpha, beta, cin)
    have = orc.to_float(got, dtype)[idx[:, 1], idx[:, 2]]
    return float(np.max(np.abs(have - want)) / np.max(np.abs(want)))


def freivalds(orc, got, a, b, dtype, ta=False, tb=False, bias=None):
    """max |C x - A (B x)| relative to max |A (B x)|, in float64."""
    x = np.random.default_rng(7).standard_normal(got.shape[-1])
    A = orc.to_float(a, dtype)
    B = orc.to_float(b, dtype)
    A = A.T if ta else A
    B = B.T if tb else B
    ref = A @ (B @ x)
    if bias is not None:
        ref = ref + float(orc.to_float(bias, dtype) @ x)
    lhs = orc.to_float(got, dtype) @ x
    return float(np.max(np.abs(lhs - ref)) / np.max(np.abs(ref)))


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
def test_config4_mm_4096(dev, ops, orc, dtype):
    K = 4096
    a = sample(orc, (K, K), dtype, 1, K ** -0.25)
    b = sample(orc, (K, K), dtype, 2, K ** -0.25)
    da, db = dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)
    got = ops.mm(da, db).numpy()
    assert sampled_entries(orc, got, a, b, dtype) <= BAR[dtype]
    assert freivalds(orc, got, a, b, dtype) <= BAR[dtype]
    # A stored [K, M] and read in place through .t()
    at = np.ascontiguousarray(a.T)
    got_t = ops.mm(dev.from_numpy(at, dtype=dtype).t(), db).numpy()
    assert sampled_entries(orc, got_t, at, b, dtype, ta=True) <= BAR[dtype]
    # addmm with a [4096] bias
    bias = sample(orc, (K,), dtype, 3)
    got_b = ops.addmm(dev.from_numpy(bias, dtype=dtype), da, db).numpy()
    assert sampled_entries(orc, got_b, a, b, dtype, beta=1.0, cin=bias) <= BAR[dtype]


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
def test_config4_linear(dev, ops, orc, dtype):
    x = sample(orc, (8192, 4096), dtype, 1, 4096 ** -0.25)
    w = sample(orc, (11008, 4096), dtype, 2, 4096 ** -0.25)
    b = sample(orc, (11008,), dtype, 3)
    got = ops.linear(dev.from_numpy(x, dtype=dtype), dev.from_numpy(w, dtype=dtype),
                     dev.from_numpy(b, dtype=dtype)).numpy()
    assert got.shape == (8192, 11008)
    assert sampled_entries(orc, got, x, w, dtype, tb=True, beta=1.0, cin=b) <= BAR[dtype]
    assert freivalds(orc, got, x, w, dtype, tb=True, bias=b) <= BAR[dtype]


def test_config5_bmm_bf16(dev, ops, orc):
    a = sample(orc, (64, 512, 128), BF16, 1, 128 ** -0.25)
    b = sample(orc, (64, 128, 512), BF16, 2, 128 ** -0.25)
    got = ops.bmm(dev.from_numpy(a, dtype=BF16), dev.from_numpy(b, dtype=BF16)).numpy()
    check(orc, got, exact(orc, a, b, BF16), BF16, "bmm 64x512x128x512")


# ---- the 256 x 256 four-wave kernel through the kernel C-ABI ---------------------


def _padded(orc, shape, pad, dtype, seed):
    """Random values of ``shape`` stored with ``pad`` extra NaN columns: the
    array returned is the storage, the view of its first columns the
    operand.  A kernel that reads the padding produces NaNs."""
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * np.float32(0.25)
    store = np.full(shape[:-1] + (shape[-1] + pad,), np.nan, np.float32)
    store[..., :shape[-1]] = x
    return orc.from_float(store, dtype)


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("bt,m,n,k", [(256, 256, 256, 256), (256, 256, 256, 384), (64, 512, 512, 320)],
                         ids=["big-tiles", "big-tiles-6-steps", "K-tail-fallback"])
def test_gemm_abi_padded_batched(amd, dev, orc, dtype, ta, tb, bt, m, n, k):
    """tp_amd_launch_gemm on a batch of products with padded leading
    dimensions (NaN padding), alpha = 0.5 and beta = 2 with a full Cin.  The
    first two shapes have one 256 x 256 tile per CU and four or six K tiles
    (the four-wave kernel: its loads of A for the K tile after next go out
    after each step's barrier, so the step pairs, the last two steps and
    the prologue all issue differently); the third, K = 320, is not a
    multiple of 128 and takes the eight-wave kernel."""
    lib = amd.load()
    pad, alpha, beta = 8, 0.5, 2.0
    a = _padded(orc, (bt, k, m) if ta else (bt, m, k), pad, dtype, 1)
    b = _padded(orc, (bt, n, k) if tb else (bt, k, n), pad, dtype, 2)
    cin = sample(orc, (bt, m, n), dtype, 3)
    lda, ldb = a.shape[-1], b.shape[-1]
    da, db, dc = (dev.from_numpy(x, dtype=dtype) for x in (a, b, cin))
    out = dev.empty((bt, m, n), dtype=dtype)
    st = lib.tp_amd_launch_gemm(0, dtype, bt, m, n, k, alpha, da.data_ptr, lda, a.shape[-2] * lda,
                                int(ta), db.data_ptr, ldb, b.shape[-2] * ldb, int(tb), beta,
                                dc.data_ptr, n, 1, m * n, out.data_ptr, n, m * n)
    assert st == 0, lib.tp_mlu_last_error()
    A = orc.to_float(a, dtype)[..., :(m if ta else k)]
    B = orc.to_float(b, dtype)[..., :(k if tb else n)]
    A = np.swapaxes(A, -1, -2) if ta else A
    B = np.swapaxes(B, -1, -2) if tb else B
    want = alpha * np.matmul(A, B) + beta * orc.to_float(cin, dtype)
    got = out.numpy()
    assert not np.isnan(orc.to_float(got, dtype)).any(), "padding leaked into the product"
    check(orc, got, want, dtype, f"gemm abi {bt}x{m}x{n}x{k} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("bt,m,n,k,pad,bcast", [(1, 515, 517, 509, 3, False), (1, 520, 512, 512, 3, False),
                                                (4, 300, 270, 255, 5, True)],
                         ids=["odd-K", "odd-ld", "odd-K-batch-broadcast"])
def test_gemm_abi_repacked_operands(amd, dev, orc, dtype, ta, tb, bt, m, n, k, pad, bcast):
    """Products whose operands the matrix-core kernels cannot read in place
    (odd K, odd leading dimensions, NaN in the padding) are repacked into
    aligned K-major copies, K padded with zeros: alpha = 0.5, beta = 2 with
    a full Cin, and in the batched case a B broadcast over the batch
    (stride 0)."""
    lib = amd.load()
    alpha, beta = 0.5, 2.0
    a = _padded(orc, (bt, k, m) if ta else (bt, m, k), pad, dtype, 1)
    b = _padded(orc, (1 if bcast else bt, n, k) if tb else (1 if bcast else bt, k, n), pad, dtype, 2)
    cin = sample(orc, (bt, m, n), dtype, 3)
    lda, ldb = a.shape[-1], b.shape[-1]
    da, db, dc = (dev.from_numpy(x, dtype=dtype) for x in (a, b, cin))
    out = dev.empty((bt, m, n), dtype=dtype)
    st = lib.tp_amd_launch_gemm(0, dtype, bt, m, n, k, alpha, da.data_ptr, lda, a.shape[-2] * lda,
                                int(ta), db.data_ptr, ldb, 0 if bcast else b.shape[-2] * ldb, int(tb),
                                beta, dc.data_ptr, n, 1, m * n, out.data_ptr, n, m * n)
    assert st == 0, lib.tp_mlu_last_error()
    A = orc.to_float(a, dtype)[..., :(m if ta else k)]
    B = orc.to_float(b, dtype)[..., :(k if tb else n)]
    A = np.swapaxes(A, -1, -2) if ta else A
    B = np.swapaxes(B, -1, -2) if tb else B
    want = alpha * np.matmul(A, B) + beta * orc.to_float(cin, dtype)
    got = out.numpy()
    assert not np.isnan(orc.to_float(got, dtype)).any(), "padding leaked into the product"
    check(orc, got, want, dtype, f"gemm abi {bt}x{m}x{n}x{k} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)], ids=["NN", "TT"])
def test_gemm_abi_odd_k_in_place_mn_major(amd, dev, orc, dtype, ta, tb):
    """An odd K with one operand stored M/N-contiguous and aligned: only the
    K-major operand is copied (zero-padded to whole packets), the other is
    read in place up to row K -- its storage has NaN rows right after row
    K, which must never reach the product."""
    lib = amd.load()
    bt, m, n, k, alpha, beta = 2, 264, 256, 509, 0.5, 2.0  # M, N and their lds whole packets
    g = np.random.default_rng(5)
    # the K-major operand: ordinary storage, ld = K
    km = g.standard_normal((bt, n, k) if tb else (bt, m, k)).astype(np.float32) * np.float32(0.25)
    km = orc.from_float(km, dtype)
    # the MN-major operand: [K + 5, MN + 8] per batch, NaN past row K and column MN
    mn_len = m if ta else n
    store = np.full((bt, k + 5, mn_len + 8), np.nan, np.float32)
    store[:, :k, :mn_len] = g.standard_normal((bt, k, mn_len)).astype(np.float32) * np.float32(0.25)
    mnm = orc.from_float(store, dtype)
    cin = sample(orc, (bt, m, n), dtype, 3)
    d_km, d_mn, dc = (dev.from_numpy(x, dtype=dtype) for x in (km, mnm, cin))
    out = dev.empty((bt, m, n), dtype=dtype)
    ld_mn, sb_mn = mn_len + 8, (k + 5) * (mn_len + 8)
    if ta:   # A stored [K, M] (M contiguous) in place, B stored [N, K] (K-major)
        args = (d_mn.data_ptr, ld_mn, sb_mn, 1, d_km.data_ptr, k, n * k, 1)
    else:    # A stored [M, K] (K-major), B stored [K, N] (N contiguous) in place
        args = (d_km.data_ptr, k, m * k, 0, d_mn.data_ptr, ld_mn, sb_mn, 0)
    st = lib.tp_amd_launch_gemm(0, dtype, bt, m, n, k, alpha, *args, beta, dc.data_ptr, n, 1, m * n,
                                out.data_ptr, n, m * n)
    assert st == 0, lib.tp_mlu_last_error()
    K = orc.to_float(km, dtype)
    Mv = orc.to_float(mnm, dtype)[:, :k, :mn_len]
    A = np.swapaxes(Mv, 1, 2) if ta else K
    B = np.swapaxes(K, 1, 2) if tb else Mv
    want = alpha * np.matmul(A, B) + beta * orc.to_float(cin, dtype)
    got = out.numpy()
    assert not np.isnan(orc.to_float(got, dtype)).any(), "rows past K leaked into the product"
    check(orc, got, want, dtype, f"odd K in place ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
def test_mm_skinny_odd_k(dev, ops, orc, dtype):
    """dX = dY W for a one-row dY and a vocabulary-sized odd K (W stored
    [K, N], N contiguous): read in place, checked against the float64
    product."""
    dy = sample(orc, (1, 3001), dtype, 21)
    w = sample(orc, (3001, 256), dtype, 22, 3001 ** -0.5)
    got = ops.mm(dev.from_numpy(dy, dtype=dtype), dev.from_numpy(w, dtype=dtype)).numpy()
    check(orc, got, exact(orc, dy, w, dtype), dtype, "skinny odd K")


@pytest.mark.parametrize("m,n,k,pad", [(1664, 1408, 520, 0), (1701, 1300, 776, 1)], ids=["aligned", "odd-M-ldc"])
def test_fp32_nn_as_transposed_product(amd, dev, ops, orc, m, n, k, pad):
    """float32 A [M, K] @ B [K, N] with enough tiles to fill the GPU runs as
    C^T = B^T A^T with C written transposed: ragged M and N, addmm's bias,
    a full Cin with beta = 2 through the kernel ABI into a C whose rows are
    ldc = N + pad apart (pad 1: rows not 16-byte aligned, element stores;
    the pad column must stay untouched), and a batch of two."""
    lib = amd.load()
    a, b = sample(orc, (m, k), F32, 31, k ** -0.5), sample(orc, (k, n), F32, 32)
    da, db = dev.from_numpy(a), dev.from_numpy(b)
    want = a.astype(np.float64) @ b.astype(np.float64)
    check(orc, ops.mm(da, db).numpy(), want, F32, "mm")
    bias = sample(orc, (n,), F32, 33)
    check(orc, ops.addmm(dev.from_numpy(bias), da, db, beta=0.5, alpha=2.0).numpy(),
          2.0 * want + 0.5 * bias.astype(np.float64), F32, "addmm")
    cin = sample(orc, (m, n), F32, 34)
    ldc = n + pad
    out = dev.from_numpy(np.full((m, ldc), 7.0, np.float32))
    st = lib.tp_amd_launch_gemm(0, F32, 1, m, n, k, 0.5, da.data_ptr, k, 0, 0, db.data_ptr, n, 0, 0, 2.0,
                                dev.from_numpy(cin).data_ptr, n, 1, 0, out.data_ptr, ldc, 0)
    assert st == 0, lib.tp_mlu_last_error()
    got = out.numpy()
    assert np.all(got[:, n:] == 7.0), "the pad column was written"
    check(orc, np.ascontiguousarray(got[:, :n]), 0.5 * want + 2.0 * cin.astype(np.float64), F32, "full Cin")
    x, y = sample(orc, (2, m, k), F32, 35, k ** -0.5), sample(orc, (2, k, n), F32, 36)
    check(orc, ops.bmm(dev.from_numpy(x), dev.from_numpy(y)).numpy(),
          np.matmul(x.astype(np.float64), y.astype(np.float64)), F32, "bmm")


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["fp32", "bf16"])
def test_mm_2047_cube(dev, ops, orc, dtype):
    """mm 2047^3 (odd everything) through ops.mm, checked on sampled
    entries and with Freivalds' test."""
    a = sample(orc, (2047, 2047), dtype, 11, 0.05)
    b = sample(orc, (2047, 2047), dtype, 12, 0.05)
    got = ops.mm(dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)).numpy()
    assert sampled_entries(orc, got, a, b, dtype) <= BAR[dtype]
    assert freivalds(orc, got, a, b, dtype) <= BAR[dtype]


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("cin_kind", ["full", "bias-row"])
def test_gemm_fp32_split_k(amd, dev, orc, ta, tb, cin_kind):
    """A float32 product with few 128 x 128 tiles and a long K (256 x 384
    outputs, K = 4096: 6 tiles) is split over K into float32 partials that are
    added in slice order: the result matches the float64 product at the fp32
    bar with alpha = 0.5, beta = 2 and a full Cin or a row-broadcast bias,
    NaN-padded leading dimensions, and two runs give the same bits."""
    lib = amd.load()
    m, n, k, pad, alpha, beta = 256, 384, 4096, 4, 0.5, 2.0
    a = _padded(orc, (k, m) if ta else (m, k), pad, F32, 7)
    b = _padded(orc, (n, k) if tb else (k, n), pad, F32, 8)
    if cin_kind == "full":
        cin = sample(orc, (m, n), F32, 9)
        rs, cs = n, 1
        cin_f = cin
    else:
        cin = sample(orc, (n,), F32, 9)
        rs, cs = 0, 1
        cin_f = np.broadcast_to(cin, (m, n))
    da, db, dc = dev.from_numpy(a), dev.from_numpy(b), dev.from_numpy(cin)
    A = a[:, :m] if ta else a[:, :k]
    B = b[:, :k] if tb else b[:, :n]
    A = A.T if ta else A
    B = B.T if tb else B
    want = alpha * (A.astype(np.float64) @ B.astype(np.float64)) + beta * cin_f.astype(np.float64)
    outs = []
    for _ in range(2):
        out = dev.empty((m, n), dtype=F32)
        st = lib.tp_amd_launch_gemm(0, F32, 1, m, n, k, alpha, da.data_ptr, a.shape[-1], 0, int(ta),
                                    db.data_ptr, b.shape[-1], 0, int(tb), beta, dc.data_ptr, rs, cs, 0,
                                    out.data_ptr, n, 0)
        assert st == 0, lib.tp_mlu_last_error()
        outs.append(out.numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "split-K sum is not deterministic"
    check(orc, outs[0], want, F32, f"split-K fp32 ta={ta} tb={tb} {cin_kind}")


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("cin_kind", ["none", "full", "bias-row"])
@pytest.mark.parametrize("k", [4096, 4000, 3001])
def test_gemm16_split_k(amd, dev, orc, dtype, ta, tb, cin_kind, k):
    """A 16-bit product with few 128 x 128 tiles and a long K (200 x 384
    outputs: 6 tiles) is split over K into float32 partials, added in slice
    order and rounded once: within the 16-bit bar of the float64 product
    with alpha = 0.5 and beta = 2 (a full Cin or a row-broadcast bias),
    NaN-padded leading dimensions, a ragged M, and two runs giving the same
    bits.  K = 4096 splits into four slices of 1024; K = 4000 into three of
    1024 and a last of 928; K = 3001 (odd: K-major operands are copied with
    zero padding first, M/N-major ones read in place) into 1536 and 1465."""
    lib = amd.load()
    m, n, pad, alpha = 200, 384, 8, 0.5
    a = _padded(orc, (k, m) if ta else (m, k), pad, dtype, 17)
    b = _padded(orc, (n, k) if tb else (k, n), pad, dtype, 18)
    A = orc.to_float(a, dtype).astype(np.float64)
    B = orc.to_float(b, dtype).astype(np.float64)
    A = A[:, :m].T if ta else A[:, :k]
    B = B[:, :k].T if tb else B[:, :n]
    want = alpha * (A @ B)
    if cin_kind == "none":
        beta, cin, rs, cs = 0.0, None, 0, 0
    elif cin_kind == "full":
        beta, cin, rs, cs = 2.0, sample(orc, (m, n), dtype, 19), n, 1
        want = want + beta * orc.to_float(cin, dtype)
    else:
        beta, cin, rs, cs = 2.0, sample(orc, (n,), dtype, 19), 0, 1
        want = want + beta * orc.to_float(cin, dtype)
    da, db = dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)
    dc = dev.from_numpy(cin, dtype=dtype) if cin is not None else None
    outs = []
    for _ in range(2):
        out = dev.empty((m, n), dtype=dtype)
        st = lib.tp_amd_launch_gemm(0, dtype, 1, m, n, k, alpha, da.data_ptr, a.shape[-1], 0, int(ta),
                                    db.data_ptr, b.shape[-1], 0, int(tb), beta,
                                    dc.data_ptr if dc is not None else 0, rs, cs, 0, out.data_ptr, n, 0)
        assert st == 0, lib.tp_mlu_last_error()
        outs.append(out.numpy())
    assert np.array_equal(outs[0], outs[1]), "split-K sum is not deterministic"
    assert not np.isnan(orc.to_float(outs[0], dtype)).any(), "padding leaked into the product"
    check(orc, outs[0], want, dtype, f"16-bit split-K k={k} ta={ta} tb={tb} {cin_kind}")


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("k", [64, 128])
@pytest.mark.parametrize("cin_kind", ["none", "bias-row", "full"])
@pytest.mark.parametrize("bt,m,n", [(64, 512, 512), (257, 256, 256)], ids=["xcd-order", "plain-order"])
def test_gemm_abi_small_k(amd, dev, orc, dtype, ta, tb, k, cin_kind, bt, m, n):
    """Batched 16-bit products with K = 64 or 128 (attention-sized: the
    one-barrier kernel that holds all of K in LDS) through
    tp_amd_launch_gemm: NaN-padded leading dimensions, the four layouts,
    alpha = 0.5 and beta = 0 / a per-column bias shared by the batch / a full
    Cin with beta = 2.  64 x 512 x 512 has 256 tiles (numbered so each batch
    stays on one XCD); 257 x 256 x 256 has a tile count that is not a
    multiple of 8 and is numbered in order."""
    lib = amd.load()
    pad, alpha = 8, 0.5
    a = _padded(orc, (bt, k, m) if ta else (bt, m, k), pad, dtype, 11)
    b = _padded(orc, (bt, n, k) if tb else (bt, k, n), pad, dtype, 12)
    lda, ldb = a.shape[-1], b.shape[-1]
    da, db = dev.from_numpy(a, dtype=dtype), dev.from_numpy(b, dtype=dtype)
    A = orc.to_float(a, dtype)[..., :(m if ta else k)]
    B = orc.to_float(b, dtype)[..., :(k if tb else n)]
    A = np.swapaxes(A, -1, -2) if ta else A
    B = np.swapaxes(B, -1, -2) if tb else B
    want = alpha * np.matmul(A, B)
    if cin_kind == "none":
        beta, cin, rs, cs, sb = 0.0, None, 0, 0, 0
    elif cin_kind == "bias-row":
        beta, cin, rs, cs, sb = 1.0, sample(orc, (n,), dtype, 13), 0, 1, 0
        want = want + orc.to_float(cin, dtype)
    else:
        beta, cin, rs, cs, sb = 2.0, sample(orc, (bt, m, n), dtype, 13), n, 1, m * n
        want = want + beta * orc.to_float(cin, dtype)
    dc = dev.from_numpy(cin, dtype=dtype) if cin is not None else None
    cptr = dc.data_ptr if dc is not None else 0
    out = dev.empty((bt, m, n), dtype=dtype)
    st = lib.tp_amd_launch_gemm(0, dtype, bt, m, n, k, alpha, da.data_ptr, lda, a.shape[-2] * lda,
                                int(ta), db.data_ptr, ldb, b.shape[-2] * ldb, int(tb), beta,
                                cptr, rs, cs, sb, out.data_ptr, n, m * n)
    assert st == 0, lib.tp_mlu_last_error()
    got = out.numpy()
    assert not np.isnan(orc.to_float(got, dtype)).any(), "padding leaked into the product"
    check(orc, got, want, dtype, f"small-K gemm {bt}x{m}x{n}x{k} ta={ta} tb={tb} {cin_kind}")


@pytest.mark.parametrize("m,n,k,dtype", [(64, 64, 64, F32), (512, 512, 512, F32), (512, 512, 512, BF16),
                                         (4096, 4096, 256, BF16), (1024, 1024, 1024, F32)],
                         ids=["fma-fp32", "mfma-fp32", "mfma-bf16", "big-bf16", "mfma-fp32-1024"])
def test_nan_and_inf_propagate(dev, ops, orc, m, n, k, dtype):
    """NaN and infinities in the operands reach the same entries of C as
    in IEEE arithmetic: a NaN fills its row (or column), an infinity fills
    its row except where it meets a 0 (NaN) -- on the FMA kernel, the MFMA
    kernels and the big bf16 kernel."""
    rng = np.random.default_rng(k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    a[3, 5], a[7, 9], b[9, 11] = np.nan, np.inf, 0.0
    a[20, :] = 0.0
    a[20, 30] = -np.inf
    b[40, 50] = np.nan
    A, B = orc.from_float(a, dtype), orc.from_float(b, dtype)
    got = orc.to_float(ops.mm(dev.from_numpy(A, dtype=dtype), dev.from_numpy(B, dtype=dtype)).numpy(), dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        want = orc.to_float(A, dtype) @ orc.to_float(B, dtype)
    assert np.array_equal(np.isnan(got), np.isnan(want)), "NaN in other places"
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf), "infinities in other places"
    assert np.array_equal(got[inf], want[inf]), "signs of the infinities"

