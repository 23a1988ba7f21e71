"""Elementwise operators on the GPU against the CPU oracle (same seeded
inputs): binary arithmetic with broadcasting, in-place and scalar forms,
unary math, activations and their backward kernels.

Mirrors the reference's cases (tests/test_mlu.py:137-233) and runs config 2
of the benchmark at full size ([8192, 8192] with row and column
broadcasts).  Tolerances are stated in tests/_check.py.
"""

import numpy as np
import pytest

from _check import BF16, F16, F32, assert_bitexact, assert_elementwise

pytestmark = pytest.mark.gpu

DTYPES = [F32, BF16, F16]
ADD, MUL, DIV = 0, 1, 2


def sample(orc, shape, dtype, seed=0, low=None, high=None):
    g = np.random.default_rng(seed)
    if low is None:
        x = g.standard_normal(shape, dtype=np.float32)
    else:
        x = g.uniform(low, high, size=shape).astype(np.float32)
    return orc.from_float(x, dtype)


def up(dev, arr, dtype):
    return dev.from_numpy(arr, dtype=dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("sa,sb", [((4, 1, 5), (3, 1)), ((6, 4), (4,)), ((33, 17), (33, 1)),
                                   ((64, 128), (64, 128)), ((5, 7), ()), ((1, 9), (8, 1)),
                                   ((4, 6, 16), (4, 1, 16)), ((3, 1, 24), (1, 5, 24)),
                                   ((2, 3, 4, 8), (3, 1, 8))])
def test_binary_with_broadcasting(dev, ops, orc, dtype, sa, sb):
    a = sample(orc, sa, dtype, 0)
    b = sample(orc, sb, dtype, 1, 0.5, 2.0)
    da, db = up(dev, a, dtype), up(dev, b, dtype)
    assert_bitexact(ops.add(da, db).numpy(), orc.binary(ADD, dtype, a, b, 1.0), "add")
    assert_bitexact(ops.sub(da, db).numpy(), orc.binary(ADD, dtype, a, b, -1.0), "sub")
    assert_elementwise(ops.sub(da, db, alpha=2).numpy(), orc.binary(ADD, dtype, a, b, -2.0),
                       dtype, "sub alpha=2", max_ulp=1)
    assert_elementwise(ops.add(da, db, alpha=0.5).numpy(), orc.binary(ADD, dtype, a, b, 0.5),
                       dtype, "add alpha=0.5", max_ulp=1)
    assert_bitexact(ops.mul(da, db).numpy(), orc.binary(MUL, dtype, a, b), "mul")
    assert_bitexact(ops.div(da, db).numpy(), orc.binary(DIV, dtype, a, b), "div")


@pytest.mark.parametrize("dtype", DTYPES)
def test_scalar_forms_and_host_scalars(dev, ops, orc, dtype):
    a = sample(orc, (8, 3), dtype)
    d = up(dev, a, dtype)
    cases = [
        (ops.add_scalar(d, 2), orc.affine(dtype, a, 1.0, 2.0)),
        (ops.mul_scalar(d, 3), orc.affine(dtype, a, 3.0, 0.0)),
        # division multiplies by the float32 reciprocal (BinaryKernels.cpp:231)
        (ops.div_scalar(d, 3), orc.affine(dtype, a, np.float32(1.0 / 3.0), 0.0)),
        (ops.rsub_scalar(d, 1), orc.affine(dtype, a, -1.0, 1.0)),
        (ops.sub_scalar(d, 2, alpha=3), orc.affine(dtype, a, 1.0, -6.0)),
        (ops.mul(d, np.float32(2.0)), orc.affine(dtype, a, 2.0, 0.0)),
        (ops.add(np.float32(2.0), d), orc.affine(dtype, a, 1.0, 2.0)),
        (ops.sub(np.float32(2.0), d), orc.affine(dtype, a, -1.0, 2.0)),
        (ops.div(d, np.float32(4.0)), orc.affine(dtype, a, 0.25, 0.0)),
    ]
    for i, (got, want) in enumerate(cases):
        assert_elementwise(got.numpy(), want, dtype, f"case {i}", max_ulp=1)


@pytest.mark.parametrize("dtype", DTYPES)
def test_in_place(dev, ops, orc, dtype):
    a, b = sample(orc, (6, 4), dtype), sample(orc, (4,), dtype, 2, 0.5, 2.0)
    d, db = up(dev, a, dtype), up(dev, b, dtype)
    ops.add_(d, db, alpha=0.5)
    ops.mul__scalar(d, 2)
    ops.sub_(d, db)
    ops.div__scalar(d, 3)
    ops.mul_(d, db)
    ops.div_(d, db)
    ops.add__scalar(d, 1.5, alpha=2)
    want = orc.binary(ADD, dtype, a, b, 0.5)
    want = orc.affine(dtype, want, 2.0, 0.0)
    want = orc.binary(ADD, dtype, want, b, -1.0)
    want = orc.affine(dtype, want, np.float32(1.0 / 3.0), 0.0)
    want = orc.binary(MUL, dtype, want, b)
    want = orc.binary(DIV, dtype, want, b)
    want = orc.affine(dtype, want, 1.0, 3.0)
    assert_elementwise(d.numpy(), want, dtype, "in-place chain", max_ulp=1)


@pytest.mark.parametrize("dtype", DTYPES)
def test_scalar_forms_of_strided_operands(dev, ops, orc, dtype):
    base = sample(orc, (1, 5), dtype)
    expanded = up(dev, base, dtype).expand(4, 5)
    want = orc.affine(dtype, np.broadcast_to(base, (4, 5)).copy(), 3.0, 0.0)
    assert_elementwise(ops.mul_scalar(expanded, 3).numpy(), want, dtype, "expanded * 3", max_ulp=1)
    a = sample(orc, (6, 8), dtype)
    d = up(dev, a, dtype)
    ops.mul__scalar(d.t(), 0.5)
    ops.add__scalar(d[:, ::2], 1.0)
    want = orc.affine(dtype, a, 0.5, 0.0)
    want[:, ::2] = orc.affine(dtype, np.ascontiguousarray(want[:, ::2]), 1.0, 1.0)
    assert_elementwise(d.numpy(), want, dtype, "strided in-place", max_ulp=1)


@pytest.mark.parametrize("dtype", DTYPES)
def test_row_padded_views_in_packets(dev, ops, orc, dtype):
    """A view whose rows are a prefix of longer rows (inner dimension
    contiguous, row starts 16-byte aligned) against an operand repeated
    along the inner dimension, and a unary op on such a view: the inner
    dimension moves in 16-byte packets.  Bit-exact against the oracle."""
    big = sample(orc, (4, 6, 32), dtype, 5)
    col = sample(orc, (4, 6, 1), dtype, 6, 0.5, 2.0)
    d = up(dev, big, dtype)
    view = d[:, :, 0:16]
    a = np.ascontiguousarray(big[:, :, 0:16])
    assert_bitexact(ops.add(view, up(dev, col, dtype)).numpy(), orc.binary(ADD, dtype, a, col, 1.0), "view + column")
    assert_bitexact(ops.mul(up(dev, col, dtype), view).numpy(), orc.binary(MUL, dtype, col, a), "column * view")
    assert_bitexact(ops.relu(view).numpy(), orc.unary(8, dtype, a), "relu of a view")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(64, 64), (300, 200), (1000, 77), (5, 130)])
def test_transposed_operands_in_tiles(dev, ops, orc, dtype, rows, cols):
    """Binary ops with a transposed (column-major) operand into a row-major
    output, which run through LDS tiles of 64 x 64: either side transposed,
    both, a transposed operand with a broadcast row, a transposed slice of
    a wider matrix at an odd and at an even element offset (the same
    kernel; the two offsets give different alignments of the tile loads),
    and an in-place update.  Bit-exact against the oracle."""
    x = sample(orc, (cols, rows), dtype, 1)       # stored [cols][rows]; used as x.T
    y = sample(orc, (rows, cols), dtype, 2)
    z = sample(orc, (cols, rows), dtype, 3, 0.5, 2.0)
    bias = sample(orc, (1, cols), dtype, 4)
    dx, dy, dz = up(dev, x, dtype), up(dev, y, dtype), up(dev, z, dtype)
    xt, zt = np.ascontiguousarray(x.T), np.ascontiguousarray(z.T)
    assert_bitexact(ops.add(dx.t(), dy).numpy(), orc.binary(ADD, dtype, xt, y, 1.0), "x.t() + y")
    assert_bitexact(ops.mul(dy, dx.t()).numpy(), orc.binary(MUL, dtype, y, xt), "y * x.t()")
    assert_bitexact(ops.div(dx.t(), dz.t()).numpy(), orc.binary(DIV, dtype, xt, zt), "x.t() / z.t()")
    assert_bitexact(ops.add(dx.t(), up(dev, bias, dtype)).numpy(), orc.binary(ADD, dtype, xt, bias, 1.0),
                    "x.t() + row")
    wide = sample(orc, (cols, rows + 9), dtype, 5)
    wt = np.ascontiguousarray(wide[:, 3:3 + rows].T)
    got = ops.add(up(dev, wide, dtype)[:, 3:3 + rows].t(), dy).numpy()
    assert_bitexact(got, orc.binary(ADD, dtype, wt, y, 1.0), "slice.t() + y")
    wide2 = sample(orc, (cols, rows + 10), dtype, 6)
    w2 = np.ascontiguousarray(wide2[:, 2:2 + rows].T)
    got = ops.mul(dy, up(dev, wide2, dtype)[:, 2:2 + rows].t()).numpy()
    assert_bitexact(got, orc.binary(MUL, dtype, y, w2), "y * even-slice.t()")
    ops.add_(dy, dx.t())
    assert_bitexact(dy.numpy(), orc.binary(ADD, dtype, y, xt, 1.0), "y.add_(x.t())")


def test_strided_operands(dev, ops, orc):
    a = sample(orc, (5, 7), F32)
    d = up(dev, a, F32)
    assert_bitexact(ops.add(d.t(), d.t()).numpy(), orc.binary(ADD, F32, a.T, a.T), "t + t")
    got = ops.mul(d[:, ::2][:, :3], d[:, 1::2]).numpy()
    assert_bitexact(got, orc.binary(MUL, F32, a[:, ::2][:, :3], a[:, 1::2]), "strided mul")


def test_integer_math_is_declined(dev, ops):
    tensor = __import__("importlib").import_module("tensorplay-mlu_amd.tensor")
    x = dev.from_numpy(np.arange(10, dtype=np.int64))
    with pytest.raises(tensor.DeclinedError):
        ops.mul(x, x)
    with pytest.raises(tensor.DeclinedError):
        ops.mul_scalar(x, 3)


UNARY = {  # name -> (oracle op code, input transform)
    "exp": (0, None), "log": (1, "pos"), "sqrt": (2, "pos"), "rsqrt": (3, "pos"),
    "neg": (4, None), "abs": (5, None), "relu": (8, None), "sigmoid": (9, None),
    "tanh": (10, None), "silu": (11, None),
}
EXACT_UNARY = {"neg", "abs", "relu", "sqrt"}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("name", sorted(UNARY))
def test_unary(dev, ops, orc, dtype, name):
    code, transform = UNARY[name]
    x = np.random.default_rng(3).standard_normal((33, 17)).astype(np.float32)
    if transform == "pos":
        x = np.abs(x) + 0.1
    a = orc.from_float(x, dtype)
    got = getattr(ops, name)(up(dev, a, dtype)).numpy()
    want = orc.unary(code, dtype, a)
    if name in EXACT_UNARY:
        assert_bitexact(got, want, name)
    else:
        assert_elementwise(got, want, dtype, name)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("exponent", [2, 1, 0, 0.5, -0.5, 3, 1.7])
def test_pow_scalar(dev, ops, orc, dtype, exponent):
    x = np.abs(np.random.default_rng(4).standard_normal((6, 9)).astype(np.float32)) + 0.5
    a = orc.from_float(x, dtype)
    got = ops.pow_scalar(up(dev, a, dtype), exponent).numpy()
    want = orc.unary(7, dtype, a, float(exponent))
    assert_elementwise(got, want, dtype, f"pow {exponent}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_activations(dev, ops, orc, dtype):
    a = sample(orc, (16, 32), dtype)
    d = up(dev, a, dtype)
    assert_elementwise(ops.gelu(d).numpy(), orc.unary(12, dtype, a), dtype, "gelu")
    assert_elementwise(ops.gelu(d, "tanh").numpy(), orc.unary(13, dtype, a), dtype, "gelu tanh")
    assert_elementwise(ops.silu(d).numpy(), orc.unary(11, dtype, a), dtype, "silu")
    r = up(dev, a.copy(), dtype)
    ops.relu_(r)
    assert_bitexact(r.numpy(), orc.unary(8, dtype, a), "relu_")


SPECIAL = np.float32([0.0, -0.0, 1.0, -1.0, 1.5, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-40,
                      -1e-40, 1.17549435e-38, 65504.0, 6.1e-5, 5.96e-8, 1e30, 0.5, 2.0, 3.0])


@pytest.mark.parametrize("dtype", DTYPES)
def test_special_values_bitexact(dev, ops, orc, dtype):
    """Every pair of special operands -- signed zeros, infinities, NaN,
    float32 subnormals, the largest float32 and float16 values, the
    smallest float16 normal and subnormal, as stored in the dtype -- through
    the arithmetic, scalar, sign and threshold ops: the same bits as the
    oracle, with a NaN anywhere the oracle has one and the sign of every
    zero kept."""
    with np.errstate(over="ignore"):
        v = orc.from_float(SPECIAL, dtype)
    a, b = np.repeat(v, len(v)), np.tile(v, len(v))
    da, db = up(dev, a, dtype), up(dev, b, dtype)
    cases = [("add", ops.add(da, db), orc.binary(ADD, dtype, a, b, 1.0)),
             ("sub", ops.sub(da, db), orc.binary(ADD, dtype, a, b, -1.0)),
             ("add alpha=2", ops.add(da, db, alpha=2), orc.binary(ADD, dtype, a, b, 2.0)),
             ("mul", ops.mul(da, db), orc.binary(MUL, dtype, a, b)),
             ("div", ops.div(da, db), orc.binary(DIV, dtype, a, b)),
             ("mul_scalar 3", ops.mul_scalar(da, 3), orc.affine(dtype, a, 3.0, 0.0)),
             ("div_scalar 3", ops.div_scalar(da, 3), orc.affine(dtype, a, np.float32(1.0 / 3.0), 0.0)),
             ("add_scalar 1", ops.add_scalar(da, 1), orc.affine(dtype, a, 1.0, 1.0)),
             ("neg", ops.neg(da), orc.unary(4, dtype, a)),
             ("abs", ops.abs(da), orc.unary(5, dtype, a)),
             ("relu", ops.relu(da), orc.unary(8, dtype, a)),
             ("square", ops.pow_scalar(da, 2), orc.unary(6, dtype, a)),
             ("threshold_backward", ops.threshold_backward(db, da, 0), orc.activation_backward(0, dtype, b, a, 0.0))]
    for what, got, want in cases:
        g, w = orc.to_float(got.numpy(), dtype), orc.to_float(want, dtype)
        nan = np.isnan(w)
        assert np.array_equal(np.isnan(g), nan), f"{what}: NaN in other places"
        assert np.array_equal(g[~nan], w[~nan]), f"{what}: values differ"
        assert np.array_equal(np.signbit(g[~nan]), np.signbit(w[~nan])), f"{what}: signs of zero differ"


def test_gelu_erf_form_float32_sweep(dev, ops, orc):
    """gelu (erf form) and its backward in float32 over a dense grid of
    [-14, 14] and special values: the rtol 1e-5 bar everywhere, and gelu
    within 16 ulps of the correctly rounded value wherever it is a normal
    float (|x| <= 12), the bound the float32 normal CDF is built to (it keeps
    the rounding error of x / sqrt 2, which a plain erfcf(-x / sqrt 2) drops:
    ~200 ulps at |x| > 8)."""
    x = np.concatenate([np.linspace(-14, 14, (1 << 20) + 1, dtype=np.float32),
                        np.float32([0.0, -0.0, 1e-30, -1e-30, 1e30, -1e30])])
    dx_ = up(dev, x, F32)
    got = ops.gelu(dx_).numpy()
    want = orc.unary(12, F32, x)
    assert_elementwise(got, want, F32, "gelu")
    normal = np.abs(x) <= 12
    assert_elementwise(got[normal], want[normal], F32, "gelu, |x| <= 12", max_ulp=16)
    assert np.array_equal(np.signbit(got[want == 0]), np.signbit(want[want == 0])), "signs of zero results"
    ones = np.ones_like(x)
    gb = ops.gelu_backward(up(dev, ones, F32), dx_).numpy()
    assert_elementwise(gb, orc.activation_backward(3, F32, ones, x), F32, "gelu_backward")
    # infinities and NaN: x Phi(x) is inf at +inf, NaN at -inf (-inf * 0) and NaN
    special = np.float32([np.inf, -np.inf, np.nan])
    got_s = ops.gelu(up(dev, special, F32)).numpy()
    assert got_s[0] == np.inf and np.isnan(got_s[1]) and np.isnan(got_s[2])
    assert np.array_equal(np.isnan(orc.unary(12, F32, special)), np.isnan(got_s))


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
def test_narrow_float_math_at_every_value(dev, ops, orc, dtype):
    """Every transcendental unary op and activation backward at every finite
    16-bit value, within one storage ulp of the oracle (NaN where it gives
    NaN).  The backward ops take an upstream gradient of 1, so dx is the
    derivative rounded once.  bfloat16 reaches float32's exponent range, so
    this covers the subnormal results of exp, sigmoid, silu and both gelu
    forms far out in their tails and sqrt of subnormal inputs."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    every = bits if dtype == BF16 else bits.view(np.float16)
    a = every[np.isfinite(orc.to_float(every, dtype))]
    d = up(dev, a, dtype)
    one = orc.from_float(np.ones(a.shape, np.float32), dtype)
    dg = up(dev, one, dtype)
    y_sig, y_tanh = orc.unary(9, dtype, a), orc.unary(10, dtype, a)
    cases = [("exp", ops.exp(d), orc.unary(0, dtype, a)),
             ("log", ops.log(d), orc.unary(1, dtype, a)),
             ("sqrt", ops.sqrt(d), orc.unary(2, dtype, a)),
             ("rsqrt", ops.rsqrt(d), orc.unary(3, dtype, a)),
             ("sigmoid", ops.sigmoid(d), y_sig),
             ("tanh", ops.tanh(d), y_tanh),
             ("silu", ops.silu(d), orc.unary(11, dtype, a)),
             ("gelu", ops.gelu(d), orc.unary(12, dtype, a)),
             ("gelu tanh", ops.gelu(d, "tanh"), orc.unary(13, dtype, a)),
             ("sigmoid_backward", ops.sigmoid_backward(dg, up(dev, y_sig, dtype)),
              orc.activation_backward(1, dtype, one, y_sig)),
             ("tanh_backward", ops.tanh_backward(dg, up(dev, y_tanh, dtype)),
              orc.activation_backward(2, dtype, one, y_tanh)),
             ("gelu_backward", ops.gelu_backward(dg, d), orc.activation_backward(3, dtype, one, a)),
             ("gelu_backward tanh", ops.gelu_backward(dg, d, "tanh"), orc.activation_backward(4, dtype, one, a)),
             ("silu_backward", ops.silu_backward(dg, d), orc.activation_backward(5, dtype, one, a))]
    for what, got, want in cases:
        got = got.numpy()
        nan_g, nan_w = np.isnan(orc.to_float(got, dtype)), np.isnan(orc.to_float(want, dtype))
        assert np.array_equal(nan_g, nan_w), f"{what}: NaN at {int((nan_g != nan_w).sum())} inputs differs"
        assert_elementwise(got[~nan_w], want[~nan_w], dtype, what)


def test_math_tails_float32(dev, ops, orc):
    """float32 tails: sigmoid and silu far below -88.7 (where 1 / (1 + e^-x)
    would give 0 instead of a subnormal), and the tanh-form gelu derivative at
    |x| up to 1e30 (where x^2 overflows float32), against the oracle; the
    derivative must be finite there."""
    x = np.concatenate([-np.geomspace(80.0, 110.0, 4001, dtype=np.float32),
                        np.float32([1e19, -1e19, 2e19, -2e19, 1e30, -1e30, 3.4e38, -3.4e38])])
    d = up(dev, x, F32)
    assert_elementwise(ops.sigmoid(d).numpy(), orc.unary(9, F32, x), F32, "sigmoid", max_ulp=2)
    assert_elementwise(ops.silu(d).numpy(), orc.unary(11, F32, x), F32, "silu")
    ones = np.ones_like(x)
    got = ops.gelu_backward(up(dev, ones, F32), d, "tanh").numpy()
    assert np.isfinite(got).all(), "gelu tanh backward: NaN or inf"
    assert_elementwise(got, orc.activation_backward(4, F32, ones, x), F32, "gelu_backward tanh")


@pytest.mark.parametrize("dtype", DTYPES)
def test_activation_backward(dev, ops, orc, dtype):
    x = sample(orc, (37, 29), dtype, 5)
    g = sample(orc, (37, 29), dtype, 6)
    dx_, dg = up(dev, x, dtype), up(dev, g, dtype)
    assert_bitexact(ops.threshold_backward(dg, dx_, 0).numpy(),
                    orc.activation_backward(0, dtype, g, x, 0.0), "threshold_backward")
    assert_bitexact(ops.threshold_backward(dg, dx_, 0.3).numpy(),
                    orc.activation_backward(0, dtype, g, x, float(orc.to_float(orc.from_float(np.float32([0.3]), dtype), dtype)[0])),
                    "threshold_backward 0.3")
    y = orc.unary(9, dtype, x)
    assert_elementwise(ops.sigmoid_backward(dg, up(dev, y, dtype)).numpy(),
                       orc.activation_backward(1, dtype, g, y), dtype, "sigmoid_backward")
    t = orc.unary(10, dtype, x)
    assert_elementwise(ops.tanh_backward(dg, up(dev, t, dtype)).numpy(),
                       orc.activation_backward(2, dtype, g, t), dtype, "tanh_backward")
    assert_elementwise(ops.gelu_backward(dg, dx_).numpy(),
                       orc.activation_backward(3, dtype, g, x), dtype, "gelu_backward")
    assert_elementwise(ops.gelu_backward(dg, dx_, "tanh").numpy(),
                       orc.activation_backward(4, dtype, g, x), dtype, "gelu_backward tanh")
    assert_elementwise(ops.silu_backward(dg, dx_).numpy(),
                       orc.activation_backward(5, dtype, g, x), dtype, "silu_backward")


def test_large_narrow_float_elementwise(dev, ops, orc):
    # The reference's 64 MiB narrow-float case (tests/test_mlu.py:336-341).
    for dtype in (F16, BF16):
        a = sample(orc, (4096, 8192), dtype)
        d = up(dev, a, dtype)
        assert_bitexact(ops.add(d, d).numpy(), orc.binary(ADD, dtype, a, a), "d + d")
        assert_elementwise(ops.sigmoid(d).numpy(), orc.unary(9, dtype, a), dtype, "sigmoid")


# ---- benchmark config 2 at full size ------------------------------------------------

N = 8192


@pytest.fixture(scope="module", params=[F32, BF16], ids=["fp32", "bf16"])
def config2(request, dev, orc):
    dtype = request.param
    a = sample(orc, (N, N), dtype, 0)
    row = sample(orc, (N,), dtype, 1, 0.5, 2.0)
    col = sample(orc, (N, 1), dtype, 2, 0.5, 2.0)
    g = sample(orc, (N, N), dtype, 3)
    return dtype, a, row, col, g, up(dev, a, dtype), up(dev, row, dtype), up(dev, col, dtype), up(dev, g, dtype)


def test_config2_binary_full_size(ops, orc, config2):
    dtype, a, row, col, g, da, drow, dcol, dg = config2
    for b, db, name in ((row, drow, "row"), (col, dcol, "col")):
        assert_bitexact(ops.add(da, db).numpy(), orc.binary(ADD, dtype, a, b), f"add {name}")
        assert_bitexact(ops.sub(da, db).numpy(), orc.binary(ADD, dtype, a, b, -1.0), f"sub {name}")
        assert_bitexact(ops.mul(da, db).numpy(), orc.binary(MUL, dtype, a, b), f"mul {name}")
        assert_bitexact(ops.div(da, db).numpy(), orc.binary(DIV, dtype, a, b), f"div {name}")
    assert_elementwise(ops.mul_scalar(da, 1.5).numpy(), orc.affine(dtype, a, 1.5, 0.0), dtype,
                       "mul scalar", max_ulp=1)
    work = ops.clone(da)
    ops.add_(work, drow, alpha=0.5)
    assert_elementwise(work.numpy(), orc.binary(ADD, dtype, a, row, 0.5), dtype, "add_ row",
                       max_ulp=1)


def test_config2_unary_full_size(ops, orc, config2):
    dtype, a, row, col, g, da, drow, dcol, dg = config2
    assert_elementwise(ops.exp(da).numpy(), orc.unary(0, dtype, a), dtype, "exp")
    absa = ops.abs(da)
    shifted = ops.add_scalar(absa, 1e-3)
    assert_elementwise(ops.log(shifted).numpy(), orc.unary(1, dtype, shifted.numpy()), dtype,
                       "log(|a|+1e-3)")
    assert_bitexact(ops.sqrt(absa).numpy(), orc.unary(2, dtype, absa.numpy()), "sqrt(|a|)")
    assert_bitexact(ops.pow_scalar(da, 2).numpy(), orc.unary(6, dtype, a), "pow(a, 2)")
    assert_bitexact(ops.relu(da).numpy(), orc.unary(8, dtype, a), "relu")
    assert_elementwise(ops.gelu(da).numpy(), orc.unary(12, dtype, a), dtype, "gelu")
    assert_elementwise(ops.sigmoid(da).numpy(), orc.unary(9, dtype, a), dtype, "sigmoid")


def test_config2_backward_full_size(ops, orc, config2):
    dtype, a, row, col, g, da, drow, dcol, dg = config2
    assert_bitexact(ops.threshold_backward(dg, da, 0).numpy(),
                    orc.activation_backward(0, dtype, g, a, 0.0), "relu backward")
    assert_elementwise(ops.gelu_backward(dg, da).numpy(), orc.activation_backward(3, dtype, g, a),
                       dtype, "gelu backward")
    y = ops.sigmoid(da)
    assert_elementwise(ops.sigmoid_backward(dg, y).numpy(),
                       orc.activation_backward(1, dtype, g, y.numpy()), dtype, "sigmoid backward")
