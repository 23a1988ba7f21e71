"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is compared with expected values that do not come from
its own code (tests/golden/make_golden.py: numpy / scipy float64 routines,
exact rational bfloat16 rounding, finite differences, math.fsum) and with
closed forms and invariants chosen so that a plausible slip -- a dropped
alpha, a wrong sign, a transposed operand, a wrong reduction axis, a
rounding that truncates or ties away -- fails at least one check.
"""

import os

import numpy as np
import pytest

from _check import ulp_distance

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32, F16, BF16, F64, I8, I16, I32, I64, U8, BOOL = range(10)
ADD, MUL, DIV = 0, 1, 2


def fixture(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def within_ulp(got, want, n=1):
    d = ulp_distance(np.ascontiguousarray(got, np.float32), np.ascontiguousarray(want, np.float32), F32)
    assert int(d.max()) <= n, f"{int(d.max())} ulp apart"


# ---- binary arithmetic (orc_binary, orc_affine) ----------------------------------

def test_binary_against_numpy(orc):
    f = fixture("binary")
    a, b = f["a"], f["b"]
    assert np.array_equal(orc.binary(ADD, F32, a, b, 1.0), f["add"])
    assert np.array_equal(orc.binary(ADD, F32, a, b, -2.0), f["sub_alpha2"])
    assert np.array_equal(orc.binary(ADD, F32, a, b, 0.5), f["add_alpha05"])
    assert np.array_equal(orc.binary(MUL, F32, a, b), f["mul"])
    assert np.array_equal(orc.binary(DIV, F32, a, b), f["div"])
    assert np.array_equal(orc.affine(F32, a, 3.0, -1.0), f["affine_3_m1"])
    assert np.array_equal(orc.affine(F32, a, np.float32(1 / 3), 0.0), f["div_scalar_3"])
    # broadcasting the other way round is not the same operation
    assert not np.array_equal(orc.binary(DIV, F32, np.broadcast_to(b, (4, 3, 5)).copy(), a), f["div"])


def test_binary_narrow_dtypes_round_the_float32_result(orc):
    f = fixture("binary")
    a, b = f["a"], f["b"]
    ab, bb = orc.to_bf16(a), orc.to_bf16(b)
    want = orc.to_bf16(orc.binary(MUL, F32, orc.from_bf16(ab), orc.from_bf16(bb)))
    assert np.array_equal(orc.binary(MUL, BF16, ab, bb), want)
    ah, bh = a.astype(np.float16), b.astype(np.float16)
    want = (ah.astype(np.float64) + bh.astype(np.float64)).astype(np.float32).astype(np.float16)
    assert np.array_equal(orc.binary(ADD, F16, ah, bh, 1.0), want)


# ---- rounding (orc_f32_to_bf16 / f16, orc_cast) ----------------------------------

def test_bf16_rounding_matches_exact_rational_rounding(orc):
    f = fixture("bf16_round")
    assert np.array_equal(orc.to_bf16(f["f32"]), f["bf16"])


def test_f16_rounding_matches_numpy(orc):
    f = fixture("bf16_round")
    assert np.array_equal(orc.cast(F32, F16, f["f32"]).view(np.uint16), f["f16"])


def test_widening_every_16_bit_pattern(orc):
    bits = np.arange(1 << 16, dtype=np.uint16)
    h = orc.cast(F16, F32, bits.view(np.float16))
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(h[~nan], want[~nan]) and np.isnan(h[nan]).all()
    bf = orc.from_bf16(bits)
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bf[~nan], want[~nan]) and np.isnan(bf[nan]).all()


def test_bf16_round_is_nearest_with_ties_to_even(orc):
    # Every float32 in [1, 2) whose low 16 bits are 0x8000 lies exactly halfway.
    hi = np.arange(0x3F80, 0x4000, dtype=np.uint32)
    ties = ((hi << 16) | 0x8000).view(np.float32)
    got = orc.to_bf16(ties)
    want = np.where(hi % 2 == 0, hi, hi + 1).astype(np.uint16)
    assert np.array_equal(got, want)
    above = ((hi << 16) | 0x8001).view(np.float32)
    assert np.array_equal(orc.to_bf16(above), (hi + 1).astype(np.uint16))
    below = ((hi << 16) | 0x7FFF).view(np.float32)
    assert np.array_equal(orc.to_bf16(below), hi.astype(np.uint16))


def test_integer_conversions(orc):
    f = fixture("cast")
    assert np.array_equal(orc.cast(F32, I32, f["f32"]), f["to_i32"])
    assert np.array_equal(orc.cast(F32, BOOL, f["f32"]), f["to_bool"])
    assert np.array_equal(orc.cast(I64, F32, f["i64"]), f["i64"].astype(np.float32))
    assert np.array_equal(orc.cast(I32, I8, np.array([127, 128, -129, 300], np.int32)),
                          np.array([127, -128, 127, 44], np.int8))
    assert np.array_equal(orc.cast(F32, U8, np.array([np.nan, 3.7], np.float32)),
                          np.array([0, 3], np.uint8))


# ---- unary and activations (orc_unary) ---------------------------------------------

UNARY = {"exp": 0, "log": 1, "sqrt": 2, "rsqrt": 3, "neg": 4, "abs": 5, "square": 6,
         "pow17": 7, "relu": 8, "sigmoid": 9, "tanh": 10, "silu": 11, "gelu": 12, "gelu_tanh": 13}


@pytest.mark.parametrize("name", sorted(UNARY))
def test_unary_against_numpy_scipy(orc, name):
    f = fixture("unary")
    x = f["pos"] if name in ("log", "sqrt", "rsqrt", "pow17") else f["x"]
    got = orc.unary(UNARY[name], F32, x, 1.7)
    within_ulp(got, f[name], 1)


def test_unary_closed_forms(orc):
    z = np.zeros(4, np.float32)
    assert np.array_equal(orc.unary(9, F32, z), np.full(4, 0.5, np.float32))
    assert np.array_equal(orc.unary(0, F32, z), np.ones(4, np.float32))
    for op in (8, 10, 11, 12, 13):
        assert np.array_equal(orc.unary(op, F32, z), z)
    x = np.array([-3.0, -0.5, 0.5, 3.0], np.float32)
    assert np.array_equal(orc.unary(8, F32, x), np.array([0, 0, 0.5, 3.0], np.float32))
    # gelu(x) - gelu(-x) = x for the erf form
    g = orc.unary(12, F32, x).astype(np.float64)
    assert np.allclose(g - g[::-1], x, rtol=1e-6)


def _round16(v64, dtype, orc):
    """float64 values -> float32 -> the 16-bit dtype (numpy's float16 rounding
    and the oracle's bfloat16 rounding, each pinned above), as storage."""
    with np.errstate(over="ignore", invalid="ignore"):
        v32 = np.asarray(v64, np.float64).astype(np.float32)
        return orc.to_bf16(v32) if dtype == BF16 else v32.astype(np.float16)


@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
def test_transcendentals_at_every_16bit_value(orc, dtype):
    """Every transcendental unary op and activation derivative of the oracle
    at every finite 16-bit value, against numpy / scipy float64 rounded the
    same way (float64 -> float32 -> storage): within one storage ulp, NaN in
    the same places.  These are the points the GPU's every-value tests
    compare against."""
    from scipy import special

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    every = bits if dtype == BF16 else bits.view(np.float16)
    a = every[np.isfinite(orc.to_float(every, dtype))]
    x = orc.to_float(a, dtype)
    c = np.sqrt(2.0 / np.pi)
    with np.errstate(all="ignore"):
        u = c * (x + 0.044715 * x ** 3)
        sig = special.expit(x)
        phi = np.exp(-0.5 * x * x) / np.sqrt(2.0 * np.pi)
        cdf = 0.5 * special.erfc(-x / np.sqrt(2.0))
        forward = {0: np.exp(x), 1: np.log(x), 2: np.sqrt(x), 3: 1.0 / np.sqrt(x), 9: sig, 10: np.tanh(x),
                   11: x * sig, 12: x * cdf, 13: x * special.expit(2.0 * u)}
        sg = special.expit(2.0 * u)
        derivative = {3: cdf + x * phi, 5: sig * (1.0 + x * (1.0 - sig)),
                      4: sg + x * sg * (1.0 - sg) * 2.0 * c * (1.0 + 3.0 * 0.044715 * x * x)}
    one = np.ones(a.shape, np.float32)
    ones16 = orc.from_float(one, dtype)

    def check(got, want64, what):
        want = _round16(want64, dtype, orc)
        gn, wn = np.isnan(orc.to_float(got, dtype)), np.isnan(orc.to_float(want, dtype))
        assert np.array_equal(gn, wn), f"{what}: NaN in other places"
        d = ulp_distance(np.ascontiguousarray(got[~wn]), np.ascontiguousarray(want[~wn]), dtype)
        assert int(d.max()) <= 1, f"{what}: {int(d.max())} ulp apart"

    for op, want in forward.items():
        check(orc.unary(op, dtype, a), want, f"unary {op}")
    for op, want in derivative.items():
        check(orc.activation_backward(op, dtype, ones16, a), want, f"backward {op}")
    # sigmoid / tanh backward take the saved output y
    for op, fwd, f in ((1, 9, lambda y: y * (1.0 - y)), (2, 10, lambda y: 1.0 - y * y)):
        y = orc.unary(fwd, dtype, a)
        check(orc.activation_backward(op, dtype, ones16, y), f(orc.to_float(y, dtype)), f"backward {op}")


# ---- activation backward (orc_activation_backward) ---------------------------------

@pytest.mark.parametrize("name,op,saved", [("sigmoid", 1, "sigmoid_out"), ("tanh", 2, "tanh_out"),
                                           ("gelu", 3, "x"), ("gelu_tanh", 4, "x"), ("silu", 5, "x")])
def test_backward_matches_finite_differences(orc, name, op, saved):
    f = fixture("backward")
    s = f[saved].astype(np.float32)
    got = orc.activation_backward(op, F32, f["g"], s).astype(np.float64)
    want = f[name]
    assert np.all(np.abs(got - want) <= 2e-6 * np.abs(want) + 2e-6), name


def test_threshold_backward(orc):
    g = np.array([1.0, 2.0, 3.0, 4.0, 5.0], np.float32)
    x = np.array([-1.0, 0.0, 0.25, 0.5, 2.0], np.float32)
    assert np.array_equal(orc.activation_backward(0, F32, g, x, 0.0), np.array([0, 0, 3, 4, 5], np.float32))
    assert np.array_equal(orc.activation_backward(0, F32, g, x, 0.25), np.array([0, 0, 0, 4, 5], np.float32))


# ---- reductions (orc_reduce) ---------------------------------------------------------

def test_reduce_against_fsum_and_numpy(orc):
    f = fixture("reduce")
    x = f["x"]
    within_ulp(orc.reduce(0, F32, x, 6, 7, 8).reshape(6, 8), f["sum_dim1"])
    within_ulp(orc.reduce(1, F32, x, 6, 7, 8).reshape(6, 8), f["mean_dim1"])
    assert np.array_equal(orc.reduce(2, F32, x, 6, 7, 8).reshape(6, 8), f["amax_dim1"])
    assert np.array_equal(orc.reduce(3, F32, x, 6, 7, 8).reshape(6, 8), f["amin_dim1"])
    within_ulp(orc.reduce(0, F32, x, 1, x.size, 1), f["sum_all"].reshape(1))


def test_reduce_closed_forms(orc):
    ones = np.ones((3, 4096, 5), np.float32)
    assert np.array_equal(orc.reduce(0, F32, ones, 3, 4096, 5), np.full(15, 4096, np.float32))
    ar = np.arange(1000, dtype=np.float32)
    assert orc.reduce(0, F32, ar, 1, 1000, 1)[0] == 499500.0
    assert orc.reduce(1, F32, ar, 1, 1000, 1)[0] == np.float32(499.5)
    assert orc.reduce(2, F32, ar, 1, 1000, 1)[0] == 999.0
    assert orc.reduce(3, F32, ar[::-1].copy(), 1, 1000, 1)[0] == 0.0


def test_amax_amin_signed_zero_and_nan(orc):
    x = np.array([[0.0, -0.0], [-0.0, 0.0], [-0.0, -0.0], [np.nan, -1.0], [np.nan, np.nan]], np.float32)
    mx = orc.reduce(2, F32, x, 5, 2, 1)
    mn = orc.reduce(3, F32, x, 5, 2, 1)
    assert [np.signbit(v) for v in mx[:3]] == [False, False, True]
    assert [np.signbit(v) for v in mn[:3]] == [True, True, True]
    assert mx[3] == -1.0 and mn[3] == -1.0
    assert np.isnan(mx[4]) and np.isnan(mn[4])


# ---- softmax (orc_softmax, orc_softmax_backward) ---------------------------------------

@pytest.mark.parametrize("dim", [0, 1, 2])
def test_softmax_against_scipy_and_jacobian(orc, dim):
    f = fixture("softmax")
    x, dy = f["x"], f["dy"]
    outer, size, inner = int(np.prod(x.shape[:dim])), x.shape[dim], int(np.prod(x.shape[dim + 1:]))
    y = orc.softmax(False, F32, x, outer, size, inner)
    ly = orc.softmax(True, F32, x, outer, size, inner)
    within_ulp(y, f[f"softmax_{dim}"], 2)
    assert np.allclose(ly, f[f"log_softmax_{dim}"], rtol=1e-6, atol=1e-6)
    dx = orc.softmax_backward(False, F32, f[f"softmax_{dim}"], dy, outer, size, inner)
    assert np.allclose(dx, f[f"softmax_back_{dim}"], rtol=1e-5, atol=1e-6)
    dlx = orc.softmax_backward(True, F32, f[f"log_softmax_{dim}"], dy, outer, size, inner)
    assert np.allclose(dlx, f[f"log_softmax_back_{dim}"], rtol=1e-5, atol=1e-6)


def test_softmax_invariants(orc):
    x = (np.random.default_rng(1).standard_normal((16, 300)) * 20).astype(np.float32)
    y = orc.softmax(False, F32, x, 16, 300, 1).astype(np.float64)
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-5)
    c = np.full((2, 8), 3.5, np.float32)
    assert np.allclose(orc.softmax(False, F32, c, 2, 8, 1), 1 / 8, rtol=1e-7)
    dx = orc.softmax_backward(False, F32, y.astype(np.float32), np.ones_like(x), 16, 300, 1)
    assert np.allclose(dx.astype(np.float64).sum(axis=1), 0.0, atol=1e-5)


# ---- matrix products (orc_gemm, orc_gemm_entries) --------------------------------------

def test_gemm_against_numpy(orc):
    f = fixture("gemm")
    A, B, bias = f["A"], f["B"], f["bias"]
    within_ulp(orc.gemm(F32, A, B), f["mm"])
    within_ulp(orc.gemm(F32, A, B, alpha=2.0, beta=0.5, cin=bias), f["addmm"])
    # transposed storage: op(A) = (A^T)^T
    within_ulp(orc.gemm(F32, np.ascontiguousarray(A.T), B, trans_a=True), f["mm"])
    within_ulp(orc.gemm(F32, A, np.ascontiguousarray(B.T), trans_b=True), f["mm"])
    # (A B)^T = B^T A^T
    within_ulp(orc.gemm(F32, B, A, trans_a=True, trans_b=True), f["mm"].T)


def test_gemm_identities(orc):
    g = np.random.default_rng(3)
    A = g.standard_normal((9, 6)).astype(np.float32)
    assert np.array_equal(orc.gemm(F32, A, np.eye(6, dtype=np.float32)), A)
    P = np.eye(9, dtype=np.float32)[g.permutation(9)]
    assert np.array_equal(orc.gemm(F32, P, A), P @ A)
    Ab = g.standard_normal((3, 4, 5)).astype(np.float32)
    Bb = g.standard_normal((3, 5, 2)).astype(np.float32)
    within_ulp(orc.gemm(F32, Ab, Bb), (Ab.astype(np.float64) @ Bb.astype(np.float64)).astype(np.float32))
    idx = np.array([[1, 2, 1], [0, 3, 0]], np.int64)
    exact = orc.gemm_entries(F32, Ab, Bb, idx)
    ref = Ab.astype(np.float64) @ Bb.astype(np.float64)
    assert np.allclose(exact, [ref[1, 2, 1], ref[0, 3, 0]], rtol=1e-12)
