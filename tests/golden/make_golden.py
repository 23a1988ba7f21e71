"""Writes the golden fixtures that pin the CPU oracle (tests/golden/*.npz).

The reference repository holds no golden vectors or fixtures for this path
(its tests compare live against TensorPlay's host kernels,
tests/test_mlu.py:21-34), and neither TensorPlay nor CNNL is available here.
So every expected value below comes from an implementation independent of
the oracle's C code:
  * numpy / scipy.special float64 routines (arithmetic with broadcasting,
    exp, log, erfc, expit, tanh, softmax, log_softmax, matmul), rounded to
    float32 with numpy's round-to-nearest-even cast;
  * bfloat16 rounding decided exactly with fractions.Fraction (nearest
    representable value, ties to the even significand);
  * backward kernels from central finite differences of the float64
    forward functions;
  * sums with math.fsum (exactly rounded).

  python tests/golden/make_golden.py      # rewrites the .npz files
"""

from __future__ import annotations

import math
import os
from fractions import Fraction

import numpy as np
from scipy import special

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_exact(x: float) -> int:
    """bfloat16 bit pattern nearest to float32 value x (ties to even),
    decided with exact rational arithmetic."""
    f = np.float32(x)
    bits = int(np.array(f).view(np.uint32))
    if math.isnan(f):
        return (bits >> 16) | 0x40
    sign = bits & 0x80000000
    if math.isinf(f):
        return (sign >> 16) | 0x7F80
    v = Fraction(abs(float(f)))
    # candidates: every bf16 magnitude pattern below and above
    lo_bits = (bits & 0x7FFFFFFF) >> 16
    best = None
    for cand in (lo_bits, lo_bits + 1):
        cf = np.array([cand << 16], np.uint32).view(np.float32)[0]
        # the pattern after the largest finite value stands for 2^128: round
        # as if the exponent were unbounded, then overflow to infinity
        cv = Fraction(2) ** 128 if math.isinf(cf) else Fraction(float(cf))
        d = abs(cv - v)
        if best is None or d < best[1] or (d == best[1] and cand % 2 == 0):
            best = (cand, d)
    return (sign >> 16) | best[0]


def central_difference(f, x, h=1e-5):
    return (f(x + h) - f(x - h)) / (2 * h)


def main() -> None:
    g = np.random.default_rng(2024)

    # ---- binary arithmetic with broadcasting -----------------------------
    a = g.standard_normal((4, 1, 5)).astype(np.float32)
    b = g.uniform(0.5, 2.0, (3, 1)).astype(np.float32)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    np.savez(os.path.join(HERE, "binary.npz"), a=a, b=b,
             add=(a64 + b64).astype(np.float32),
             sub_alpha2=(a64 - np.float64(np.float32(2.0)) * b64).astype(np.float32),
             add_alpha05=(a64 + 0.5 * b64).astype(np.float32),
             mul=(a64 * b64).astype(np.float32),
             div=(a64 / b64).astype(np.float32),
             affine_3_m1=(3.0 * a64 - 1.0).astype(np.float32),
             # division by a scalar multiplies by the float32 reciprocal
             div_scalar_3=(np.float64(np.float32(1 / 3)) * a64).astype(np.float32))

    # ---- bfloat16 rounding ------------------------------------------------
    special_vals = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.005859375, 1.0078125,
                             1.001953125, 1.0029296875, 3.4028235e38, 3.3961776e38, 1e-40,
                             -1e-40, 1.1754944e-38, 9.18355e-41, np.inf, -np.inf, 65504.0,
                             0.1, 2.5, 7.0, -123.456], np.float32)
    rand = (g.standard_normal(4000) * 10.0 ** g.integers(-30, 30, 4000)).astype(np.float32)
    vals = np.concatenate([special_vals, rand]).astype(np.float32)
    bf = np.array([bf16_exact(float(v)) for v in vals], np.uint16)
    np.savez(os.path.join(HERE, "bf16_round.npz"), f32=vals, bf16=bf,
             f16=np.where(np.abs(vals) > 65520.0, np.copysign(np.inf, vals),
                          vals).astype(np.float16).view(np.uint16))

    # ---- unary math and activations ---------------------------------------
    x = np.concatenate([g.standard_normal(512) * 2.5, [0.0, -0.0, 1e-3, -1e-3, 8.0, -8.0]])
    x = x.astype(np.float32)
    x64 = x.astype(np.float64)
    pos = (np.abs(x64) + 0.1).astype(np.float32).astype(np.float64)
    k = math.sqrt(2 / math.pi)
    # 0.5 t (1 + tanh u) evaluated as t * expit(2u) (the same function; scipy's
    # expit keeps relative accuracy where 1 + tanh(u) cancels)
    gelu_tanh = lambda t: t * special.expit(2 * k * (t + 0.044715 * t ** 3))  # noqa: E731
    gelu = lambda t: 0.5 * t * special.erfc(-t / math.sqrt(2))  # noqa: E731
    silu = lambda t: t * special.expit(t)  # noqa: E731
    unary = {
        "exp": np.exp(x64), "log": np.log(pos), "sqrt": np.sqrt(pos), "rsqrt": 1 / np.sqrt(pos),
        "neg": -x64, "abs": np.abs(x64), "square": x64 * x64, "pow17": np.power(pos, np.float64(np.float32(1.7))),
        "relu": np.maximum(x64, 0.0), "sigmoid": special.expit(x64), "tanh": np.tanh(x64),
        "silu": silu(x64), "gelu": gelu(x64), "gelu_tanh": gelu_tanh(x64),
    }
    np.savez(os.path.join(HERE, "unary.npz"), x=x, pos=pos.astype(np.float32),
             **{n: v.astype(np.float32) for n, v in unary.items()})

    # ---- activation backward: finite differences of the forward ------------
    xs = (g.standard_normal(256) * 2).astype(np.float32).astype(np.float64)
    gr = g.standard_normal(256).astype(np.float32).astype(np.float64)
    sig, th = special.expit(xs), np.tanh(xs)
    back = {
        "sigmoid": gr * central_difference(special.expit, xs),
        "tanh": gr * central_difference(np.tanh, xs),
        "gelu": gr * central_difference(gelu, xs),
        "gelu_tanh": gr * central_difference(gelu_tanh, xs),
        "silu": gr * central_difference(silu, xs),
    }
    np.savez(os.path.join(HERE, "backward.npz"), x=xs.astype(np.float32), g=gr.astype(np.float32),
             sigmoid_out=sig, tanh_out=th, **back)

    # ---- reductions -------------------------------------------------------------
    r = g.standard_normal((6, 7, 8)).astype(np.float32)
    r64 = r.astype(np.float64)
    sum_dim1 = np.array([[math.fsum(r64[i, :, j]) for j in range(8)] for i in range(6)])
    np.savez(os.path.join(HERE, "reduce.npz"), x=r,
             sum_dim1=sum_dim1.astype(np.float32),
             mean_dim1=(sum_dim1 / 7).astype(np.float32),
             amax_dim1=r.max(axis=1), amin_dim1=r.min(axis=1),
             sum_all=np.float32(math.fsum(r64.ravel())))

    # ---- softmax ---------------------------------------------------------------------
    s = (g.standard_normal((5, 6, 7)) * 3).astype(np.float32)
    s64 = s.astype(np.float64)
    dy = g.standard_normal((5, 6, 7)).astype(np.float32).astype(np.float64)
    out = {}
    for dim in (0, 1, 2):
        y = special.softmax(s64, axis=dim)
        ly = special.log_softmax(s64, axis=dim)
        out[f"softmax_{dim}"] = y
        out[f"log_softmax_{dim}"] = ly
        # backward from the explicit Jacobian J = diag(y) - y y^T along dim
        ym = np.moveaxis(y, dim, -1)
        gm = np.moveaxis(dy, dim, -1)
        jac = np.einsum("...i,ij->...ij", ym, np.eye(ym.shape[-1])) - ym[..., :, None] * ym[..., None, :]
        out[f"softmax_back_{dim}"] = np.moveaxis(np.einsum("...ij,...j->...i", jac, gm), -1, dim)
        # log_softmax: J = I - 1 softmax^T  =>  dx = dy - softmax * sum(dy)
        jl = np.eye(ym.shape[-1]) - ym[..., None, :]
        out[f"log_softmax_back_{dim}"] = np.moveaxis(np.einsum("...ji,...j->...i", jl, gm), -1, dim)
    np.savez(os.path.join(HERE, "softmax.npz"), x=s, dy=dy.astype(np.float32),
             **{k2: v.astype(np.float32) for k2, v in out.items()})

    # ---- matrix products ---------------------------------------------------------------
    A = g.standard_normal((7, 5)).astype(np.float32)
    B = g.standard_normal((5, 3)).astype(np.float32)
    bias = g.standard_normal(3).astype(np.float32)
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    np.savez(os.path.join(HERE, "gemm.npz"), A=A, B=B, bias=bias,
             mm=(A64 @ B64).astype(np.float32),
             addmm=(0.5 * bias.astype(np.float64) + 2.0 * (A64 @ B64)).astype(np.float32))

    # ---- integer conversions -------------------------------------------------------------
    f = np.array([0.0, -0.0, 0.5, -0.5, 1.9, -1.9, 126.7, -128.9, 1e6, -3.99, 2.0 ** 31 - 256,
                  7.0], np.float32)
    np.savez(os.path.join(HERE, "cast.npz"), f32=f, to_i32=np.trunc(f).astype(np.int64).astype(np.int32),
             to_bool=(f != 0), i64=np.array([0, 1, -1, 2 ** 24 + 1, -(2 ** 40), 123456789], np.int64))
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
