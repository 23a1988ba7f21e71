"""numpy-facing wrappers over liboracle.so -- TEST INFRASTRUCTURE ONLY.

Arrays are numpy; bfloat16 travels as uint16 bit patterns (dtype code 2).
Every wrapper allocates its result and returns it.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32, F16, BF16, F64, I8, I16, I32, I64, U8, BOOL = range(10)
NP = {F32: np.float32, F16: np.float16, BF16: np.uint16, F64: np.float64, I8: np.int8,
      I16: np.int16, I32: np.int32, I64: np.int64, U8: np.uint8, BOOL: np.bool_}
VP, I64P = C.c_void_p, C.POINTER(C.c_int64)


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.isfile(path):
            subprocess.run(["make", "-C", _HERE], check=True, capture_output=True)
        L = C.CDLL(path)
        i32, i64, f32 = C.c_int, C.c_int64, C.c_float
        L.orc_binary.argtypes = [i32, i32, i32, I64P, VP, I64P, VP, I64P, VP, I64P, f32]
        L.orc_affine.argtypes = [i32, i64, VP, f32, f32, VP]
        L.orc_unary.argtypes = [i32, i32, i64, VP, VP, f32]
        L.orc_activation_backward.argtypes = [i32, i32, i64, VP, VP, VP, f32]
        L.orc_reduce.argtypes = [i32, i32, i64, i64, i64, VP, VP]
        L.orc_softmax.argtypes = [i32, i32, i64, i64, i64, VP, VP]
        L.orc_softmax_backward.argtypes = [i32, i32, i64, i64, i64, VP, VP, VP]
        L.orc_gemm.argtypes = [i32, i64, i64, i64, i64, f32, VP, i64, i64, i32, VP, i64, i64, i32,
                               f32, VP, i64, i64, i64, VP, i64, i64]
        L.orc_gemm_entries.argtypes = [i32, i64, f32, VP, i64, i64, i32, VP, i64, i64, i32, f32,
                                       VP, i64, i64, i64, I64P, i64, VP]
        L.orc_cast.argtypes = [i32, i32, i64, VP, VP]
        L.orc_f32_to_bf16.argtypes = [f32]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_bf16_to_f32.restype = f32
        L.orc_f32_to_f16.argtypes = [f32]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = f32
        L.orc_num_threads.restype = i32
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    return a.ctypes.data_as(VP)


def _i64(seq):
    seq = list(seq)
    return (C.c_int64 * max(len(seq), 1))(*seq)


def _elem_strides(a: np.ndarray):
    return [s // a.itemsize for s in a.strides]


# ---- conversions --------------------------------------------------------------

def to_bf16(x) -> np.ndarray:
    """float32 values -> bfloat16 bit patterns (round to nearest even)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_cast(F32, BF16, x.size, _p(x), _p(out))
    return out


def from_bf16(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_cast(BF16, F32, bits.size, _p(bits), _p(out))
    return out


def to_float(x: np.ndarray, dtype: int) -> np.ndarray:
    """Storage array of ``dtype`` -> float64 values."""
    if dtype == BF16:
        return from_bf16(x).astype(np.float64)
    return np.asarray(x).astype(np.float64)


def from_float(x, dtype: int) -> np.ndarray:
    """float values -> storage of ``dtype`` (through float32 for the narrow
    floats, as the reference's compute type)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == BF16:
        return to_bf16(x)
    return x.astype(NP[dtype])


# ---- operators ----------------------------------------------------------------

def binary(op: int, dtype: int, a: np.ndarray, b: np.ndarray, alpha: float = 1.0,
           out: np.ndarray | None = None) -> np.ndarray:
    """op 0 add (a + alpha b), 1 mul, 2 div, with numpy-style broadcasting."""
    shape = np.broadcast_shapes(a.shape, b.shape)
    ae, be = np.broadcast_to(a, shape), np.broadcast_to(b, shape)
    if out is None:
        out = np.empty(shape, NP[dtype])
    lib().orc_binary(op, dtype, len(shape), _i64(shape), _p(ae), _i64(_elem_strides(ae)),
                     _p(be), _i64(_elem_strides(be)), _p(out), _i64(_elem_strides(out)), alpha)
    return out


def affine(dtype, x, alpha, beta):
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    lib().orc_affine(dtype, x.size, _p(x), alpha, beta, _p(y))
    return y


def unary(op: int, dtype: int, x: np.ndarray, param: float = 0.0) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    lib().orc_unary(op, dtype, x.size, _p(x), _p(y), param)
    return y


def activation_backward(op: int, dtype: int, grad, saved, param: float = 0.0):
    g, s = np.ascontiguousarray(grad), np.ascontiguousarray(saved)
    dx = np.empty_like(g)
    lib().orc_activation_backward(op, dtype, g.size, _p(g), _p(s), _p(dx), param)
    return dx


def reduce(op: int, dtype: int, x: np.ndarray, outer: int, r: int, inner: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    out = np.empty(outer * inner, NP[dtype])
    lib().orc_reduce(op, dtype, outer, r, inner, _p(x), _p(out))
    return out


def softmax(log: bool, dtype: int, x: np.ndarray, outer: int, dim: int, inner: int):
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    lib().orc_softmax(int(log), dtype, outer, dim, inner, _p(x), _p(y))
    return y


def softmax_backward(log: bool, dtype: int, y, dy, outer: int, dim: int, inner: int):
    y, dy = np.ascontiguousarray(y), np.ascontiguousarray(dy)
    dx = np.empty_like(dy)
    lib().orc_softmax_backward(int(log), dtype, outer, dim, inner, _p(y), _p(dy), _p(dx))
    return dx


def gemm(dtype, a, b, trans_a=False, trans_b=False, alpha=1.0, beta=0.0, cin=None):
    """C = alpha op(A) op(B) + beta cin for 2-d or batched 3-d operands given
    as stored (op = transpose of the stored matrix when trans_*)."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    batched = a.ndim == 3
    A = a if batched else a[None]
    B = b if batched else b[None]
    batch = max(A.shape[0], B.shape[0])
    m = A.shape[2] if trans_a else A.shape[1]
    k = A.shape[1] if trans_a else A.shape[2]
    n = B.shape[1] if trans_b else B.shape[2]
    c = np.empty((batch, m, n), NP[dtype])
    sa = 0 if A.shape[0] == 1 else A.shape[1] * A.shape[2]
    sb = 0 if B.shape[0] == 1 else B.shape[1] * B.shape[2]
    if cin is not None:
        ce = np.broadcast_to(cin, (batch, m, n)) if batched else np.broadcast_to(cin, (m, n))[None]
        cs = _elem_strides(ce)
        cptr, rs, cst, sbc = _p(ce), cs[1], cs[2], cs[0]
    else:
        cptr, rs, cst, sbc = None, 0, 0, 0
    lib().orc_gemm(dtype, batch, m, n, k, alpha, _p(A), A.shape[2], sa, int(trans_a), _p(B),
                   B.shape[2], sb, int(trans_b), beta, cptr, rs, cst, sbc, _p(c), n, m * n)
    return c if batched else c[0]


def gemm_entries(dtype, a, b, idx, trans_a=False, trans_b=False, alpha=1.0, beta=0.0,
                 cin=None) -> np.ndarray:
    """Exact float64 values of C at ``idx`` (rows of (batch, i, j))."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    batched = a.ndim == 3
    A = a if batched else a[None]
    B = b if batched else b[None]
    k = A.shape[1] if trans_a else A.shape[2]
    sa = 0 if A.shape[0] == 1 else A.shape[1] * A.shape[2]
    sb = 0 if B.shape[0] == 1 else B.shape[1] * B.shape[2]
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(len(idx), np.float64)
    if cin is not None:
        m = A.shape[2] if trans_a else A.shape[1]
        n = B.shape[1] if trans_b else B.shape[2]
        batch = max(A.shape[0], B.shape[0])
        ce = np.broadcast_to(cin, (batch, m, n)) if batched else np.broadcast_to(cin, (m, n))[None]
        cs = _elem_strides(ce)
        cptr, rs, cst, sbc = _p(ce), cs[1], cs[2], cs[0]
    else:
        cptr, rs, cst, sbc = None, 0, 0, 0
    lib().orc_gemm_entries(dtype, k, alpha, _p(A), A.shape[2], sa, int(trans_a), _p(B),
                           B.shape[2], sb, int(trans_b), beta, cptr, rs, cst, sbc,
                           idx.ctypes.data_as(I64P), len(idx), _p(out))
    return out


def cast(src_dtype: int, dst_dtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    out = np.empty(x.shape, NP[dst_dtype])
    lib().orc_cast(src_dtype, dst_dtype, x.size, _p(x), _p(out))
    return out
