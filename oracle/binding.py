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
        f64, u64 = C.c_double, C.c_uint64
        L.orc_layer_norm.argtypes = [i32, i64, i64, VP, VP, VP, f64, VP, VP, VP]
        L.orc_layer_norm_backward.argtypes = [i32, i64, i64, VP, VP, VP, VP, VP, VP, VP, VP]
        L.orc_philox4x32_10.argtypes = [VP, VP, VP]
        L.orc_dropout.argtypes = [i32, i64, VP, f64, u64, u64, VP, VP]
        L.orc_dropout_backward.argtypes = [i32, i64, VP, VP, f64, VP]
        L.orc_embedding.argtypes = [i32, i64, i64, VP, i32, i64, VP, VP]
        L.orc_embedding_backward.argtypes = [i32, i64, i64, VP, i32, VP, i64, i64, i32, VP]
        L.orc_nll_loss.argtypes = [i32, i64, i64, VP, i32, VP, VP, i32, i64, VP, VP]
        L.orc_nll_loss_backward.argtypes = [i32, i64, i64, VP, i32, VP, VP, i32, i64, VP, VP]
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


# ---- neural-network layers ----------------------------------------------------

def _opt(a):
    return None if a is None else _p(a)


def _stats_np(dtype: int):
    return np.float64 if dtype == F64 else np.float32


def _index_code(idx: np.ndarray) -> int:
    if idx.dtype == np.int32:
        return I32
    assert idx.dtype == np.int64, idx.dtype
    return I64


def layer_norm(dtype: int, x, D: int, w=None, b=None, eps: float = 1e-5):
    """(y, mean, rstd) over the trailing D elements of each row of x."""
    x = np.ascontiguousarray(x)
    rows = x.size // D
    w = None if w is None else np.ascontiguousarray(w)
    b = None if b is None else np.ascontiguousarray(b)
    y = np.empty_like(x)
    mean = np.empty(rows, _stats_np(dtype))
    rstd = np.empty(rows, _stats_np(dtype))
    lib().orc_layer_norm(dtype, rows, D, _p(x), _opt(w), _opt(b), eps, _p(y), _p(mean), _p(rstd))
    return y, mean, rstd


def layer_norm_backward(dtype: int, dy, x, D: int, mean, rstd, w=None,
                        mask=(True, True, True)):
    """(dx, dw, db), None where ``mask`` says not wanted."""
    dy, x = np.ascontiguousarray(dy), np.ascontiguousarray(x)
    rows = x.size // D
    mean = np.ascontiguousarray(mean, _stats_np(dtype))
    rstd = np.ascontiguousarray(rstd, _stats_np(dtype))
    w = None if w is None else np.ascontiguousarray(w)
    dx = np.empty_like(x) if mask[0] else None
    dw = np.empty(D, x.dtype) if mask[1] else None
    db = np.empty(D, x.dtype) if mask[2] else None
    lib().orc_layer_norm_backward(dtype, rows, D, _p(dy), _p(x), _p(mean), _p(rstd), _opt(w),
                                  _opt(dx), _opt(dw), _opt(db))
    return dx, dw, db


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().orc_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def dropout(dtype: int, x, p: float, seed: int, offset: int = 0):
    """(out, mask) with mask as uint8 0/1."""
    x = np.ascontiguousarray(x)
    out = np.empty_like(x)
    mask = np.empty(x.shape, np.uint8)
    lib().orc_dropout(dtype, x.size, _p(x), p, seed, offset, _p(out), _p(mask))
    return out, mask


def dropout_backward(dtype: int, grad, mask, scale: float):
    g = np.ascontiguousarray(grad)
    m = np.ascontiguousarray(mask, np.uint8)
    out = np.empty_like(g)
    lib().orc_dropout_backward(dtype, g.size, _p(g), _p(m), scale, _p(out))
    return out


def embedding(dtype: int, weight, idx):
    w = np.ascontiguousarray(weight)
    idx = np.ascontiguousarray(idx)
    V, D = w.shape
    out = np.empty(idx.shape + (D,), w.dtype)
    lib().orc_embedding(dtype, V, D, _p(w), _index_code(idx), idx.size, _p(idx), _p(out))
    return out


def embedding_backward(dtype: int, dy, idx, num_weights: int, padding_idx: int = -1,
                       scale_grad_by_freq: bool = False):
    dy = np.ascontiguousarray(dy)
    idx = np.ascontiguousarray(idx)
    D = dy.shape[-1]
    out = np.empty((num_weights, D), dy.dtype)
    lib().orc_embedding_backward(dtype, idx.size, D, _p(dy), _index_code(idx), _p(idx),
                                 num_weights, padding_idx, int(scale_grad_by_freq), _p(out))
    return out


def nll_loss(dtype: int, x, target, w=None, reduction: int = 1, ignore_index: int = -100):
    """(output, total_weight); output has shape (N,) for reduction 0, () otherwise."""
    x = np.ascontiguousarray(x)
    t = np.ascontiguousarray(target)
    w = None if w is None else np.ascontiguousarray(w)
    n, c = x.shape
    y = np.empty((n,) if reduction == 0 else (), x.dtype)
    total = np.empty((), x.dtype)
    lib().orc_nll_loss(dtype, n, c, _p(x), _index_code(t), _p(t), _opt(w), reduction,
                       ignore_index, _p(y), _p(total))
    return y, total


def nll_loss_backward(dtype: int, grad, x_shape, target, total, w=None, reduction: int = 1,
                      ignore_index: int = -100):
    g = np.ascontiguousarray(grad)
    t = np.ascontiguousarray(target)
    tot = np.ascontiguousarray(total)
    w = None if w is None else np.ascontiguousarray(w)
    n, c = x_shape
    dx = np.empty((n, c), g.dtype)
    lib().orc_nll_loss_backward(dtype, n, c, _p(g), _index_code(t), _p(t), _opt(w), reduction,
                                ignore_index, _p(tot), _p(dx))
    return dx
