"""The hot-path operators under the names TensorPlay registers them with
(the reference's 64 ``m.impl`` registrations: CopyKernels.cpp:349-364,
BinaryKernels.cpp:252-269, UnaryKernels.cpp:291-310, BlasKernels.cpp:416-422,
ReduceKernels.cpp:267-282), each one call into libtp_amd.so's operator
C-ABI.  A declined call raises ``DeclinedError`` -- TensorPlay's adapter would
run the host kernel instead; this mirror has no host path.

Operands are ``DeviceTensor``s; a Python number or a 0-d host numpy array
stands for a host 0-d tensor where the reference accepts one.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi
from . import _library
from .tensor import DeviceTensor, check, dtype_code, host_view

_keep = []  # host buffers referenced by views during one call


def _ref(x):
    """tp_amd_tensor pointer for a DeviceTensor, a host 0-d value or None."""
    if x is None:
        return None
    if isinstance(x, DeviceTensor):
        return C.byref(x.ref)
    if isinstance(x, (int, float, bool, np.generic, np.ndarray)):
        arr = np.asarray(x)
        if arr.dtype == np.float64 and not isinstance(x, np.ndarray):
            arr = arr.astype(np.float32)  # a Python float is a float32 host scalar
        if arr.dtype == np.int64 and isinstance(x, bool):
            arr = arr.astype(np.bool_)
        arr = np.asarray(arr, order="C")
        _keep.append(arr)
        return C.byref(host_view(arr))
    raise TypeError(f"unsupported operand {type(x)}")


def _call_result(fn, *args, base=None) -> DeviceTensor:
    out = _abi.Tensor()
    try:
        check(fn(*args, C.byref(out)))
    finally:
        _keep.clear()
    return DeviceTensor.from_result(out, base)


def _call(fn, *args) -> None:
    try:
        check(fn(*args))
    finally:
        _keep.clear()


def _dtype(dtype) -> int:
    return _abi.UNDEFINED if dtype is None else dtype_code(dtype)


def _dims(dims):
    if dims is None:
        return None, 0
    if isinstance(dims, int):
        dims = [dims]
    arr = (C.c_int64 * max(len(dims), 1))(*dims)
    return arr, len(dims)


L = _library

# ---- factories, copies, casts, fills -------------------------------------------


def empty(shape, dtype=None, device: int = 0) -> DeviceTensor:
    shape = tuple(shape)
    sizes = (C.c_int64 * max(len(shape), 1))(*shape)
    return _call_result(L().tp_amd_empty, sizes, len(shape), _dtype(dtype), device, 0)


def empty_like(self, dtype=None, device: int = -1):
    return _call_result(L().tp_amd_empty_like, _ref(self), _dtype(dtype), device)


def zeros_like(self, dtype=None, device: int = -1):
    return _call_result(L().tp_amd_zeros_like, _ref(self), _dtype(dtype), device)


def ones_like(self, dtype=None, device: int = -1):
    return _call_result(L().tp_amd_ones_like, _ref(self), _dtype(dtype), device)


def full_like(self, value, dtype=None, device: int = -1):
    return _call_result(L().tp_amd_full_like, _ref(self), _abi.scalar(value), _dtype(dtype), device)


def item(self):
    s = _abi.Scalar()
    _call(L().tp_amd_item, _ref(self), C.byref(s))
    if s.kind == _abi.SCALAR_FLOAT:
        return s.f
    if s.kind == _abi.SCALAR_BOOL:
        return bool(s.i)
    return int(s.i)


_local_scalar_dense = item


def copy_(self: DeviceTensor, src, non_blocking: bool = False) -> DeviceTensor:
    if isinstance(src, np.ndarray) and src.ndim > 0:
        arr = src
        if not arr.flags.c_contiguous and not arr.flags.f_contiguous:
            arr = np.array(arr)
        _keep.append(arr)
        src_ref = C.byref(host_view(arr))
    else:
        src_ref = _ref(src)
    _call(L().tp_amd_copy_, _ref(self), src_ref, int(non_blocking))
    return self


def fill_(self: DeviceTensor, value) -> DeviceTensor:
    _call(L().tp_amd_fill_, _ref(self), _abi.scalar(value))
    return self


def zero_(self: DeviceTensor) -> DeviceTensor:
    _call(L().tp_amd_zero_, _ref(self))
    return self


def clone(self):
    return _call_result(L().tp_amd_clone, _ref(self))


def contiguous(self):
    return _call_result(L().tp_amd_contiguous, _ref(self), base=self)


def to(self, dtype):
    return _call_result(L().tp_amd_to_dtype, _ref(self), dtype_code(dtype))


# ---- binary arithmetic ---------------------------------------------------------


def add(self, other, alpha=1):
    return _call_result(L().tp_amd_add, _ref(self), _ref(other), _abi.scalar(alpha))


def sub(self, other, alpha=1):
    return _call_result(L().tp_amd_sub, _ref(self), _ref(other), _abi.scalar(alpha))


def mul(self, other):
    return _call_result(L().tp_amd_mul, _ref(self), _ref(other))


def div(self, other):
    return _call_result(L().tp_amd_div, _ref(self), _ref(other))


def add_(self, other, alpha=1):
    _call(L().tp_amd_add_, _ref(self), _ref(other), _abi.scalar(alpha))
    return self


def sub_(self, other, alpha=1):
    _call(L().tp_amd_sub_, _ref(self), _ref(other), _abi.scalar(alpha))
    return self


def mul_(self, other):
    _call(L().tp_amd_mul_, _ref(self), _ref(other))
    return self


def div_(self, other):
    _call(L().tp_amd_div_, _ref(self), _ref(other))
    return self


def add_scalar(self, other, alpha=1):
    return _call_result(L().tp_amd_add_scalar, _ref(self), _abi.scalar(other), _abi.scalar(alpha))


def sub_scalar(self, other, alpha=1):
    return _call_result(L().tp_amd_sub_scalar, _ref(self), _abi.scalar(other), _abi.scalar(alpha))


def rsub_scalar(self, other, alpha=1):
    return _call_result(L().tp_amd_rsub_scalar, _ref(self), _abi.scalar(other), _abi.scalar(alpha))


def mul_scalar(self, other):
    return _call_result(L().tp_amd_mul_scalar, _ref(self), _abi.scalar(other))


def div_scalar(self, other):
    return _call_result(L().tp_amd_div_scalar, _ref(self), _abi.scalar(other))


def add__scalar(self, other, alpha=1):
    _call(L().tp_amd_add__scalar, _ref(self), _abi.scalar(other), _abi.scalar(alpha))
    return self


def mul__scalar(self, other):
    _call(L().tp_amd_mul__scalar, _ref(self), _abi.scalar(other))
    return self


def div__scalar(self, other):
    _call(L().tp_amd_div__scalar, _ref(self), _abi.scalar(other))
    return self


# ---- unary and activations --------------------------------------------------------


def _unary(name):
    def op(self):
        return _call_result(getattr(L(), "tp_amd_" + name), _ref(self))
    op.__name__ = name
    return op


exp = _unary("exp")
log = _unary("log")
sqrt = _unary("sqrt")
rsqrt = _unary("rsqrt")
neg = _unary("neg")
abs = _unary("abs")  # noqa: A001 - the operator's name
relu = _unary("relu")
sigmoid = _unary("sigmoid")
tanh = _unary("tanh")
silu = _unary("silu")


def pow_scalar(self, exponent):
    return _call_result(L().tp_amd_pow_scalar, _ref(self), _abi.scalar(exponent))


def relu_(self):
    _call(L().tp_amd_relu_, _ref(self))
    return self


def gelu(self, approximate: str = "none"):
    return _call_result(L().tp_amd_gelu, _ref(self), int(approximate == "tanh"))


def threshold_backward(grad_output, self, threshold):
    return _call_result(L().tp_amd_threshold_backward, _ref(grad_output), _ref(self),
                        _abi.scalar(threshold))


def sigmoid_backward(grad_output, output):
    return _call_result(L().tp_amd_sigmoid_backward, _ref(grad_output), _ref(output))


def tanh_backward(grad_output, output):
    return _call_result(L().tp_amd_tanh_backward, _ref(grad_output), _ref(output))


def gelu_backward(grad_output, self, approximate: str = "none"):
    return _call_result(L().tp_amd_gelu_backward, _ref(grad_output), _ref(self),
                        int(approximate == "tanh"))


def silu_backward(grad_output, self):
    return _call_result(L().tp_amd_silu_backward, _ref(grad_output), _ref(self))


# ---- matrix products -----------------------------------------------------------------


def mm(self, mat2):
    return _call_result(L().tp_amd_mm, _ref(self), _ref(mat2))


def bmm(self, mat2):
    return _call_result(L().tp_amd_bmm, _ref(self), _ref(mat2))


def addmm(self, mat1, mat2, beta=1, alpha=1):
    return _call_result(L().tp_amd_addmm, _ref(self), _ref(mat1), _ref(mat2),
                        _abi.scalar(beta), _abi.scalar(alpha))


def linear(input, weight, bias=None):  # noqa: A002 - the operator's argument name
    return _call_result(L().tp_amd_linear, _ref(input), _ref(weight), _ref(bias))


def matmul(self, other):
    return _call_result(L().tp_amd_matmul, _ref(self), _ref(other))


# ---- reductions and softmax ------------------------------------------------------------


def sum(self, dtype=None):  # noqa: A001 - the operator's name
    return _call_result(L().tp_amd_sum, _ref(self), _dtype(dtype))


def mean(self, dtype=None):
    return _call_result(L().tp_amd_mean, _ref(self), _dtype(dtype))


def sum_dim(self, dim, keepdim=False, dtype=None):
    d, n = _dims(dim)
    return _call_result(L().tp_amd_sum_dim, _ref(self), d, n, int(keepdim), _dtype(dtype))


def mean_dim(self, dim, keepdim=False, dtype=None):
    d, n = _dims(dim)
    return _call_result(L().tp_amd_mean_dim, _ref(self), d, n, int(keepdim), _dtype(dtype))


def amax(self, dim=(), keepdim=False):
    d, n = _dims(dim)
    return _call_result(L().tp_amd_amax, _ref(self), d, n, int(keepdim))


def amin(self, dim=(), keepdim=False):
    d, n = _dims(dim)
    return _call_result(L().tp_amd_amin, _ref(self), d, n, int(keepdim))


def softmax(self, dim, dtype=None):
    return _call_result(L().tp_amd_softmax, _ref(self), dim, _dtype(dtype))


def log_softmax(self, dim, dtype=None):
    return _call_result(L().tp_amd_log_softmax, _ref(self), dim, _dtype(dtype))


def _softmax(self, dim, half_to_float=False):
    return _call_result(L().tp_amd__softmax, _ref(self), dim, int(half_to_float))


def _log_softmax(self, dim, half_to_float=False):
    return _call_result(L().tp_amd__log_softmax, _ref(self), dim, int(half_to_float))


def _softmax_backward_data(grad_output, output, dim, input_dtype):
    return _call_result(L().tp_amd__softmax_backward_data, _ref(grad_output), _ref(output), dim,
                        dtype_code(input_dtype))


def _log_softmax_backward_data(grad_output, output, dim, input_dtype):
    return _call_result(L().tp_amd__log_softmax_backward_data, _ref(grad_output), _ref(output),
                        dim, dtype_code(input_dtype))


# ---- neural-network layers (NNKernels.cpp:57-395) -------------------------------


def _call_results(fn, *args, count):
    """An entry with ``count`` result slots; a slot the call leaves undefined
    (an output masked off) comes back as None."""
    outs = [_abi.Tensor() for _ in range(count)]
    try:
        check(fn(*args, *[C.byref(o) for o in outs]))
    finally:
        _keep.clear()
    return tuple(None if (not o.data and o.dtype == _abi.UNDEFINED) else DeviceTensor.from_result(o)
                 for o in outs)


def native_layer_norm(input, normalized_shape, weight=None, bias=None, eps=1e-5):
    """(y, mean, rstd); mean and rstd are float32 of shape [outer]."""
    shape, n = _dims(list(normalized_shape))
    return _call_results(L().tp_amd_native_layer_norm, _ref(input), shape, n, _ref(weight),
                         _ref(bias), float(eps), count=3)


def native_layer_norm_backward(grad_out, input, normalized_shape, mean, rstd, weight=None,
                               bias=None, output_mask=(True, True, True)):
    """(dx, dweight, dbias), None where output_mask is False."""
    shape, n = _dims(list(normalized_shape))
    mask = (C.c_int * 3)(*[int(bool(m)) for m in output_mask])
    return _call_results(L().tp_amd_native_layer_norm_backward, _ref(grad_out), _ref(input), shape,
                         n, _ref(mean), _ref(rstd), _ref(weight), _ref(bias), mask, count=3)


def native_dropout(input, p, train=None, seed=0):
    """(out, mask); ``train`` None counts as training.  The stream of random
    numbers is keyed by ``seed``."""
    t = -1 if train is None else int(bool(train))
    return _call_results(L().tp_amd_native_dropout, _ref(input), float(p), t,
                         int(seed) & 0xFFFFFFFFFFFFFFFF, count=2)


def native_dropout_backward(grad_output, mask, scale):
    return _call_result(L().tp_amd_native_dropout_backward, _ref(grad_output), _ref(mask),
                        float(scale))


def embedding(weight, indices, padding_idx=-1, scale_grad_by_freq=False, sparse=False):
    return _call_result(L().tp_amd_embedding, _ref(weight), _ref(indices), int(padding_idx),
                        int(bool(scale_grad_by_freq)), int(bool(sparse)))


def embedding_dense_backward(grad_output, indices, num_weights, padding_idx=-1,
                             scale_grad_by_freq=False):
    return _call_result(L().tp_amd_embedding_dense_backward, _ref(grad_output), _ref(indices),
                        int(num_weights), int(padding_idx), int(bool(scale_grad_by_freq)))


def nll_loss(self, target, weight=None, reduction=1, ignore_index=-100):
    """(output, total_weight); reduction 0 none, 1 mean, 2 sum."""
    return _call_results(L().tp_amd_nll_loss, _ref(self), _ref(target), _ref(weight),
                         int(reduction), int(ignore_index), count=2)


def nll_loss_backward(grad_output, self, target, weight, reduction, ignore_index, total_weight):
    return _call_result(L().tp_amd_nll_loss_backward, _ref(grad_output), _ref(self), _ref(target),
                        _ref(weight), int(reduction), int(ignore_index), _ref(total_weight))


#: The 72 operator names of the reference's registrations (64 on the hot
#: path, 8 neural-network layers) and the function here that serves each.
REGISTRATIONS = {
    "empty_like": empty_like, "zeros_like": zeros_like, "ones_like": ones_like,
    "full_like": full_like, "item": item, "_local_scalar_dense": _local_scalar_dense,
    "empty": empty, "empty.memory_format": empty, "copy_": copy_, "fill_.Scalar": fill_,
    "zero_": zero_, "clone": clone, "contiguous": contiguous,
    "add.Tensor": add, "sub.Tensor": sub, "mul.Tensor": mul, "div.Tensor": div,
    "add_.Tensor": add_, "sub_.Tensor": sub_, "mul_.Tensor": mul_, "div_.Tensor": div_,
    "add.Scalar": add_scalar, "sub.Scalar": sub_scalar, "rsub.Scalar": rsub_scalar,
    "mul.Scalar": mul_scalar, "div.Scalar": div_scalar, "add_.Scalar": add__scalar,
    "mul_.Scalar": mul__scalar, "div_.Scalar": div__scalar,
    "exp": exp, "log": log, "sqrt": sqrt, "rsqrt": rsqrt, "neg": neg, "abs": abs,
    "pow.Tensor_Scalar": pow_scalar, "relu": relu, "relu_": relu_, "sigmoid": sigmoid,
    "tanh": tanh, "silu": silu, "gelu": gelu, "threshold_backward": threshold_backward,
    "sigmoid_backward": sigmoid_backward, "tanh_backward": tanh_backward,
    "gelu_backward": gelu_backward, "silu_backward": silu_backward,
    "mm": mm, "bmm": bmm, "addmm": addmm, "matmul": matmul, "linear": linear,
    "sum": sum, "sum.dim_IntList": sum_dim, "amax": amax, "amin": amin, "mean": mean,
    "mean.dim": mean_dim, "softmax": softmax, "log_softmax": log_softmax,
    "_softmax": _softmax, "_log_softmax": _log_softmax,
    "_softmax_backward_data": _softmax_backward_data,
    "_log_softmax_backward_data": _log_softmax_backward_data,
    "native_layer_norm": native_layer_norm,
    "native_layer_norm_backward": native_layer_norm_backward,
    "native_dropout": native_dropout, "native_dropout_backward": native_dropout_backward,
    "embedding": embedding, "embedding_dense_backward": embedding_dense_backward,
    "nll_loss": nll_loss, "nll_loss_backward": nll_loss_backward,
}
