"""ctypes declarations for every entry point of libtp_amd.so.

The prototypes mirror ``include/tp_amd_types.h``, ``tp_amd_runtime.h``,
``tp_amd_kernels.h`` and ``tp_amd_ops.h``; ``bind`` attaches them to a loaded
library so every call is type-checked by ctypes.
"""

from __future__ import annotations

import ctypes as C

MAX_DIMS = 8

OK, DECLINED, ERROR = 0, 1, -1

# dtype codes (tp_amd_dtype)
FLOAT32, FLOAT16, BFLOAT16, FLOAT64 = 0, 1, 2, 3
INT8, INT16, INT32, INT64, UINT8, BOOL = 4, 5, 6, 7, 8, 9
UNDEFINED = -1

SCALAR_FLOAT, SCALAR_INT, SCALAR_BOOL = 0, 1, 2


class Tensor(C.Structure):
    """tp_amd_tensor: a strided view (data, owning block, sizes, strides)."""

    _fields_ = [
        ("data", C.c_void_p),
        ("ctx", C.c_void_p),
        ("sizes", C.c_int64 * MAX_DIMS),
        ("strides", C.c_int64 * MAX_DIMS),
        ("ndim", C.c_int32),
        ("dtype", C.c_int32),
        ("device", C.c_int32),
        ("reserved", C.c_int32),
    ]


class Scalar(C.Structure):
    """tp_amd_scalar: TensorPlay's Scalar (float, int or bool)."""

    _fields_ = [
        ("f", C.c_double),
        ("i", C.c_int64),
        ("kind", C.c_int32),
        ("reserved", C.c_int32),
    ]


def scalar(value) -> Scalar:
    if isinstance(value, bool):
        return Scalar(float(value), int(value), SCALAR_BOOL, 0)
    if isinstance(value, int):
        return Scalar(float(value), value, SCALAR_INT, 0)
    return Scalar(float(value), int(value) if abs(float(value)) < 2 ** 63 else 0, SCALAR_FLOAT, 0)


COPY_OTHER, COPY_HTOD, COPY_DTOH, COPY_DTOD = 0, 1, 2, 3
NO_EXTERNAL = 2 ** 64 - 1


class Activity(C.Structure):
    """tp_amd_activity: one kernel or copy of a tracing session."""

    _fields_ = [
        ("name", C.c_char_p),
        ("kind", C.c_char),
        ("copy_kind", C.c_uint8),
        ("start_ns", C.c_uint64),
        ("end_ns", C.c_uint64),
        ("external_id", C.c_uint64),
        ("correlation", C.c_uint32),
        ("device", C.c_int32),
        ("stream", C.c_int32),
        ("bytes", C.c_uint64),
    ]


T = C.POINTER(Tensor)
I64P = C.POINTER(C.c_int64)
VP = C.c_void_p
i32, i64, f32, f64 = C.c_int, C.c_int64, C.c_float, C.c_double
u64 = C.c_uint64

# name -> (restype, argtypes)
PROTOTYPES = {
    # runtime (tp_amd_runtime.h)
    "tp_mlu_init": (i32, []),
    "tp_mlu_device_count": (i32, []),
    "tp_mlu_memory_stats": (None, [i32, I64P]),
    "tp_mlu_reset_peak_memory_stats": (None, [i32]),
    "tp_mlu_empty_cache": (None, []),
    "tp_mlu_last_error": (C.c_char_p, []),
    "tp_mlu_capture_begin": (i32, [i32]),
    "tp_mlu_capture_end": (i32, [i32]),
    "tp_mlu_capture_invoke": (i32, [i32]),
    "tp_mlu_capture_reset": (i32, []),
    "tp_mlu_capture_ready": (i32, []),
    "tp_mlu_capture_stats": (None, [I64P]),
    "tp_amd_capture_direct_kernels": (i32, []),
    "tp_amd_is_available": (i32, []),
    "tp_amd_current_device": (i32, [C.POINTER(C.c_int)]),
    "tp_amd_set_device": (i32, [i32]),
    "tp_amd_synchronize": (i32, [i32]),
    "tp_amd_mem_get_info": (i32, [i32, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "tp_amd_compute_units": (i32, [i32, C.POINTER(C.c_int)]),
    "tp_amd_copy_bytes": (i32, [VP, i32, VP, i32, C.c_size_t]),
    "tp_amd_stream": (i32, [i32, C.POINTER(VP)]),
    "tp_amd_malloc": (i32, [C.c_size_t, i32, C.POINTER(VP), C.POINTER(VP)]),
    "tp_amd_free": (None, [VP]),
    "tp_amd_block_size": (C.c_size_t, [VP]),
    "tp_amd_event_create": (i32, [C.POINTER(VP)]),
    "tp_amd_event_record": (i32, [VP, i32]),
    "tp_amd_event_elapsed_ms": (i32, [VP, VP, C.POINTER(C.c_float)]),
    "tp_amd_event_destroy": (i32, [VP]),
    "tp_amd_timer_record": (i32, [i32, C.POINTER(VP)]),
    "tp_amd_timer_elapsed_ms": (i32, [VP, VP, C.POINTER(C.c_float)]),
    "tp_amd_timer_release": (None, [VP]),
    "tp_amd_activity_start": (i32, []),
    "tp_amd_activity_stop": (i32, [C.POINTER(C.POINTER(Activity)), C.POINTER(C.c_size_t)]),
    "tp_amd_activity_push_external": (i32, [u64]),
    "tp_amd_activity_pop_external": (i32, []),
    "tp_amd_activity_error": (C.c_char_p, []),
    # kernels (tp_amd_kernels.h)
    "tp_amd_launch_binary": (i32, [i32, i32, i32, i32, I64P, VP, I64P, VP, I64P, VP, I64P, f32]),
    "tp_amd_launch_affine": (i32, [i32, i32, i64, VP, f32, f32, VP]),
    "tp_amd_launch_unary": (i32, [i32, i32, i32, i32, I64P, VP, I64P, VP, f32]),
    "tp_amd_launch_activation_backward": (i32, [i32, i32, i32, i64, VP, VP, VP, f32]),
    "tp_amd_launch_reduce": (i32, [i32, i32, i32, i64, i64, i64, VP, VP]),
    "tp_amd_launch_reduce_noalloc": (i32, [i32, i32, i32, i64, i64, i64, VP, VP]),
    "tp_amd_reduce_noalloc_scratch_bytes": (C.c_size_t, []),
    "tp_amd_reduce_partial_bytes": (i64, [i32, i32, i64, i64, i64]),
    "tp_amd_launch_softmax": (i32, [i32, i32, i32, i64, i64, i64, VP, VP]),
    "tp_amd_launch_softmax_backward": (i32, [i32, i32, i32, i64, i64, i64, VP, VP, VP]),
    "tp_amd_launch_gemm": (i32, [i32, i32, i64, i64, i64, i64, f32, VP, i64, i64, i32, VP, i64,
                                 i64, i32, f32, VP, i64, i64, i64, VP, i64, i64]),
    "tp_amd_launch_cast": (i32, [i32, i32, i32, i64, VP, VP]),
    "tp_amd_launch_fill": (i32, [i32, i32, VP, i32, I64P, VP, I64P]),
    "tp_amd_launch_strided_copy": (i32, [i32, i32, i32, I64P, VP, I64P, VP, I64P]),
    "tp_amd_launch_layer_norm": (i32, [i32, i32, i64, i64, VP, VP, VP, f64, VP, VP, VP]),
    "tp_amd_launch_layer_norm_backward": (i32, [i32, i32, i64, i64, VP, VP, VP, VP, VP, VP, VP,
                                                VP]),
    "tp_amd_launch_dropout": (i32, [i32, i32, i64, VP, f64, u64, u64, VP, VP]),
    "tp_amd_launch_dropout_backward": (i32, [i32, i32, i64, VP, VP, f64, VP]),
    "tp_amd_launch_embedding": (i32, [i32, i32, i64, i64, VP, i32, i64, VP, VP]),
    "tp_amd_launch_embedding_backward": (i32, [i32, i32, i64, i64, VP, i32, VP, i64, i64, i32,
                                               VP]),
    "tp_amd_launch_nll_loss": (i32, [i32, i32, i64, i64, VP, i32, VP, VP, i32, i64, VP, VP]),
    "tp_amd_launch_nll_loss_backward": (i32, [i32, i32, i64, i64, VP, i32, VP, VP, i32, i64, VP,
                                              VP]),
    # operators (tp_amd_ops.h)
    "tp_amd_empty": (i32, [I64P, i32, i32, i32, i32, T]),
    "tp_amd_empty_like": (i32, [T, i32, i32, T]),
    "tp_amd_zeros_like": (i32, [T, i32, i32, T]),
    "tp_amd_ones_like": (i32, [T, i32, i32, T]),
    "tp_amd_full_like": (i32, [T, Scalar, i32, i32, T]),
    "tp_amd_item": (i32, [T, C.POINTER(Scalar)]),
    "tp_amd_copy_": (i32, [T, T, i32]),
    "tp_amd_fill_": (i32, [T, Scalar]),
    "tp_amd_zero_": (i32, [T]),
    "tp_amd_clone": (i32, [T, T]),
    "tp_amd_contiguous": (i32, [T, T]),
    "tp_amd_to_dtype": (i32, [T, i32, T]),
    "tp_amd_add": (i32, [T, T, Scalar, T]),
    "tp_amd_sub": (i32, [T, T, Scalar, T]),
    "tp_amd_mul": (i32, [T, T, T]),
    "tp_amd_div": (i32, [T, T, T]),
    "tp_amd_add_": (i32, [T, T, Scalar]),
    "tp_amd_sub_": (i32, [T, T, Scalar]),
    "tp_amd_mul_": (i32, [T, T]),
    "tp_amd_div_": (i32, [T, T]),
    "tp_amd_add_scalar": (i32, [T, Scalar, Scalar, T]),
    "tp_amd_sub_scalar": (i32, [T, Scalar, Scalar, T]),
    "tp_amd_rsub_scalar": (i32, [T, Scalar, Scalar, T]),
    "tp_amd_mul_scalar": (i32, [T, Scalar, T]),
    "tp_amd_div_scalar": (i32, [T, Scalar, T]),
    "tp_amd_add__scalar": (i32, [T, Scalar, Scalar]),
    "tp_amd_mul__scalar": (i32, [T, Scalar]),
    "tp_amd_div__scalar": (i32, [T, Scalar]),
    "tp_amd_exp": (i32, [T, T]),
    "tp_amd_log": (i32, [T, T]),
    "tp_amd_sqrt": (i32, [T, T]),
    "tp_amd_rsqrt": (i32, [T, T]),
    "tp_amd_neg": (i32, [T, T]),
    "tp_amd_abs": (i32, [T, T]),
    "tp_amd_pow_scalar": (i32, [T, Scalar, T]),
    "tp_amd_relu": (i32, [T, T]),
    "tp_amd_relu_": (i32, [T]),
    "tp_amd_sigmoid": (i32, [T, T]),
    "tp_amd_tanh": (i32, [T, T]),
    "tp_amd_silu": (i32, [T, T]),
    "tp_amd_gelu": (i32, [T, i32, T]),
    "tp_amd_threshold_backward": (i32, [T, T, Scalar, T]),
    "tp_amd_sigmoid_backward": (i32, [T, T, T]),
    "tp_amd_tanh_backward": (i32, [T, T, T]),
    "tp_amd_gelu_backward": (i32, [T, T, i32, T]),
    "tp_amd_silu_backward": (i32, [T, T, T]),
    "tp_amd_mm": (i32, [T, T, T]),
    "tp_amd_bmm": (i32, [T, T, T]),
    "tp_amd_addmm": (i32, [T, T, T, Scalar, Scalar, T]),
    "tp_amd_linear": (i32, [T, T, T, T]),
    "tp_amd_matmul": (i32, [T, T, T]),
    "tp_amd_sum": (i32, [T, i32, T]),
    "tp_amd_mean": (i32, [T, i32, T]),
    "tp_amd_sum_dim": (i32, [T, I64P, i32, i32, i32, T]),
    "tp_amd_mean_dim": (i32, [T, I64P, i32, i32, i32, T]),
    "tp_amd_amax": (i32, [T, I64P, i32, i32, T]),
    "tp_amd_amin": (i32, [T, I64P, i32, i32, T]),
    "tp_amd_softmax": (i32, [T, i64, i32, T]),
    "tp_amd_log_softmax": (i32, [T, i64, i32, T]),
    "tp_amd__softmax": (i32, [T, i64, i32, T]),
    "tp_amd__log_softmax": (i32, [T, i64, i32, T]),
    "tp_amd__softmax_backward_data": (i32, [T, T, i64, i32, T]),
    "tp_amd__log_softmax_backward_data": (i32, [T, T, i64, i32, T]),
    "tp_amd_native_layer_norm": (i32, [T, I64P, i32, T, T, f64, T, T, T]),
    "tp_amd_native_layer_norm_backward": (i32, [T, T, I64P, i32, T, T, T, T, C.POINTER(C.c_int),
                                                T, T, T]),
    "tp_amd_native_dropout": (i32, [T, f64, i32, u64, T, T]),
    "tp_amd_native_dropout_backward": (i32, [T, T, f64, T]),
    "tp_amd_embedding": (i32, [T, T, i64, i32, i32, T]),
    "tp_amd_embedding_dense_backward": (i32, [T, T, i64, i64, i32, T]),
    "tp_amd_nll_loss": (i32, [T, T, T, i64, i64, T, T]),
    "tp_amd_nll_loss_backward": (i32, [T, T, T, T, i64, i64, T, T]),
    "tp_amd_binary_result_dtype": (i32, [i32, i32, i32, i32]),
    "tp_amd_broadcast_shape": (i32, [I64P, i32, I64P, i32, I64P, C.POINTER(C.c_int)]),
    "tp_amd_is_dense": (i32, [T]),
    "tp_amd_is_native_float": (i32, [i32]),
    "tp_amd_element_size": (i32, [i32]),
}


def bind(lib: C.CDLL) -> C.CDLL:
    """Attach the prototypes; a missing symbol raises AttributeError."""
    for name, (restype, argtypes) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib
