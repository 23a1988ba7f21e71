/* Plain-C types shared by every entry point of libtp_amd.so.
 *
 * The library is the MI355X (gfx950) device backend for TensorPlay's
 * PrivateUse1 slot.  Nothing here names a TensorPlay or torch type: tensors
 * cross the boundary as a device address plus sizes, strides and a dtype
 * code, scalars as a tagged double/int64, and every call returns a status.
 *
 * Status convention (mirrors the reference's C entry points, which return
 * 0 / non-zero and keep a thread-local message, reference
 * tensorplay_mlu/csrc/Cncl.cpp:23-27 and GraphCapture.cpp:38-57, plus the
 * "declined, run on the host" outcome of TP_CNNL_TRY, MLURuntime.h:34-51):
 *   TP_AMD_OK        the work was issued (asynchronously, on the device's
 *                    single stream) or done;
 *   TP_AMD_DECLINED  the device path does not handle these arguments (dtype,
 *                    layout); nothing was written and the caller runs the
 *                    operator on the host;
 *   TP_AMD_ERROR     a real failure; tp_mlu_last_error() has the message.
 * No C++ exception crosses this boundary.
 */
#ifndef TP_AMD_TYPES_H
#define TP_AMD_TYPES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TP_AMD_OK 0
#define TP_AMD_DECLINED 1
#define TP_AMD_ERROR (-1)

/* Most dimensions a tensor view may have (the reference's descriptors hold
 * at most 8, tensorplay_mlu/csrc/Cnnl.h:16). */
#define TP_AMD_MAX_DIMS 8

/* Element types, named after TensorPlay's DType values that the reference's
 * cast table covers (tensorplay_mlu/csrc/CopyKernels.cpp:42-108).
 * TP_AMD_UNDEFINED stands for DType::Undefined ("no dtype requested"). */
typedef enum tp_amd_dtype {
    TP_AMD_FLOAT32 = 0,
    TP_AMD_FLOAT16 = 1,
    TP_AMD_BFLOAT16 = 2,
    TP_AMD_FLOAT64 = 3,
    TP_AMD_INT8 = 4,
    TP_AMD_INT16 = 5,
    TP_AMD_INT32 = 6,
    TP_AMD_INT64 = 7,
    TP_AMD_UINT8 = 8,
    TP_AMD_BOOL = 9,
    TP_AMD_NUM_DTYPES = 10,
    TP_AMD_UNDEFINED = -1
} tp_amd_dtype;

/* A strided view of memory.  ``data`` is the address of element
 * [0, ..., 0] (storage base plus the view's offset), sizes and strides are in
 * elements, ``device`` is a device index or -1 for host memory.  ``ctx`` is
 * the allocator block that owns the memory when the library allocated it
 * (release it with tp_amd_free), NULL for borrowed memory.  A 0-d tensor has
 * ndim == 0 and one element. */
typedef struct tp_amd_tensor {
    void* data;
    void* ctx;
    int64_t sizes[TP_AMD_MAX_DIMS];
    int64_t strides[TP_AMD_MAX_DIMS];
    int32_t ndim;
    int32_t dtype;
    int32_t device;
    int32_t reserved;
} tp_amd_tensor;

/* TensorPlay's Scalar: a floating, integral or boolean value. */
typedef enum tp_amd_scalar_kind {
    TP_AMD_SCALAR_FLOAT = 0,
    TP_AMD_SCALAR_INT = 1,
    TP_AMD_SCALAR_BOOL = 2
} tp_amd_scalar_kind;

typedef struct tp_amd_scalar {
    double f;    /* the value as a double (always set) */
    int64_t i;   /* the value as an integer (set for INT and BOOL) */
    int32_t kind;
    int32_t reserved;
} tp_amd_scalar;

#ifdef __cplusplus
}
#endif

#endif /* TP_AMD_TYPES_H */
