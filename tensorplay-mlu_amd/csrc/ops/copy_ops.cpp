// Factories, copies, casts and fills: the C entry points for the reference's
// 13 copy registrations (tensorplay_mlu/csrc/CopyKernels.cpp:231-364).

#include <cstring>

#include "../runtime.h"
#include "tensor.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

int resolve_dtype(int requested, int fallback) {
    return requested == TP_AMD_UNDEFINED ? fallback : requested;
}

Owned like(const tp_amd_tensor* self, int dtype, int device) {
    TP_AMD_CHECK(self != nullptr, "null tensor");
    check_view(*self, "self");
    const int type = resolve_dtype(dtype, self->dtype);
    const int index = device >= 0 ? device : (self->device >= 0 ? self->device : -1);
    return empty_on(sizes_of(*self), type, index);
}

}  // namespace

extern "C" {

int tp_amd_empty(const int64_t* sizes, int ndim, int dtype, int device, int pin_memory,
                 tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        TP_AMD_CHECK(!pin_memory, "device tensors cannot be pinned host memory");
        TP_AMD_CHECK(ndim >= 0 && (ndim == 0 || sizes != nullptr), "bad sizes");
        return empty_on(Sizes(sizes, sizes + ndim), resolve_dtype(dtype, TP_AMD_FLOAT32),
                        device);
    });
}

int tp_amd_empty_like(const tp_amd_tensor* self, int dtype, int device, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return like(self, dtype, device); });
}

int tp_amd_full_like(const tp_amd_tensor* self, tp_amd_scalar value, int dtype, int device,
                     tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        Owned out = like(self, dtype, device);
        fill(out.ref(), value);
        return out;
    });
}

int tp_amd_zeros_like(const tp_amd_tensor* self, int dtype, int device, tp_amd_tensor* result) {
    tp_amd_scalar zero{};
    zero.kind = TP_AMD_SCALAR_INT;
    return tp_amd_full_like(self, zero, dtype, device, result);
}

int tp_amd_ones_like(const tp_amd_tensor* self, int dtype, int device, tp_amd_tensor* result) {
    tp_amd_scalar one{};
    one.f = 1.0;
    one.i = 1;
    one.kind = TP_AMD_SCALAR_INT;
    return tp_amd_full_like(self, one, dtype, device, result);
}

int tp_amd_item(const tp_amd_tensor* self, tp_amd_scalar* value) {
    return guarded([&] {
        TP_AMD_CHECK(self != nullptr && value != nullptr, "null argument");
        check_view(*self, "self");
        TP_AMD_CHECK(numel(*self) == 1, "item() only supported for 1-element tensors");
        alignas(8) unsigned char bytes[8] = {};
        if (on_device(*self)) {
            copy_to_host(bytes, self->data, element_size(self->dtype), self->device);
        } else {
            std::memcpy(bytes, self->data, element_size(self->dtype));
        }
        TensorRef host = *self;
        host.data = bytes;
        host.device = -1;
        tp_amd_scalar out{};
        out.f = host_scalar_value(host);
        if (is_floating(self->dtype)) {
            out.kind = TP_AMD_SCALAR_FLOAT;
            out.i = static_cast<int64_t>(out.f);
        } else {
            out.kind = self->dtype == TP_AMD_BOOL ? TP_AMD_SCALAR_BOOL : TP_AMD_SCALAR_INT;
            if (self->dtype == TP_AMD_INT64) {
                std::memcpy(&out.i, bytes, 8);
            } else {
                out.i = static_cast<int64_t>(out.f);
            }
        }
        *value = out;
    });
}

int tp_amd_copy_(tp_amd_tensor* self, const tp_amd_tensor* src, int non_blocking) {
    (void)non_blocking;
    return guarded([&] {
        TP_AMD_CHECK(self != nullptr && src != nullptr, "null tensor");
        copy_into(*self, *src);
    });
}

int tp_amd_fill_(tp_amd_tensor* self, tp_amd_scalar value) {
    return guarded([&] {
        TP_AMD_CHECK(self != nullptr, "null tensor");
        check_view(*self, "self");
        fill(*self, value);
    });
}

int tp_amd_zero_(tp_amd_tensor* self) {
    tp_amd_scalar zero{};
    zero.kind = TP_AMD_SCALAR_INT;
    return tp_amd_fill_(self, zero);
}

int tp_amd_clone(const tp_amd_tensor* self, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        TP_AMD_CHECK(self != nullptr, "null tensor");
        check_view(*self, "self");
        Owned out = empty_on(sizes_of(*self), self->dtype, self->device);
        strided_copy(out.ref(), *self);
        return out;
    });
}

int tp_amd_contiguous(const tp_amd_tensor* self, tp_amd_tensor* result) {
    return guarded([&] {
        TP_AMD_CHECK(self != nullptr && result != nullptr, "null tensor");
        check_view(*self, "self");
        if (is_contiguous(*self)) {
            *result = *self;
            result->ctx = nullptr;
            return;
        }
        Owned out = empty_on(sizes_of(*self), self->dtype, self->device);
        strided_copy(out.ref(), *self);
        *result = out.release();
    });
}

int tp_amd_to_dtype(const tp_amd_tensor* self, int dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        TP_AMD_CHECK(self != nullptr, "null tensor");
        check_view(*self, "self");
        Owned out = empty_on(sizes_of(*self), dtype, self->device);
        copy_into(out.ref(), *self);
        return out;
    });
}

int tp_amd_binary_result_dtype(int a_dtype, int a_ndim, int b_dtype, int b_ndim) {
    return binary_result_dtype(a_dtype, a_ndim, b_dtype, b_ndim);
}

int tp_amd_broadcast_shape(const int64_t* a, int a_ndim, const int64_t* b, int b_ndim,
                           int64_t* out, int* out_ndim) {
    return guarded([&] {
        const Sizes s = broadcast_shape(Sizes(a, a + a_ndim), Sizes(b, b + b_ndim));
        TP_AMD_CHECK(s.size() <= TP_AMD_MAX_DIMS, "broadcast result has too many dims");
        for (size_t i = 0; i < s.size(); ++i) out[i] = s[i];
        *out_ndim = static_cast<int>(s.size());
    });
}

int tp_amd_is_dense(const tp_amd_tensor* t) { return t != nullptr && is_dense(*t) ? 1 : 0; }

int tp_amd_is_native_float(int dtype) { return is_native_float(dtype) ? 1 : 0; }

int tp_amd_element_size(int dtype) { return element_size(dtype); }

}  // extern "C"
