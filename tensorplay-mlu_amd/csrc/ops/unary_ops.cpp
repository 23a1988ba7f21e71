// Unary math, activations and their backward kernels: the C entry points for
// the reference's 18 unary registrations
// (tensorplay_mlu/csrc/UnaryKernels.cpp:23-310), over the gfx950 unary and
// activation-backward kernels.

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

bool native_operand(const TensorRef& t) { return on_device(t) && is_native_float(t.dtype); }

// y = f(x) into a dense result in x's dtype, or into ``out`` (unary(),
// :29-45: the result is dense; a strided ``out`` is written through a dense
// temporary).  The kernel reads a strided x in place instead of densifying
// it first; the values are the same.
Owned unary(const TensorRef& self, int op, float param, const TensorRef* out) {
    check_view(self, "self");
    if (!native_operand(self)) TP_AMD_DECLINE("unary operand is not a device float tensor");
    Owned fresh;
    TensorRef y;
    if (out != nullptr && is_contiguous(*out)) {
        y = *out;
    } else {
        fresh = empty_on(sizes_of(self), self.dtype, self.device);
        y = fresh.ref();
    }
    if (numel(y) > 0) {
        const int st = tp_amd_launch_unary(self.device, op, self.dtype, self.ndim, self.sizes,
                                           self.data, self.strides, y.data, param);
        TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    }
    if (out != nullptr && !is_contiguous(*out)) {
        strided_copy(*out, y);
        return Owned();
    }
    return fresh;
}

// self ** exponent: the common exponents take their own kernels
// (pow_scalar_native, :140-186).
Owned pow_scalar(const TensorRef& self, const tp_amd_scalar& exponent) {
    check_view(self, "self");
    if (!native_operand(self) || exponent.kind == TP_AMD_SCALAR_BOOL) {
        TP_AMD_DECLINE("pow: operand or exponent has no device kernel");
    }
    const double e = exponent.f;
    if (e == 1.0) {
        Owned out = empty_on(sizes_of(self), self.dtype, self.device);
        strided_copy(out.ref(), self);
        return out;
    }
    if (e == 0.0) {
        Owned out = empty_on(sizes_of(self), self.dtype, self.device);
        fill(out.ref(), scalar_of(1.0));
        return out;
    }
    if (e == 2.0) return unary(self, TP_AMD_UNARY_SQUARE, 0.0f, nullptr);
    if (e == 0.5) return unary(self, TP_AMD_UNARY_SQRT, 0.0f, nullptr);
    if (e == -0.5) return unary(self, TP_AMD_UNARY_RSQRT, 0.0f, nullptr);
    return unary(self, TP_AMD_UNARY_POW, static_cast<float>(e), nullptr);
}

// Both operands of a backward kernel must be native and agree in dtype and
// shape (native_backward, :217-220).
Owned backward(const TensorRef& grad, const TensorRef& saved, int op, float param) {
    check_view(grad, "grad_output");
    check_view(saved, "saved operand");
    if (!native_operand(grad) || !native_operand(saved) || grad.dtype != saved.dtype ||
        sizes_of(grad) != sizes_of(saved) || grad.device != saved.device) {
        TP_AMD_DECLINE("backward operands differ in dtype, shape or device");
    }
    MaybeOwned dy = contiguous_on_device(grad);
    MaybeOwned s = contiguous_on_device(saved);
    Owned dx = empty_on(sizes_of(grad), grad.dtype, grad.device);
    if (numel(dx.ref()) == 0) return dx;
    const int st = tp_amd_launch_activation_backward(grad.device, op, grad.dtype,
                                                     numel(dx.ref()), dy.ref.data, s.ref.data,
                                                     dx.ref().data, param);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    return dx;
}

}  // namespace

extern "C" {

#define TP_AMD_UNARY_ENTRY(NAME, OP)                                                  \
    int tp_amd_##NAME(const tp_amd_tensor* self, tp_amd_tensor* result) {             \
        return guarded_result(result,                                                 \
                              [&] { return unary(deref(self, "self"), OP, 0.0f, nullptr); }); \
    }

TP_AMD_UNARY_ENTRY(exp, TP_AMD_UNARY_EXP)
TP_AMD_UNARY_ENTRY(log, TP_AMD_UNARY_LOG)
TP_AMD_UNARY_ENTRY(sqrt, TP_AMD_UNARY_SQRT)
TP_AMD_UNARY_ENTRY(rsqrt, TP_AMD_UNARY_RSQRT)
TP_AMD_UNARY_ENTRY(neg, TP_AMD_UNARY_NEG)
TP_AMD_UNARY_ENTRY(abs, TP_AMD_UNARY_ABS)
TP_AMD_UNARY_ENTRY(relu, TP_AMD_UNARY_RELU)
TP_AMD_UNARY_ENTRY(sigmoid, TP_AMD_UNARY_SIGMOID)
TP_AMD_UNARY_ENTRY(tanh, TP_AMD_UNARY_TANH)
TP_AMD_UNARY_ENTRY(silu, TP_AMD_UNARY_SILU)
#undef TP_AMD_UNARY_ENTRY

int tp_amd_pow_scalar(const tp_amd_tensor* self, tp_amd_scalar exponent, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return pow_scalar(deref(self, "self"), exponent); });
}

int tp_amd_relu_(tp_amd_tensor* self) {
    return guarded([&] {
        const TensorRef& s = deref(self, "self");
        unary(s, TP_AMD_UNARY_RELU, 0.0f, &s);
    });
}

int tp_amd_gelu(const tp_amd_tensor* self, int approximate, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return unary(deref(self, "self"), approximate ? TP_AMD_UNARY_GELU_TANH : TP_AMD_UNARY_GELU,
                     0.0f, nullptr);
    });
}

int tp_amd_threshold_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                              tp_amd_scalar threshold, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        const TensorRef& s = deref(self, "self");
        // The threshold is encoded in the operand's dtype (:229-236).
        const float thr = round_to_dtype(static_cast<float>(threshold.f), s.dtype);
        return backward(deref(grad_output, "grad_output"), s, TP_AMD_BACKWARD_THRESHOLD, thr);
    });
}

int tp_amd_sigmoid_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* output,
                            tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return backward(deref(grad_output, "grad_output"), deref(output, "output"),
                        TP_AMD_BACKWARD_SIGMOID, 0.0f);
    });
}

int tp_amd_tanh_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* output,
                         tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return backward(deref(grad_output, "grad_output"), deref(output, "output"),
                        TP_AMD_BACKWARD_TANH, 0.0f);
    });
}

int tp_amd_gelu_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                         int approximate, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return backward(deref(grad_output, "grad_output"), deref(self, "self"),
                        approximate ? TP_AMD_BACKWARD_GELU_TANH : TP_AMD_BACKWARD_GELU, 0.0f);
    });
}

int tp_amd_silu_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                         tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return backward(deref(grad_output, "grad_output"), deref(self, "self"),
                        TP_AMD_BACKWARD_SILU, 0.0f);
    });
}

}  // extern "C"
