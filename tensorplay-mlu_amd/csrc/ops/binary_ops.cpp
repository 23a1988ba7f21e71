// Binary arithmetic: the reference's binary() dispatch, affine folding of
// host scalars and the scalar forms (tensorplay_mlu/csrc/BinaryKernels.cpp:
// 20-248), over the gfx950 binary and affine kernels.

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

enum class BinOp { Add, Sub, Mul, Div };

// y = alpha * x + beta into ``out`` (same shape as x).  The transform reads
// and writes dense memory: a strided x is made dense first and a strided
// out written through a dense result (BinaryKernels.cpp:30-40).
void affine(const TensorRef& x, float alpha, float beta, const TensorRef& out) {
    MaybeOwned xc = contiguous_on_device(x);
    Owned tmp;
    TensorRef y = out;
    if (!is_contiguous(out)) {
        tmp = empty_on(sizes_of(out), out.dtype, out.device);
        y = tmp.ref();
    }
    const int st = tp_amd_launch_affine(out.device, out.dtype, numel(out), xc.ref.data, alpha,
                                        beta, y.data);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    if (!is_contiguous(out)) strided_copy(out, y);
}

// out = a (op) scale * b with broadcasting (launch_binary, :44-87).
void launch_binary(const TensorRef& a, const TensorRef& b, BinOp op, const TensorRef& out,
                   float scale) {
    const Sizes shape = sizes_of(out);
    const TensorRef ae = expand_to(a, shape), be = expand_to(b, shape);
    const int kop = op == BinOp::Mul ? TP_AMD_BINARY_MUL
                    : op == BinOp::Div ? TP_AMD_BINARY_DIV : TP_AMD_BINARY_ADD;
    const float alpha = op == BinOp::Sub ? -scale : scale;
    const int st = tp_amd_launch_binary(out.device, kop, out.dtype, out.ndim, out.sizes, ae.data,
                                        ae.strides, be.data, be.strides, out.data, out.strides,
                                        alpha);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
}

// The native path (binary(), :92-146); declines when the operands need the
// host.  ``out`` (in-place forms) must already have the result's shape and
// dtype.
Owned binary(const TensorRef& a, const TensorRef& b, double alpha, BinOp op,
             const TensorRef* out) {
    check_view(a, "self");
    check_view(b, "other");
    const bool a_dev = on_device(a), b_dev = on_device(b);
    if (!(a_dev || is_host_scalar(a)) || !(b_dev || is_host_scalar(b))) {
        TP_AMD_DECLINE("operands are neither device tensors nor host 0-d scalars");
    }
    if (!a_dev && !b_dev) TP_AMD_DECLINE("no operand is on the device");
    const int device = a_dev ? a.device : b.device;
    if (a_dev && b_dev && a.device != b.device) TP_AMD_DECLINE("operands on different devices");
    const int dtype = binary_result_dtype(a.dtype, a.ndim, b.dtype, b.ndim);
    if (!is_native_float(dtype)) TP_AMD_DECLINE("result dtype has no device kernel");
    const Sizes shape = broadcast_shape(sizes_of(a), sizes_of(b));
    if (out != nullptr) {
        if (out->dtype != dtype || sizes_of(*out) != shape || !on_device(*out)) {
            TP_AMD_DECLINE("in-place result does not match the operation's shape or dtype");
        }
    }
    Owned fresh;
    TensorRef result;
    if (out != nullptr) {
        result = *out;
    } else {
        fresh = empty_on(shape, dtype, device);
        result = fresh.ref();
    }
    if (numel(result) == 0) return fresh;

    // A host scalar folds into an affine transform of the other operand
    // (:113-140).
    if (!a_dev || !b_dev) {
        const double s = host_scalar_value(a_dev ? b : a);
        MaybeOwned x = to_dtype(a_dev ? a : b, dtype);
        if (sizes_of(x.ref) != shape) TP_AMD_DECLINE("host scalar with a broadcast operand");
        if (a_dev) {
            switch (op) {
                case BinOp::Add: affine(x.ref, 1.0f, static_cast<float>(alpha * s), result); break;
                case BinOp::Sub: affine(x.ref, 1.0f, static_cast<float>(-alpha * s), result); break;
                case BinOp::Mul: affine(x.ref, static_cast<float>(alpha * s), 0.0f, result); break;
                case BinOp::Div: affine(x.ref, static_cast<float>(1.0 / s), 0.0f, result); break;
            }
        } else {
            switch (op) {
                case BinOp::Add:
                    affine(x.ref, static_cast<float>(alpha), static_cast<float>(s), result);
                    break;
                case BinOp::Sub:
                    affine(x.ref, static_cast<float>(-alpha), static_cast<float>(s), result);
                    break;
                case BinOp::Mul: affine(x.ref, static_cast<float>(alpha * s), 0.0f, result); break;
                case BinOp::Div: TP_AMD_DECLINE("host scalar divided by a device tensor");
            }
        }
        return fresh;
    }
    MaybeOwned ac = to_dtype(a, dtype), bc = to_dtype(b, dtype);
    launch_binary(ac.ref, bc.ref, op, result, static_cast<float>(alpha));
    return fresh;
}

// Scalar forms: one affine transform (scalar_affine, :189-202).
Owned scalar_affine(const TensorRef& self, double alpha, double beta, const TensorRef* out) {
    check_view(self, "self");
    if (!on_device(self) || !is_native_float(self.dtype)) {
        TP_AMD_DECLINE("scalar form of a host or non-float tensor");
    }
    Owned fresh;
    TensorRef result;
    if (out != nullptr) {
        result = *out;
    } else {
        fresh = empty_on(sizes_of(self), self.dtype, self.device);
        result = fresh.ref();
    }
    if (numel(result) > 0) affine(self, static_cast<float>(alpha), static_cast<float>(beta), result);
    return fresh;
}

}  // namespace

extern "C" {

int tp_amd_add(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha,
               tp_amd_tensor* result) {
    return guarded_result(result, [&] { return binary(deref(self, "self"), deref(other, "other"), alpha.f, BinOp::Add, nullptr); });
}

int tp_amd_sub(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha,
               tp_amd_tensor* result) {
    return guarded_result(result, [&] { return binary(deref(self, "self"), deref(other, "other"), alpha.f, BinOp::Sub, nullptr); });
}

int tp_amd_mul(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return binary(deref(self, "self"), deref(other, "other"), 1.0, BinOp::Mul, nullptr); });
}

int tp_amd_div(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return binary(deref(self, "self"), deref(other, "other"), 1.0, BinOp::Div, nullptr); });
}

int tp_amd_add_(tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha) {
    return guarded([&] { binary(deref(self, "self"), deref(other, "other"), alpha.f, BinOp::Add, &deref(self, "self")); });
}

int tp_amd_sub_(tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha) {
    return guarded([&] { binary(deref(self, "self"), deref(other, "other"), alpha.f, BinOp::Sub, &deref(self, "self")); });
}

int tp_amd_mul_(tp_amd_tensor* self, const tp_amd_tensor* other) {
    return guarded([&] { binary(deref(self, "self"), deref(other, "other"), 1.0, BinOp::Mul, &deref(self, "self")); });
}

int tp_amd_div_(tp_amd_tensor* self, const tp_amd_tensor* other) {
    return guarded([&] { binary(deref(self, "self"), deref(other, "other"), 1.0, BinOp::Div, &deref(self, "self")); });
}

int tp_amd_add_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                      tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_affine(deref(self, "self"), 1.0, alpha.f * other.f, nullptr); });
}

int tp_amd_sub_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                      tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_affine(deref(self, "self"), 1.0, -alpha.f * other.f, nullptr); });
}

int tp_amd_rsub_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                       tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_affine(deref(self, "self"), -alpha.f, other.f, nullptr); });
}

int tp_amd_mul_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_affine(deref(self, "self"), other.f, 0.0, nullptr); });
}

int tp_amd_div_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_affine(deref(self, "self"), 1.0 / other.f, 0.0, nullptr); });
}

int tp_amd_add__scalar(tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha) {
    return guarded([&] { scalar_affine(deref(self, "self"), 1.0, alpha.f * other.f, &deref(self, "self")); });
}

int tp_amd_mul__scalar(tp_amd_tensor* self, tp_amd_scalar other) {
    return guarded([&] { scalar_affine(deref(self, "self"), other.f, 0.0, &deref(self, "self")); });
}

int tp_amd_div__scalar(tp_amd_tensor* self, tp_amd_scalar other) {
    return guarded([&] { scalar_affine(deref(self, "self"), 1.0 / other.f, 0.0, &deref(self, "self")); });
}

}  // extern "C"
