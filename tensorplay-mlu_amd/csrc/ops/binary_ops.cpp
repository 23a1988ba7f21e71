// Elementwise add, sub, mul and div: the tensor forms, their in-place forms
// and the Scalar forms (the 16 binary registrations of
// tensorplay_mlu/csrc/BinaryKernels.cpp:252-269).
//
// Two device kernels carry all of them:
//   * tp_amd_launch_binary, out = x + k*y, x * y or x / y with broadcasting
//     strides on every operand (sub is + with k negated);
//   * tp_amd_launch_affine, out = alpha * x + beta over dense memory.
// A Scalar form, or a tensor form whose other side is a 0-d host tensor, is
// an affine map of the device tensor.  The coefficients come from one table
// (kFold), indexed by the operator and by which side the scalar is on; they
// are formed in double and rounded once to float32, as the reference rounds
// them (:113-140, :189-248).  Division by a scalar multiplies by its
// reciprocal; a scalar divided by a tensor has no affine form and declines.
//
// Declines (the host kernels run instead) follow the reference's binary()
// (:92-111): an operand that is neither a device tensor nor a 0-d host
// tensor, two host operands, two devices, a result dtype without a device
// kernel, or an in-place target whose dtype, shape or place differs from the
// result's.

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

enum Arith { kAdd = 0, kSub = 1, kMul = 2, kDiv = 3 };

struct Affine {
    double alpha;
    double beta;
};

// f(tensor) for "tensor (op) k*s" (kFold[op][0]) and "s (op) k*tensor"
// (kFold[op][1]); k is the operator's alpha (1 for mul and div).  A null
// entry has no affine form.
using FoldRule = Affine (*)(double k, double s);
constexpr FoldRule kFold[4][2] = {
    {[](double k, double s) { return Affine{1.0, k * s}; },    // t + k s
     [](double k, double s) { return Affine{k, s}; }},         // s + k t
    {[](double k, double s) { return Affine{1.0, -(k * s)}; }, // t - k s
     [](double k, double s) { return Affine{-k, s}; }},        // s - k t
    {[](double k, double s) { return Affine{k * s, 0.0}; },    // t * s
     [](double k, double s) { return Affine{k * s, 0.0}; }},   // s * t
    {[](double, double s) { return Affine{1.0 / s, 0.0}; },    // t / s
     nullptr},                                                  // s / t
};

// out = alpha * x + beta elementwise (x and out of one shape and dtype, both
// on out's device).  The kernel walks dense memory: a strided x is packed
// first, a strided out receives a dense result.
void apply_affine(const TensorRef& x, const Affine& f, const TensorRef& out) {
    if (numel(out) == 0) return;
    const MaybeOwned src = contiguous_on_device(x);
    Owned staging;
    void* dst = out.data;
    if (!is_contiguous(out)) {
        staging = empty_on(sizes_of(out), out.dtype, out.device);
        dst = staging.ref().data;
    }
    const int st = tp_amd_launch_affine(out.device, out.dtype, numel(out), src.ref.data,
                                        static_cast<float>(f.alpha), static_cast<float>(f.beta), dst);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    if (staging.ref().ctx != nullptr) strided_copy(out, staging.ref());
}

// Where the result of a tensor form goes: ``target`` (in-place forms) or a
// new tensor of the broadcast shape.
struct Destination {
    Owned fresh;
    TensorRef view;
};

Destination destination(const TensorRef* target, const Sizes& shape, int dtype, int device) {
    Destination d;
    if (target != nullptr) {
        if (!on_device(*target) || target->dtype != dtype || sizes_of(*target) != shape) {
            TP_AMD_DECLINE("in-place target differs from the result in dtype, shape or device");
        }
        d.view = *target;
    } else {
        d.fresh = empty_on(shape, dtype, device);
        d.view = d.fresh.ref();
    }
    return d;
}

// x (op) k*y for the tensor forms, written to ``target`` when given.
Owned tensor_form(const TensorRef& x, const TensorRef& y, Arith op, double k, const TensorRef* target) {
    check_view(x, "self");
    check_view(y, "other");
    const bool x_dev = on_device(x), y_dev = on_device(y);
    const bool x_ok = x_dev || is_host_scalar(x), y_ok = y_dev || is_host_scalar(y);
    if (!x_ok || !y_ok || !(x_dev || y_dev)) {
        TP_AMD_DECLINE("binary operands must be device tensors or 0-d host scalars, one on the device");
    }
    if (x_dev && y_dev && x.device != y.device) TP_AMD_DECLINE("binary operands on two devices");
    const int dtype = binary_result_dtype(x.dtype, x.ndim, y.dtype, y.ndim);
    if (!is_native_float(dtype)) TP_AMD_DECLINE("binary result dtype has no device kernel");
    const int device = x_dev ? x.device : y.device;
    const Sizes shape = broadcast_shape(sizes_of(x), sizes_of(y));
    Destination out = destination(target, shape, dtype, device);
    if (numel(out.view) == 0) return std::move(out.fresh);

    if (!(x_dev && y_dev)) {
        // One side is a host scalar; the device side already has the full
        // shape (a 0-d operand broadcasts to the other's shape).
        const int side = x_dev ? 0 : 1;
        const FoldRule rule = kFold[op][side];
        if (rule == nullptr) TP_AMD_DECLINE("a host scalar divided by a device tensor");
        const MaybeOwned t = to_dtype(x_dev ? x : y, dtype);
        apply_affine(t.ref, rule(k, host_scalar_value(x_dev ? y : x)), out.view);
        return std::move(out.fresh);
    }
    const MaybeOwned xc = to_dtype(x, dtype), yc = to_dtype(y, dtype);
    const TensorRef xe = expand_to(xc.ref, shape), ye = expand_to(yc.ref, shape);
    const int kernel_op = op == kMul ? TP_AMD_BINARY_MUL : op == kDiv ? TP_AMD_BINARY_DIV : TP_AMD_BINARY_ADD;
    const float scale = static_cast<float>(op == kSub ? -k : k);
    const int st = tp_amd_launch_binary(out.view.device, kernel_op, dtype, out.view.ndim, out.view.sizes,
                                        xe.data, xe.strides, ye.data, ye.strides, out.view.data,
                                        out.view.strides, scale);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    return std::move(out.fresh);
}

// A Scalar form: self (op) k*s, or s (op) k*self for rsub.
Owned scalar_form(const TensorRef& self, Arith op, int side, double k, double s, const TensorRef* target) {
    check_view(self, "self");
    if (!on_device(self) || !is_native_float(self.dtype)) {
        TP_AMD_DECLINE("Scalar forms run on the device for float device tensors");
    }
    Destination out = destination(target, sizes_of(self), self.dtype, self.device);
    apply_affine(self, kFold[op][side](k, s), out.view);
    return std::move(out.fresh);
}

const TensorRef& lhs(const tp_amd_tensor* p) { return deref(p, "self"); }
const TensorRef& rhs(const tp_amd_tensor* p) { return deref(p, "other"); }

}  // namespace

extern "C" {

int tp_amd_add(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha,
               tp_amd_tensor* result) {
    return guarded_result(result, [&] { return tensor_form(lhs(self), rhs(other), kAdd, alpha.f, nullptr); });
}

int tp_amd_sub(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha,
               tp_amd_tensor* result) {
    return guarded_result(result, [&] { return tensor_form(lhs(self), rhs(other), kSub, alpha.f, nullptr); });
}

int tp_amd_mul(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return tensor_form(lhs(self), rhs(other), kMul, 1.0, nullptr); });
}

int tp_amd_div(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return tensor_form(lhs(self), rhs(other), kDiv, 1.0, nullptr); });
}

int tp_amd_add_(tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha) {
    return guarded([&] { tensor_form(lhs(self), rhs(other), kAdd, alpha.f, &lhs(self)); });
}

int tp_amd_sub_(tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha) {
    return guarded([&] { tensor_form(lhs(self), rhs(other), kSub, alpha.f, &lhs(self)); });
}

int tp_amd_mul_(tp_amd_tensor* self, const tp_amd_tensor* other) {
    return guarded([&] { tensor_form(lhs(self), rhs(other), kMul, 1.0, &lhs(self)); });
}

int tp_amd_div_(tp_amd_tensor* self, const tp_amd_tensor* other) {
    return guarded([&] { tensor_form(lhs(self), rhs(other), kDiv, 1.0, &lhs(self)); });
}

int tp_amd_add_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                      tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_form(lhs(self), kAdd, 0, alpha.f, other.f, nullptr); });
}

int tp_amd_sub_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                      tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_form(lhs(self), kSub, 0, alpha.f, other.f, nullptr); });
}

int tp_amd_rsub_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                       tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_form(lhs(self), kSub, 1, alpha.f, other.f, nullptr); });
}

int tp_amd_mul_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_form(lhs(self), kMul, 0, 1.0, other.f, nullptr); });
}

int tp_amd_div_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return scalar_form(lhs(self), kDiv, 0, 1.0, other.f, nullptr); });
}

int tp_amd_add__scalar(tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha) {
    return guarded([&] { scalar_form(lhs(self), kAdd, 0, alpha.f, other.f, &lhs(self)); });
}

int tp_amd_mul__scalar(tp_amd_tensor* self, tp_amd_scalar other) {
    return guarded([&] { scalar_form(lhs(self), kMul, 0, 1.0, other.f, &lhs(self)); });
}

int tp_amd_div__scalar(tp_amd_tensor* self, tp_amd_scalar other) {
    return guarded([&] { scalar_form(lhs(self), kDiv, 0, 1.0, other.f, &lhs(self)); });
}

}  // extern "C"
