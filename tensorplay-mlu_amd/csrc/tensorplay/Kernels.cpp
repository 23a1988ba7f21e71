// The 72 PrivateUse1 operator registrations (the 64 of the hot path and the
// 8 neural-network layers), each a thin wrapper over one operator C-ABI
// entry (tp_amd_ops.h).  The C-ABI keeps the
// reference operators' dtype rules and decline conditions; when it declines
// (TP_AMD_DECLINED), or a tensor cannot be described as a view, the wrapper
// runs TensorPlay's host kernel through cpu_fallback, as the reference does.
//
// Registration blocks mirror tensorplay_mlu/csrc/CopyKernels.cpp:349-364,
// BinaryKernels.cpp:252-269, UnaryKernels.cpp:291-310,
// BlasKernels.cpp:416-422, ReduceKernels.cpp:267-282 and
// NNKernels.cpp:399-410: same operator names, same signature types.

#include <array>
#include <functional>
#include <tuple>

#include "Adapter.h"
#include "Generator.h"

namespace tensorplay {
namespace amd {

namespace {

namespace sig = kernel_signatures;

// ---- helpers -------------------------------------------------------------

using UnaryEntry = int (*)(const tp_amd_tensor*, tp_amd_tensor*);
using BinaryEntry = int (*)(const tp_amd_tensor*, const tp_amd_tensor*, tp_amd_tensor*);

Native<Tensor> unary(const char* op, UnaryEntry entry, const Tensor& self) {
    tp_amd_tensor x;
    if (!view(self, &x)) return std::nullopt;
    return produce(op, [&](tp_amd_tensor* r) { return entry(&x, r); });
}

Native<Tensor> binary(const char* op, BinaryEntry entry, const Tensor& a, const Tensor& b) {
    tp_amd_tensor x, y;
    if (!view(a, &x) || !view(b, &y)) return std::nullopt;
    return produce(op, [&](tp_amd_tensor* r) { return entry(&x, &y, r); });
}

Tensor must(const char* op, Native<Tensor> r) {
    TP_CHECK(r.has_value(), "tensorplay-mlu_amd: ", op, " was declined");
    return std::move(*r);
}

int dtype_arg(DType dtype) {
    return dtype == DType::Undefined ? TP_AMD_UNDEFINED : dtype_code(dtype);
}

// ---- factories, copies, fills (reference CopyKernels.cpp:231-345) ---------

// empty on the device: any dtype TensorPlay stores, as raw bytes.
Tensor empty_on(const std::vector<int64_t>& size, DType dtype, int index) {
    const int code = dtype_code(dtype);
    if (code != TP_AMD_UNDEFINED && size.size() <= TP_AMD_MAX_DIMS) {
        return must("empty", produce("empty", [&](tp_amd_tensor* r) {
                        return tp_amd_empty(size.data(), static_cast<int>(size.size()), code,
                                            index, 0, r);
                    }));
    }
    int64_t numel = 1;
    for (int64_t d : size) {
        TP_CHECK(d >= 0, "negative dimension in empty");
        numel *= d;
    }
    const int placed = index >= 0 ? index : index_of(Device(DeviceType::PrivateUse1, -1));
    Storage storage(static_cast<size_t>(numel) * elementSize(dtype), allocator(),
                    Device(DeviceType::PrivateUse1, placed));
    return Tensor(std::move(storage), size, dtype);
}

Tensor empty_kernel(const std::vector<int64_t>& size, std::optional<DType> dtype,
                    std::optional<Device> device, bool pin_memory) {
    TP_CHECK(!pin_memory, "device tensors cannot be pinned host memory");
    return empty_on(size, dtype.value_or(DType::Float32), device ? index_of(*device) : -1);
}

Tensor empty_memory_format_kernel(const std::vector<int64_t>& size, std::optional<DType> dtype,
                                  std::optional<int64_t> layout, std::optional<Device> device,
                                  std::optional<bool> pin_memory,
                                  std::optional<int64_t> memory_format) {
    (void)layout;
    (void)memory_format;
    return empty_kernel(size, dtype, device, pin_memory.value_or(false));
}

Tensor empty_like_kernel(const Tensor& self, DType dtype, std::optional<Device> device) {
    const DType type = dtype == DType::Undefined ? self.dtype() : dtype;
    if (device && !device->is_privateuse1()) return Tensor(self.sizes().vec(), type, *device);
    return empty_on(self.sizes().vec(), type,
                    device ? index_of(*device) : index_of(self.device()));
}

Tensor full_like_kernel(const Tensor& self, const Scalar& value, DType dtype,
                        std::optional<Device> device) {
    Tensor result = empty_like_kernel(self, dtype, device);
    result.fill_(value);
    return result;
}

Tensor zeros_like_kernel(const Tensor& self, DType dtype, std::optional<Device> device) {
    return full_like_kernel(self, Scalar(int64_t(0)), dtype, device);
}

Tensor ones_like_kernel(const Tensor& self, DType dtype, std::optional<Device> device) {
    return full_like_kernel(self, Scalar(int64_t(1)), dtype, device);
}

Scalar item_kernel(const Tensor& self) {
    TP_CHECK(self.numel() == 1, "item() only supported for 1-element tensors");
    tp_amd_tensor x;
    if (view(self, &x)) {
        tp_amd_scalar value{};
        const int status = tp_amd_item(&x, &value);
        if (status == TP_AMD_OK) return to_scalar(value);
        if (status != TP_AMD_DECLINED) raise("item");
    }
    return cpu_fallback::Kernel<"item", sig::item>::call(self);
}

Tensor& copy_kernel(Tensor& self, const Tensor& src, bool non_blocking) {
    tp_amd_tensor dst, from;
    if (view(self, &dst) && view(src, &from) &&
        in_place("copy_", [&] { return tp_amd_copy_(&dst, &from, non_blocking ? 1 : 0); })) {
        return self;
    }
    return cpu_fallback::Kernel<"copy_", sig::copy_>::call(self, src, non_blocking);
}

Tensor& fill_kernel(Tensor& self, const Scalar& value) {
    tp_amd_tensor t;
    if (view(self, &t) && in_place("fill_", [&] { return tp_amd_fill_(&t, scalar(value)); })) {
        return self;
    }
    return cpu_fallback::Kernel<"fill_.Scalar", sig::fill___Scalar>::call(self, value);
}

Tensor& zero_kernel(Tensor& self) { return fill_kernel(self, Scalar(int64_t(0))); }

Tensor clone_kernel(const Tensor& self, std::optional<int64_t> memory_format) {
    if (auto r = unary("clone", tp_amd_clone, self)) return *r;
    return cpu_fallback::Kernel<"clone", sig::clone>::call(self, memory_format);
}

Tensor contiguous_kernel(const Tensor& self, int64_t memory_format) {
    if (self.is_contiguous()) return self;
    if (auto r = unary("contiguous", tp_amd_clone, self)) return *r;
    return cpu_fallback::Kernel<"contiguous", sig::contiguous>::call(self, memory_format);
}

// ---- binary arithmetic (reference BinaryKernels.cpp:148-248) -------------

using AlphaEntry = int (*)(const tp_amd_tensor*, const tp_amd_tensor*, tp_amd_scalar,
                           tp_amd_tensor*);

Native<Tensor> with_alpha(const char* op, AlphaEntry entry, const Tensor& a, const Tensor& b,
                          const Scalar& alpha) {
    tp_amd_tensor x, y;
    if (!view(a, &x) || !view(b, &y)) return std::nullopt;
    return produce(op, [&](tp_amd_tensor* r) { return entry(&x, &y, scalar(alpha), r); });
}

bool into_self(const char* op, const Tensor& self, const Tensor& other,
               const std::function<int(tp_amd_tensor*, const tp_amd_tensor*)>& entry) {
    tp_amd_tensor x, y;
    if (!view(self, &x) || !view(other, &y)) return false;
    return in_place(op, [&] { return entry(&x, &y); });
}

Tensor add_kernel(const Tensor& self, const Tensor& other, const Scalar& alpha) {
    if (auto r = with_alpha("add", tp_amd_add, self, other, alpha)) return *r;
    return cpu_fallback::Kernel<"add.Tensor", sig::add__Tensor>::call(self, other, alpha);
}

Tensor sub_kernel(const Tensor& self, const Tensor& other, const Scalar& alpha) {
    if (auto r = with_alpha("sub", tp_amd_sub, self, other, alpha)) return *r;
    return cpu_fallback::Kernel<"sub.Tensor", sig::sub__Tensor>::call(self, other, alpha);
}

Tensor mul_kernel(const Tensor& self, const Tensor& other) {
    if (auto r = binary("mul", tp_amd_mul, self, other)) return *r;
    return cpu_fallback::Kernel<"mul.Tensor", sig::mul__Tensor>::call(self, other);
}

Tensor div_kernel(const Tensor& self, const Tensor& other) {
    if (auto r = binary("div", tp_amd_div, self, other)) return *r;
    return cpu_fallback::Kernel<"div.Tensor", sig::div__Tensor>::call(self, other);
}

Tensor& add__kernel(Tensor& self, const Tensor& other, const Scalar& alpha) {
    const tp_amd_scalar a = scalar(alpha);
    if (into_self("add_", self, other, [&](tp_amd_tensor* x, const tp_amd_tensor* y) {
            return tp_amd_add_(x, y, a);
        })) {
        return self;
    }
    return cpu_fallback::Kernel<"add_.Tensor", sig::add___Tensor>::call(self, other, alpha);
}

Tensor& sub__kernel(Tensor& self, const Tensor& other, const Scalar& alpha) {
    const tp_amd_scalar a = scalar(alpha);
    if (into_self("sub_", self, other, [&](tp_amd_tensor* x, const tp_amd_tensor* y) {
            return tp_amd_sub_(x, y, a);
        })) {
        return self;
    }
    return cpu_fallback::Kernel<"sub_.Tensor", sig::sub___Tensor>::call(self, other, alpha);
}

Tensor& mul__kernel(Tensor& self, const Tensor& other) {
    if (into_self("mul_", self, other, tp_amd_mul_)) return self;
    return cpu_fallback::Kernel<"mul_.Tensor", sig::mul___Tensor>::call(self, other);
}

Tensor& div__kernel(Tensor& self, const Tensor& other) {
    if (into_self("div_", self, other, tp_amd_div_)) return self;
    return cpu_fallback::Kernel<"div_.Tensor", sig::div___Tensor>::call(self, other);
}

using ScalarAlphaEntry = int (*)(const tp_amd_tensor*, tp_amd_scalar, tp_amd_scalar,
                                 tp_amd_tensor*);
using ScalarEntry = int (*)(const tp_amd_tensor*, tp_amd_scalar, tp_amd_tensor*);

Native<Tensor> scalar_alpha(const char* op, ScalarAlphaEntry entry, const Tensor& self,
                            const Scalar& other, const Scalar& alpha) {
    tp_amd_tensor x;
    if (!view(self, &x)) return std::nullopt;
    return produce(op,
                   [&](tp_amd_tensor* r) { return entry(&x, scalar(other), scalar(alpha), r); });
}

Native<Tensor> scalar_only(const char* op, ScalarEntry entry, const Tensor& self,
                           const Scalar& other) {
    tp_amd_tensor x;
    if (!view(self, &x)) return std::nullopt;
    return produce(op, [&](tp_amd_tensor* r) { return entry(&x, scalar(other), r); });
}

Tensor add_scalar_kernel(const Tensor& self, const Scalar& other, const Scalar& alpha) {
    if (auto r = scalar_alpha("add.Scalar", tp_amd_add_scalar, self, other, alpha)) return *r;
    return cpu_fallback::Kernel<"add.Scalar", sig::add__Scalar>::call(self, other, alpha);
}

Tensor sub_scalar_kernel(const Tensor& self, const Scalar& other, const Scalar& alpha) {
    if (auto r = scalar_alpha("sub.Scalar", tp_amd_sub_scalar, self, other, alpha)) return *r;
    return cpu_fallback::Kernel<"sub.Scalar", sig::sub__Scalar>::call(self, other, alpha);
}

Tensor rsub_scalar_kernel(const Tensor& self, const Scalar& other, const Scalar& alpha) {
    if (auto r = scalar_alpha("rsub.Scalar", tp_amd_rsub_scalar, self, other, alpha)) return *r;
    return cpu_fallback::Kernel<"rsub.Scalar", sig::rsub__Scalar>::call(self, other, alpha);
}

Tensor mul_scalar_kernel(const Tensor& self, const Scalar& other) {
    if (auto r = scalar_only("mul.Scalar", tp_amd_mul_scalar, self, other)) return *r;
    return cpu_fallback::Kernel<"mul.Scalar", sig::mul__Scalar>::call(self, other);
}

Tensor div_scalar_kernel(const Tensor& self, const Scalar& other) {
    if (auto r = scalar_only("div.Scalar", tp_amd_div_scalar, self, other)) return *r;
    return cpu_fallback::Kernel<"div.Scalar", sig::div__Scalar>::call(self, other);
}

Tensor& add__scalar_kernel(Tensor& self, const Scalar& other, const Scalar& alpha) {
    tp_amd_tensor x;
    if (view(self, &x) && in_place("add_.Scalar", [&] {
            return tp_amd_add__scalar(&x, scalar(other), scalar(alpha));
        })) {
        return self;
    }
    return cpu_fallback::Kernel<"add_.Scalar", sig::add___Scalar>::call(self, other, alpha);
}

Tensor& mul__scalar_kernel(Tensor& self, const Scalar& other) {
    tp_amd_tensor x;
    if (view(self, &x) &&
        in_place("mul_.Scalar", [&] { return tp_amd_mul__scalar(&x, scalar(other)); })) {
        return self;
    }
    return cpu_fallback::Kernel<"mul_.Scalar", sig::mul___Scalar>::call(self, other);
}

Tensor& div__scalar_kernel(Tensor& self, const Scalar& other) {
    tp_amd_tensor x;
    if (view(self, &x) &&
        in_place("div_.Scalar", [&] { return tp_amd_div__scalar(&x, scalar(other)); })) {
        return self;
    }
    return cpu_fallback::Kernel<"div_.Scalar", sig::div___Scalar>::call(self, other);
}

// ---- unary math, activations, backward (reference UnaryKernels.cpp) ------

Tensor exp_kernel(const Tensor& self) {
    if (auto r = unary("exp", tp_amd_exp, self)) return *r;
    return cpu_fallback::Kernel<"exp", sig::exp>::call(self);
}

Tensor log_kernel(const Tensor& self) {
    if (auto r = unary("log", tp_amd_log, self)) return *r;
    return cpu_fallback::Kernel<"log", sig::log>::call(self);
}

Tensor sqrt_kernel(const Tensor& self) {
    if (auto r = unary("sqrt", tp_amd_sqrt, self)) return *r;
    return cpu_fallback::Kernel<"sqrt", sig::sqrt>::call(self);
}

Tensor rsqrt_kernel(const Tensor& self) {
    if (auto r = unary("rsqrt", tp_amd_rsqrt, self)) return *r;
    return cpu_fallback::Kernel<"rsqrt", sig::rsqrt>::call(self);
}

Tensor neg_kernel(const Tensor& self) {
    if (auto r = unary("neg", tp_amd_neg, self)) return *r;
    return cpu_fallback::Kernel<"neg", sig::neg>::call(self);
}

Tensor abs_kernel(const Tensor& self) {
    if (auto r = unary("abs", tp_amd_abs, self)) return *r;
    return cpu_fallback::Kernel<"abs", sig::abs>::call(self);
}

Tensor pow_scalar_kernel(const Tensor& self, const Scalar& exponent) {
    if (auto r = scalar_only("pow", tp_amd_pow_scalar, self, exponent)) return *r;
    return cpu_fallback::Kernel<"pow.Tensor_Scalar", sig::pow__Tensor_Scalar>::call(self,
                                                                                  exponent);
}

Tensor relu_kernel(const Tensor& self) {
    if (auto r = unary("relu", tp_amd_relu, self)) return *r;
    return cpu_fallback::Kernel<"relu", sig::relu>::call(self);
}

Tensor& relu__kernel(Tensor& self) {
    tp_amd_tensor x;
    if (view(self, &x) && in_place("relu_", [&] { return tp_amd_relu_(&x); })) return self;
    return cpu_fallback::Kernel<"relu_", sig::relu_>::call(self);
}

Tensor sigmoid_kernel(const Tensor& self) {
    if (auto r = unary("sigmoid", tp_amd_sigmoid, self)) return *r;
    return cpu_fallback::Kernel<"sigmoid", sig::sigmoid>::call(self);
}

Tensor tanh_kernel(const Tensor& self) {
    if (auto r = unary("tanh", tp_amd_tanh, self)) return *r;
    return cpu_fallback::Kernel<"tanh", sig::tanh>::call(self);
}

Tensor silu_kernel(const Tensor& self) {
    if (auto r = unary("silu", tp_amd_silu, self)) return *r;
    return cpu_fallback::Kernel<"silu", sig::silu>::call(self);
}

// gelu's ``approximate``: "none" is the erf form, "tanh" the tanh form
// (reference UnaryKernels.cpp:203-210); anything else goes to the host.
int approximate_code(const std::string& approximate) {
    if (approximate == "none") return 0;
    if (approximate == "tanh") return 1;
    return -1;
}

Tensor gelu_kernel(const Tensor& self, const std::string& approximate) {
    const int mode = approximate_code(approximate);
    tp_amd_tensor x;
    if (mode >= 0 && view(self, &x)) {
        if (auto r = produce("gelu",
                             [&](tp_amd_tensor* out) { return tp_amd_gelu(&x, mode, out); })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"gelu", sig::gelu>::call(self, approximate);
}

Tensor threshold_backward_kernel(const Tensor& grad_output, const Tensor& self,
                                 const Scalar& threshold) {
    tp_amd_tensor g, x;
    if (view(grad_output, &g) && view(self, &x)) {
        if (auto r = produce("threshold_backward", [&](tp_amd_tensor* out) {
                return tp_amd_threshold_backward(&g, &x, scalar(threshold), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"threshold_backward", sig::threshold_backward>::call(
        grad_output, self, threshold);
}

Tensor sigmoid_backward_kernel(const Tensor& grad_output, const Tensor& output) {
    if (auto r = binary("sigmoid_backward", tp_amd_sigmoid_backward, grad_output, output)) {
        return *r;
    }
    return cpu_fallback::Kernel<"sigmoid_backward", sig::sigmoid_backward>::call(grad_output,
                                                                                 output);
}

Tensor tanh_backward_kernel(const Tensor& grad_output, const Tensor& output) {
    if (auto r = binary("tanh_backward", tp_amd_tanh_backward, grad_output, output)) return *r;
    return cpu_fallback::Kernel<"tanh_backward", sig::tanh_backward>::call(grad_output, output);
}

Tensor gelu_backward_kernel(const Tensor& grad_output, const Tensor& self,
                            const std::string& approximate) {
    const int mode = approximate_code(approximate);
    tp_amd_tensor g, x;
    if (mode >= 0 && view(grad_output, &g) && view(self, &x)) {
        if (auto r = produce("gelu_backward", [&](tp_amd_tensor* out) {
                return tp_amd_gelu_backward(&g, &x, mode, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"gelu_backward", sig::gelu_backward>::call(grad_output, self,
                                                                           approximate);
}

Tensor silu_backward_kernel(const Tensor& grad_output, const Tensor& self) {
    if (auto r = binary("silu_backward", tp_amd_silu_backward, grad_output, self)) return *r;
    return cpu_fallback::Kernel<"silu_backward", sig::silu_backward>::call(grad_output, self);
}

// ---- matrix products (reference BlasKernels.cpp:261-412) -----------------

Tensor mm_kernel(const Tensor& self, const Tensor& mat2) {
    if (auto r = binary("mm", tp_amd_mm, self, mat2)) return *r;
    return cpu_fallback::Kernel<"mm", sig::mm>::call(self, mat2);
}

Tensor bmm_kernel(const Tensor& self, const Tensor& mat2) {
    if (auto r = binary("bmm", tp_amd_bmm, self, mat2)) return *r;
    return cpu_fallback::Kernel<"bmm", sig::bmm>::call(self, mat2);
}

Tensor addmm_kernel(const Tensor& self, const Tensor& mat1, const Tensor& mat2,
                    const Scalar& beta, const Scalar& alpha) {
    tp_amd_tensor c, a, b;
    if (view(self, &c) && view(mat1, &a) && view(mat2, &b)) {
        if (auto r = produce("addmm", [&](tp_amd_tensor* out) {
                return tp_amd_addmm(&c, &a, &b, scalar(beta), scalar(alpha), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"addmm", sig::addmm>::call(self, mat1, mat2, beta, alpha);
}

Tensor linear_kernel(const Tensor& input, const Tensor& weight,
                     const std::optional<Tensor>& bias_opt) {
    const bool has_bias = bias_opt.has_value() && bias_opt->defined();
    tp_amd_tensor x, w, b;
    if (view(input, &x) && view(weight, &w) && (!has_bias || view(*bias_opt, &b))) {
        if (auto r = produce("linear", [&](tp_amd_tensor* out) {
                return tp_amd_linear(&x, &w, has_bias ? &b : nullptr, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"linear", sig::linear>::call(input, weight, bias_opt);
}

Tensor matmul_kernel(const Tensor& self, const Tensor& other) {
    if (auto r = binary("matmul", tp_amd_matmul, self, other)) return *r;
    return cpu_fallback::Kernel<"matmul", sig::matmul>::call(self, other);
}

// ---- reductions and softmax (reference ReduceKernels.cpp:97-263) ---------

Tensor sum_kernel(const Tensor& self, DType dtype) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("sum", [&](tp_amd_tensor* out) {
                return tp_amd_sum(&x, dtype_arg(dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"sum", sig::sum>::call(self, dtype);
}

Tensor mean_kernel(const Tensor& self, DType dtype) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("mean", [&](tp_amd_tensor* out) {
                return tp_amd_mean(&x, dtype_arg(dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"mean", sig::mean>::call(self, dtype);
}

Tensor sum_dim_kernel(const Tensor& self, const std::vector<int64_t>& dim, bool keepdim,
                      DType dtype) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("sum.dim_IntList", [&](tp_amd_tensor* out) {
                return tp_amd_sum_dim(&x, dim.data(), static_cast<int>(dim.size()),
                                      keepdim ? 1 : 0, dtype_arg(dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"sum.dim_IntList", sig::sum__dim_IntList>::call(self, dim,
                                                                               keepdim, dtype);
}

Tensor mean_dim_kernel(const Tensor& self, const std::vector<int64_t>& dim, bool keepdim,
                       DType dtype) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("mean.dim", [&](tp_amd_tensor* out) {
                return tp_amd_mean_dim(&x, dim.data(), static_cast<int>(dim.size()),
                                       keepdim ? 1 : 0, dtype_arg(dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"mean.dim", sig::mean__dim>::call(self, dim, keepdim, dtype);
}

Tensor amax_kernel(const Tensor& self, const std::vector<int64_t>& dim, bool keepdim) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("amax", [&](tp_amd_tensor* out) {
                return tp_amd_amax(&x, dim.data(), static_cast<int>(dim.size()),
                                   keepdim ? 1 : 0, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"amax", sig::amax>::call(self, dim, keepdim);
}

Tensor amin_kernel(const Tensor& self, const std::vector<int64_t>& dim, bool keepdim) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("amin", [&](tp_amd_tensor* out) {
                return tp_amd_amin(&x, dim.data(), static_cast<int>(dim.size()),
                                   keepdim ? 1 : 0, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"amin", sig::amin>::call(self, dim, keepdim);
}

Tensor softmax_dtype(const Tensor& self, int64_t dim, DType dtype) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("softmax", [&](tp_amd_tensor* out) {
                return tp_amd_softmax(&x, dim, dtype_arg(dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"softmax", sig::softmax>::call(self, dim, dtype);
}

Tensor log_softmax_dtype(const Tensor& self, int64_t dim, DType dtype) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("log_softmax", [&](tp_amd_tensor* out) {
                return tp_amd_log_softmax(&x, dim, dtype_arg(dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"log_softmax", sig::log_softmax>::call(self, dim, dtype);
}

Tensor softmax_kernel(const Tensor& self, int64_t dim, bool half_to_float) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("_softmax", [&](tp_amd_tensor* out) {
                return tp_amd__softmax(&x, dim, half_to_float ? 1 : 0, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"_softmax", sig::_softmax>::call(self, dim, half_to_float);
}

Tensor log_softmax_kernel(const Tensor& self, int64_t dim, bool half_to_float) {
    tp_amd_tensor x;
    if (view(self, &x)) {
        if (auto r = produce("_log_softmax", [&](tp_amd_tensor* out) {
                return tp_amd__log_softmax(&x, dim, half_to_float ? 1 : 0, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"_log_softmax", sig::_log_softmax>::call(self, dim,
                                                                         half_to_float);
}

Tensor softmax_backward_kernel(const Tensor& grad_output, const Tensor& output, int64_t dim,
                               DType input_dtype) {
    tp_amd_tensor g, y;
    if (view(grad_output, &g) && view(output, &y)) {
        if (auto r = produce("_softmax_backward_data", [&](tp_amd_tensor* out) {
                return tp_amd__softmax_backward_data(&g, &y, dim, dtype_arg(input_dtype), out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"_softmax_backward_data", sig::_softmax_backward_data>::call(
        grad_output, output, dim, input_dtype);
}

Tensor log_softmax_backward_kernel(const Tensor& grad_output, const Tensor& output, int64_t dim,
                                   DType input_dtype) {
    tp_amd_tensor g, y;
    if (view(grad_output, &g) && view(output, &y)) {
        if (auto r = produce("_log_softmax_backward_data", [&](tp_amd_tensor* out) {
                return tp_amd__log_softmax_backward_data(&g, &y, dim, dtype_arg(input_dtype),
                                                         out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"_log_softmax_backward_data",
                                sig::_log_softmax_backward_data>::call(grad_output, output, dim,
                                                                       input_dtype);
}

// ---- neural-network layers (reference NNKernels.cpp:57-395) ---------------

// An optional tensor as a view pointer: nullptr when absent; false when it
// cannot be described (the host kernel runs).
bool optional_view(const std::optional<Tensor>& t, tp_amd_tensor* storage,
                   const tp_amd_tensor** out) {
    if (!t.has_value() || !t->defined()) {
        *out = nullptr;
        return true;
    }
    if (!view(*t, storage)) return false;
    *out = storage;
    return true;
}

// An entry with N result slots.
template <size_t N, typename F>
std::optional<std::array<tp_amd_tensor, N>> produce_n(const char* op, F&& call) {
    std::array<tp_amd_tensor, N> r{};
    const int status = call(r.data());
    if (status == TP_AMD_DECLINED) return std::nullopt;
    if (status != TP_AMD_OK) raise(op);
    return r;
}

// A slot the entry left undefined (an output masked off) is an undefined
// tensor.
Tensor adopt_optional(const tp_amd_tensor& r) {
    return r.data == nullptr && r.dtype == TP_AMD_UNDEFINED ? Tensor() : adopt(r);
}

std::tuple<Tensor, Tensor, Tensor> native_layer_norm_kernel(
    const Tensor& input, const std::vector<int64_t>& normalized_shape,
    const std::optional<Tensor>& weight, const std::optional<Tensor>& bias, double eps) {
    tp_amd_tensor x, ws, bs;
    const tp_amd_tensor *w = nullptr, *b = nullptr;
    if (view(input, &x) && optional_view(weight, &ws, &w) && optional_view(bias, &bs, &b)) {
        auto r = produce_n<3>("native_layer_norm", [&](tp_amd_tensor* out) {
            return tp_amd_native_layer_norm(&x, normalized_shape.data(),
                                            static_cast<int>(normalized_shape.size()), w, b, eps,
                                            &out[0], &out[1], &out[2]);
        });
        if (r) return {adopt((*r)[0]), adopt((*r)[1]), adopt((*r)[2])};
    }
    return cpu_fallback::Kernel<"native_layer_norm", sig::native_layer_norm>::call(
        input, normalized_shape, weight, bias, eps);
}

std::tuple<Tensor, Tensor, Tensor> native_layer_norm_backward_kernel(
    const Tensor& grad_out, const Tensor& input, const std::vector<int64_t>& normalized_shape,
    const Tensor& mean, const Tensor& rstd, const std::optional<Tensor>& weight,
    const std::optional<Tensor>& bias, const std::vector<bool>& output_mask) {
    tp_amd_tensor g, x, m, r, ws, bs;
    const tp_amd_tensor *w = nullptr, *b = nullptr;
    int mask[3] = {1, 1, 1};
    for (size_t i = 0; i < 3 && i < output_mask.size(); ++i) mask[i] = output_mask[i] ? 1 : 0;
    if (view(grad_out, &g) && view(input, &x) && view(mean, &m) && view(rstd, &r) &&
        optional_view(weight, &ws, &w) && optional_view(bias, &bs, &b)) {
        auto res = produce_n<3>("native_layer_norm_backward", [&](tp_amd_tensor* out) {
            return tp_amd_native_layer_norm_backward(
                &g, &x, normalized_shape.data(), static_cast<int>(normalized_shape.size()), &m, &r,
                w, b, mask, &out[0], &out[1], &out[2]);
        });
        if (res) {
            return {adopt_optional((*res)[0]), adopt_optional((*res)[1]),
                    adopt_optional((*res)[2])};
        }
    }
    return cpu_fallback::Kernel<"native_layer_norm_backward", sig::native_layer_norm_backward>::
        call(grad_out, input, normalized_shape, mean, rstd, weight, bias, output_mask);
}

std::tuple<Tensor, Tensor> native_dropout_kernel(const Tensor& input, double p,
                                                 std::optional<bool> train) {
    tp_amd_tensor x;
    if (view(input, &x)) {
        const int t = train.has_value() ? (*train ? 1 : 0) : -1;
        // One 64-bit draw from TensorPlay's host generator keys the Philox
        // stream, so a manual seed repeats the mask.
        const uint64_t seed = default_generator().random64();
        auto r = produce_n<2>("native_dropout", [&](tp_amd_tensor* out) {
            return tp_amd_native_dropout(&x, p, t, seed, &out[0], &out[1]);
        });
        if (r) return {adopt((*r)[0]), adopt((*r)[1])};
    }
    return cpu_fallback::Kernel<"native_dropout", sig::native_dropout>::call(input, p, train);
}

Tensor native_dropout_backward_kernel(const Tensor& grad_output, const Tensor& mask,
                                      double scale) {
    tp_amd_tensor g, m;
    if (view(grad_output, &g) && view(mask, &m)) {
        if (auto r = produce("native_dropout_backward", [&](tp_amd_tensor* out) {
                return tp_amd_native_dropout_backward(&g, &m, scale, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"native_dropout_backward", sig::native_dropout_backward>::call(
        grad_output, mask, scale);
}

Tensor embedding_kernel(const Tensor& weight, const Tensor& indices, int64_t padding_idx,
                        bool scale_grad_by_freq, bool sparse) {
    tp_amd_tensor w, i;
    if (view(weight, &w) && view(indices, &i)) {
        if (auto r = produce("embedding", [&](tp_amd_tensor* out) {
                return tp_amd_embedding(&w, &i, padding_idx, scale_grad_by_freq ? 1 : 0,
                                        sparse ? 1 : 0, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"embedding", sig::embedding>::call(weight, indices, padding_idx,
                                                                   scale_grad_by_freq, sparse);
}

Tensor embedding_dense_backward_kernel(const Tensor& grad_output, const Tensor& indices,
                                       int64_t num_weights, int64_t padding_idx,
                                       bool scale_grad_by_freq) {
    tp_amd_tensor g, i;
    if (view(grad_output, &g) && view(indices, &i)) {
        if (auto r = produce("embedding_dense_backward", [&](tp_amd_tensor* out) {
                return tp_amd_embedding_dense_backward(&g, &i, num_weights, padding_idx,
                                                       scale_grad_by_freq ? 1 : 0, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"embedding_dense_backward", sig::embedding_dense_backward>::call(
        grad_output, indices, num_weights, padding_idx, scale_grad_by_freq);
}

std::tuple<Tensor, Tensor> nll_loss_kernel(const Tensor& self, const Tensor& target,
                                           const std::optional<Tensor>& weight, int64_t reduction,
                                           int64_t ignore_index) {
    tp_amd_tensor x, t, ws;
    const tp_amd_tensor* w = nullptr;
    if (view(self, &x) && view(target, &t) && optional_view(weight, &ws, &w)) {
        auto r = produce_n<2>("nll_loss", [&](tp_amd_tensor* out) {
            return tp_amd_nll_loss(&x, &t, w, reduction, ignore_index, &out[0], &out[1]);
        });
        if (r) return {adopt((*r)[0]), adopt((*r)[1])};
    }
    return cpu_fallback::Kernel<"nll_loss", sig::nll_loss>::call(self, target, weight, reduction,
                                                                 ignore_index);
}

Tensor nll_loss_backward_kernel(const Tensor& grad_output, const Tensor& self,
                                const Tensor& target, const std::optional<Tensor>& weight,
                                int64_t reduction, int64_t ignore_index,
                                const Tensor& total_weight) {
    tp_amd_tensor g, x, t, ws, tw;
    const tp_amd_tensor* w = nullptr;
    if (view(grad_output, &g) && view(self, &x) && view(target, &t) &&
        optional_view(weight, &ws, &w) && view(total_weight, &tw)) {
        if (auto r = produce("nll_loss_backward", [&](tp_amd_tensor* out) {
                return tp_amd_nll_loss_backward(&g, &x, &t, w, reduction, ignore_index, &tw, out);
            })) {
            return *r;
        }
    }
    return cpu_fallback::Kernel<"nll_loss_backward", sig::nll_loss_backward>::call(
        grad_output, self, target, weight, reduction, ignore_index, total_weight);
}

}  // namespace

}  // namespace amd

using namespace amd;
namespace sig = kernel_signatures;

TENSORPLAY_LIBRARY_IMPL(PrivateUse1, AmdCopyKernels) {
    m.impl("empty_like", static_cast<sig::empty_like*>(&empty_like_kernel));
    m.impl("zeros_like", static_cast<sig::zeros_like*>(&zeros_like_kernel));
    m.impl("ones_like", static_cast<sig::ones_like*>(&ones_like_kernel));
    m.impl("full_like", static_cast<sig::full_like*>(&full_like_kernel));
    m.impl("item", static_cast<sig::item*>(&item_kernel));
    m.impl("_local_scalar_dense", static_cast<sig::_local_scalar_dense*>(&item_kernel));
    m.impl("empty", static_cast<sig::empty*>(&empty_kernel));
    m.impl("empty.memory_format",
           static_cast<sig::empty__memory_format*>(&empty_memory_format_kernel));
    m.impl("copy_", static_cast<sig::copy_*>(&copy_kernel));
    m.impl("fill_.Scalar", static_cast<sig::fill___Scalar*>(&fill_kernel));
    m.impl("zero_", static_cast<sig::zero_*>(&zero_kernel));
    m.impl("clone", static_cast<sig::clone*>(&clone_kernel));
    m.impl("contiguous", static_cast<sig::contiguous*>(&contiguous_kernel));
}

TENSORPLAY_LIBRARY_IMPL(PrivateUse1, AmdBinaryKernels) {
    m.impl("add.Tensor", static_cast<sig::add__Tensor*>(&add_kernel));
    m.impl("sub.Tensor", static_cast<sig::sub__Tensor*>(&sub_kernel));
    m.impl("mul.Tensor", static_cast<sig::mul__Tensor*>(&mul_kernel));
    m.impl("div.Tensor", static_cast<sig::div__Tensor*>(&div_kernel));
    m.impl("add_.Tensor", static_cast<sig::add___Tensor*>(&add__kernel));
    m.impl("sub_.Tensor", static_cast<sig::sub___Tensor*>(&sub__kernel));
    m.impl("mul_.Tensor", static_cast<sig::mul___Tensor*>(&mul__kernel));
    m.impl("div_.Tensor", static_cast<sig::div___Tensor*>(&div__kernel));
    m.impl("add.Scalar", static_cast<sig::add__Scalar*>(&add_scalar_kernel));
    m.impl("sub.Scalar", static_cast<sig::sub__Scalar*>(&sub_scalar_kernel));
    m.impl("rsub.Scalar", static_cast<sig::rsub__Scalar*>(&rsub_scalar_kernel));
    m.impl("mul.Scalar", static_cast<sig::mul__Scalar*>(&mul_scalar_kernel));
    m.impl("div.Scalar", static_cast<sig::div__Scalar*>(&div_scalar_kernel));
    m.impl("add_.Scalar", static_cast<sig::add___Scalar*>(&add__scalar_kernel));
    m.impl("mul_.Scalar", static_cast<sig::mul___Scalar*>(&mul__scalar_kernel));
    m.impl("div_.Scalar", static_cast<sig::div___Scalar*>(&div__scalar_kernel));
}

TENSORPLAY_LIBRARY_IMPL(PrivateUse1, AmdUnaryKernels) {
    m.impl("exp", static_cast<sig::exp*>(&exp_kernel));
    m.impl("log", static_cast<sig::log*>(&log_kernel));
    m.impl("sqrt", static_cast<sig::sqrt*>(&sqrt_kernel));
    m.impl("rsqrt", static_cast<sig::rsqrt*>(&rsqrt_kernel));
    m.impl("neg", static_cast<sig::neg*>(&neg_kernel));
    m.impl("abs", static_cast<sig::abs*>(&abs_kernel));
    m.impl("pow.Tensor_Scalar", static_cast<sig::pow__Tensor_Scalar*>(&pow_scalar_kernel));
    m.impl("relu", static_cast<sig::relu*>(&relu_kernel));
    m.impl("relu_", static_cast<sig::relu_*>(&relu__kernel));
    m.impl("sigmoid", static_cast<sig::sigmoid*>(&sigmoid_kernel));
    m.impl("tanh", static_cast<sig::tanh*>(&tanh_kernel));
    m.impl("silu", static_cast<sig::silu*>(&silu_kernel));
    m.impl("gelu", static_cast<sig::gelu*>(&gelu_kernel));
    m.impl("threshold_backward",
           static_cast<sig::threshold_backward*>(&threshold_backward_kernel));
    m.impl("sigmoid_backward", static_cast<sig::sigmoid_backward*>(&sigmoid_backward_kernel));
    m.impl("tanh_backward", static_cast<sig::tanh_backward*>(&tanh_backward_kernel));
    m.impl("gelu_backward", static_cast<sig::gelu_backward*>(&gelu_backward_kernel));
    m.impl("silu_backward", static_cast<sig::silu_backward*>(&silu_backward_kernel));
}

TENSORPLAY_LIBRARY_IMPL(PrivateUse1, AmdBlasKernels) {
    m.impl("mm", static_cast<sig::mm*>(&mm_kernel));
    m.impl("bmm", static_cast<sig::bmm*>(&bmm_kernel));
    m.impl("addmm", static_cast<sig::addmm*>(&addmm_kernel));
    m.impl("matmul", static_cast<sig::matmul*>(&matmul_kernel));
    m.impl("linear", static_cast<sig::linear*>(&linear_kernel));
}

TENSORPLAY_LIBRARY_IMPL(PrivateUse1, AmdReduceKernels) {
    m.impl("sum", static_cast<sig::sum*>(&sum_kernel));
    m.impl("sum.dim_IntList", static_cast<sig::sum__dim_IntList*>(&sum_dim_kernel));
    m.impl("amax", static_cast<sig::amax*>(&amax_kernel));
    m.impl("amin", static_cast<sig::amin*>(&amin_kernel));
    m.impl("mean", static_cast<sig::mean*>(&mean_kernel));
    m.impl("mean.dim", static_cast<sig::mean__dim*>(&mean_dim_kernel));
    m.impl("softmax", static_cast<sig::softmax*>(&softmax_dtype));
    m.impl("log_softmax", static_cast<sig::log_softmax*>(&log_softmax_dtype));
    m.impl("_softmax", static_cast<sig::_softmax*>(&softmax_kernel));
    m.impl("_log_softmax", static_cast<sig::_log_softmax*>(&log_softmax_kernel));
    m.impl("_softmax_backward_data",
           static_cast<sig::_softmax_backward_data*>(&softmax_backward_kernel));
    m.impl("_log_softmax_backward_data",
           static_cast<sig::_log_softmax_backward_data*>(&log_softmax_backward_kernel));
}

TENSORPLAY_LIBRARY_IMPL(PrivateUse1, AmdNNKernels) {
    m.impl("native_layer_norm", static_cast<sig::native_layer_norm*>(&native_layer_norm_kernel));
    m.impl("native_layer_norm_backward",
           static_cast<sig::native_layer_norm_backward*>(&native_layer_norm_backward_kernel));
    m.impl("native_dropout", static_cast<sig::native_dropout*>(&native_dropout_kernel));
    m.impl("native_dropout_backward",
           static_cast<sig::native_dropout_backward*>(&native_dropout_backward_kernel));
    m.impl("embedding", static_cast<sig::embedding*>(&embedding_kernel));
    m.impl("embedding_dense_backward",
           static_cast<sig::embedding_dense_backward*>(&embedding_dense_backward_kernel));
    m.impl("nll_loss", static_cast<sig::nll_loss*>(&nll_loss_kernel));
    m.impl("nll_loss_backward", static_cast<sig::nll_loss_backward*>(&nll_loss_backward_kernel));
}

}  // namespace tensorplay
