// Signature types of the operators the adapter registers, written from the
// reference kernel definitions (tensorplay_mlu/csrc/*Kernels.cpp).
#pragma once
#include <tuple>
#include <optional>
#include <string>
#include <vector>

#include "../../api.h"

namespace tensorplay {
namespace kernel_signatures {
using IntList = std::vector<int64_t>;
using empty = Tensor(const IntList&, std::optional<DType>, std::optional<Device>, bool);
using empty__memory_format = Tensor(const IntList&, std::optional<DType>, std::optional<int64_t>,
                                    std::optional<Device>, std::optional<bool>,
                                    std::optional<int64_t>);
using empty_like = Tensor(const Tensor&, DType, std::optional<Device>);
using zeros_like = empty_like;
using ones_like = empty_like;
using full_like = Tensor(const Tensor&, const Scalar&, DType, std::optional<Device>);
using item = Scalar(const Tensor&);
using _local_scalar_dense = item;
using copy_ = Tensor&(Tensor&, const Tensor&, bool);
using fill___Scalar = Tensor&(Tensor&, const Scalar&);
using zero_ = Tensor&(Tensor&);
using clone = Tensor(const Tensor&, std::optional<int64_t>);
using contiguous = Tensor(const Tensor&, int64_t);

using add__Tensor = Tensor(const Tensor&, const Tensor&, const Scalar&);
using sub__Tensor = add__Tensor;
using mul__Tensor = Tensor(const Tensor&, const Tensor&);
using div__Tensor = mul__Tensor;
using add___Tensor = Tensor&(Tensor&, const Tensor&, const Scalar&);
using sub___Tensor = add___Tensor;
using mul___Tensor = Tensor&(Tensor&, const Tensor&);
using div___Tensor = mul___Tensor;
using add__Scalar = Tensor(const Tensor&, const Scalar&, const Scalar&);
using sub__Scalar = add__Scalar;
using rsub__Scalar = add__Scalar;
using mul__Scalar = Tensor(const Tensor&, const Scalar&);
using div__Scalar = mul__Scalar;
using add___Scalar = Tensor&(Tensor&, const Scalar&, const Scalar&);
using mul___Scalar = Tensor&(Tensor&, const Scalar&);
using div___Scalar = mul___Scalar;

using exp = Tensor(const Tensor&);
using log = exp;
using sqrt = exp;
using rsqrt = exp;
using neg = exp;
using abs = exp;
using relu = exp;
using sigmoid = exp;
using tanh = exp;
using silu = exp;
using relu_ = Tensor&(Tensor&);
using pow__Tensor_Scalar = Tensor(const Tensor&, const Scalar&);
using gelu = Tensor(const Tensor&, const std::string&);
using threshold_backward = Tensor(const Tensor&, const Tensor&, const Scalar&);
using sigmoid_backward = Tensor(const Tensor&, const Tensor&);
using tanh_backward = sigmoid_backward;
using silu_backward = sigmoid_backward;
using gelu_backward = Tensor(const Tensor&, const Tensor&, const std::string&);

using mm = Tensor(const Tensor&, const Tensor&);
using bmm = mm;
using matmul = mm;
using addmm = Tensor(const Tensor&, const Tensor&, const Tensor&, const Scalar&, const Scalar&);
using linear = Tensor(const Tensor&, const Tensor&, const std::optional<Tensor>&);

using sum = Tensor(const Tensor&, DType);
using mean = sum;
using sum__dim_IntList = Tensor(const Tensor&, const IntList&, bool, DType);
using mean__dim = sum__dim_IntList;
using amax = Tensor(const Tensor&, const IntList&, bool);
using amin = amax;
using softmax = Tensor(const Tensor&, int64_t, DType);
using log_softmax = softmax;
using _softmax = Tensor(const Tensor&, int64_t, bool);
using _log_softmax = _softmax;
using _softmax_backward_data = Tensor(const Tensor&, const Tensor&, int64_t, DType);
using _log_softmax_backward_data = _softmax_backward_data;

using native_layer_norm = std::tuple<Tensor, Tensor, Tensor>(const Tensor&, const IntList&,
                                                             const std::optional<Tensor>&,
                                                             const std::optional<Tensor>&, double);
using native_layer_norm_backward = std::tuple<Tensor, Tensor, Tensor>(
    const Tensor&, const Tensor&, const IntList&, const Tensor&, const Tensor&,
    const std::optional<Tensor>&, const std::optional<Tensor>&, const std::vector<bool>&);
using native_dropout = std::tuple<Tensor, Tensor>(const Tensor&, double, std::optional<bool>);
using native_dropout_backward = Tensor(const Tensor&, const Tensor&, double);
using embedding = Tensor(const Tensor&, const Tensor&, int64_t, bool, bool);
using embedding_dense_backward = Tensor(const Tensor&, const Tensor&, int64_t, int64_t, bool);
using nll_loss = std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&,
                                            const std::optional<Tensor>&, int64_t, int64_t);
using nll_loss_backward = Tensor(const Tensor&, const Tensor&, const Tensor&,
                                 const std::optional<Tensor>&, int64_t, int64_t, const Tensor&);
}  // namespace kernel_signatures
}  // namespace tensorplay
