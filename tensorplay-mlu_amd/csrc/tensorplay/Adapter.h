// TensorPlay side of the backend: turns TensorPlay tensors and scalars into
// the plain views of the operator C-ABI (tp_amd_ops.h) and wraps its results
// back into TensorPlay tensors.
//
// Built only against TensorPlay's C++ headers (make TENSORPLAY_INCLUDE=...),
// into the same libtp_amd.so.  It fills the slots the reference fills
// (tensorplay_mlu/csrc/*Kernels.cpp registrations, MLUAllocator.cpp:239-240,
// MLUHooks.cpp:14-56, Module.cpp:15-22) with the HIP backend.

#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "Allocator.h"
#include "CpuFallback.h"
#include "Device.h"
#include "Dispatcher.h"
#include "Exception.h"
#include "Tensor.h"
#include "tensorplay/ops/KernelSignatures.h"

#include "tp_amd_ops.h"
#include "tp_amd_runtime.h"

namespace tensorplay {
namespace amd {

// TensorPlay dtype <-> C-ABI dtype code; TP_AMD_UNDEFINED for dtypes the
// backend does not store (complex, unsigned wider than 8 bits).
int dtype_code(DType dtype);
DType dtype_of(int code);

// Device index of a PrivateUse1 device (-1 resolves to the current one).
int index_of(const Device& device);

// A non-owning view of ``t``.  Host tensors get device -1.  Returns false when
// the tensor cannot be described (more than TP_AMD_MAX_DIMS dimensions or a
// dtype the backend does not store): the caller then runs the host kernel.
bool view(const Tensor& t, tp_amd_tensor* out);

tp_amd_scalar scalar(const Scalar& s);
Scalar to_scalar(const tp_amd_scalar& s);

// Wraps a result the C-ABI allocated: the storage's DataPtr carries the
// allocator block and tp_amd_free as its deleter.
Tensor adopt(const tp_amd_tensor& result);

// The PrivateUse1 allocator (tp_amd_malloc / tp_amd_free).
Allocator* allocator();

// Throws TensorPlay's error for a TP_AMD_ERROR status.
[[noreturn]] void raise(const char* op);

// Outcome of one C-ABI call: a value, or "declined" (run the host kernel).
template <typename T>
using Native = std::optional<T>;

// Calls an entry that writes a new tensor into its last argument.
template <typename F>
Native<Tensor> produce(const char* op, F&& call) {
    tp_amd_tensor result{};
    const int status = call(&result);
    if (status == TP_AMD_DECLINED) return std::nullopt;
    if (status != TP_AMD_OK) raise(op);
    return adopt(result);
}

// Calls an entry that works in place; true on success, false when declined.
template <typename F>
bool in_place(const char* op, F&& call) {
    const int status = call();
    if (status == TP_AMD_DECLINED) return false;
    if (status != TP_AMD_OK) raise(op);
    return true;
}

}  // namespace amd
}  // namespace tensorplay
