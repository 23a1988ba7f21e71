// Tensor views for the host-side operator layer: shape queries, ownership of
// library-allocated results, and the helpers every operator is built on
// (the reference's Cnnl.h helpers: empty_on, contiguous_on_device,
// strided_copy, to_dtype, binary_result_dtype, broadcast_shape, is_dense,
// tensorplay_mlu/csrc/Cnnl.h:59-95, Cnnl.cpp:99-222).
#pragma once

#include <cstdint>
#include <vector>

#include "../allocator.h"
#include "../common.h"
#include "tp_amd_types.h"

namespace tp_amd {

using TensorRef = tp_amd_tensor;
using Sizes = std::vector<int64_t>;

int64_t numel(const TensorRef& t);
Sizes sizes_of(const TensorRef& t);
Sizes strides_of(const TensorRef& t);
bool is_contiguous(const TensorRef& t);
bool is_dense(const TensorRef& t);
inline bool on_device(const TensorRef& t) { return t.device >= 0; }
inline bool is_host_scalar(const TensorRef& t) { return t.device < 0 && t.ndim == 0; }
void check_view(const TensorRef& t, const char* what);

// ``*p`` after a null check (the entry points take pointers).
inline const TensorRef& deref(const tp_amd_tensor* p, const char* what) {
    TP_AMD_CHECK(p != nullptr, what, ": null tensor pointer");
    return *p;
}

// A view of ``base``'s memory with new sizes and strides (no ownership).
TensorRef make_view(const TensorRef& base, const Sizes& sizes, const Sizes& strides,
                    int64_t element_offset = 0);
Sizes contiguous_strides(const Sizes& sizes);

// A library-allocated tensor, freed on destruction unless released to a
// caller (the reference's Storage/DataPtr ownership, MLUAllocator.cpp:63-73).
class Owned {
public:
    Owned() { t_ = TensorRef{}; t_.device = -1; }
    explicit Owned(const TensorRef& t) : t_(t) {}
    ~Owned() { reset(); }
    Owned(Owned&& o) noexcept : t_(o.t_) { o.t_.ctx = nullptr; }
    Owned& operator=(Owned&& o) noexcept {
        if (this != &o) {
            reset();
            t_ = o.t_;
            o.t_.ctx = nullptr;
        }
        return *this;
    }
    Owned(const Owned&) = delete;
    Owned& operator=(const Owned&) = delete;

    const TensorRef& ref() const { return t_; }
    TensorRef& ref() { return t_; }
    TensorRef release() {
        TensorRef t = t_;
        t_.ctx = nullptr;
        return t;
    }

private:
    void reset() {
        if (t_.ctx != nullptr) device_free(static_cast<Block*>(t_.ctx));
        t_.ctx = nullptr;
    }
    TensorRef t_;
};

// A tensor that is either an existing view or a new allocation.
struct MaybeOwned {
    TensorRef ref;
    Owned hold;
};

// Dense row-major tensor on ``device`` (empty_on, Cnnl.cpp:99-105).
Owned empty_on(const Sizes& sizes, int dtype, int device);

// dst = src element for element: same dtype and shape, either strided
// (strided_copy, Cnnl.cpp:154-176).
void strided_copy(const TensorRef& dst, const TensorRef& src);

// ``t`` itself when contiguous, else a contiguous copy
// (contiguous_on_device, Cnnl.cpp:217-222).
MaybeOwned contiguous_on_device(const TensorRef& t);

// ``t`` converted to ``dtype`` on its device; ``t`` itself when it already
// has that dtype (to_dtype, CopyKernels.cpp:222-227).
MaybeOwned to_dtype(const TensorRef& t, int dtype);

// ``t`` broadcast to ``sizes`` (stride 0 on expanded dimensions).
TensorRef expand_to(const TensorRef& t, const Sizes& sizes);

// Dtype rules (Cnnl.cpp:178-192) and broadcasting (Cnnl.cpp:194-205).
int promote_types(int a, int b);
int binary_result_dtype(int a_dtype, int a_ndim, int b_dtype, int b_ndim);
Sizes broadcast_shape(const Sizes& a, const Sizes& b);

// Value of a 0-d host tensor as a double (BinaryKernels.cpp:115 item()).
double host_scalar_value(const TensorRef& t);

// A float rounded to ``dtype``'s precision and back (what the reference's
// Half(float) / BFloat16(float) encodings hold, UnaryKernels.cpp:229-236).
float round_to_dtype(float v, int dtype);
uint16_t host_float_to_bf16(float f);
uint16_t host_float_to_f16(float f);
float host_bf16_to_float(uint16_t b);
float host_f16_to_float(uint16_t h);

// Fill ``self`` with ``value`` encoded per dtype (fill_kernel,
// CopyKernels.cpp:266-299).
void fill(const TensorRef& self, const tp_amd_scalar& value);

// Conversion between dense tensors of one shape (cast_into,
// CopyKernels.cpp:125-139), routed as the reference routes it.
void cast_dense(const TensorRef& dst, const TensorRef& src);

// Copy between any two views (copy_kernel, CopyKernels.cpp:248-264).
void copy_into(const TensorRef& self, const TensorRef& src);

inline tp_amd_scalar scalar_of(double v) {
    tp_amd_scalar s{};
    s.f = v;
    s.i = static_cast<int64_t>(v);
    s.kind = TP_AMD_SCALAR_FLOAT;
    return s;
}

// Run ``body`` with a result slot: on success the owned result moves to
// ``*result`` (ownership to the caller).
template <typename Body>
int guarded_result(tp_amd_tensor* result, Body&& body) noexcept {
    return guarded([&] {
        TP_AMD_CHECK(result != nullptr, "null result pointer");
        Owned out = body();
        *result = out.release();
    });
}

}  // namespace tp_amd
