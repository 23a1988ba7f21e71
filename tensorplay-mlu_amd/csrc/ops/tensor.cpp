// Shape, dtype and copy helpers of the operator layer (restating
// tensorplay_mlu/csrc/Cnnl.cpp:99-222 and CopyKernels.cpp:42-264 over plain
// tensor views).

#include "tensor.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <numeric>
#include <set>
#include <utility>

#include "../runtime.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

namespace tp_amd {

int64_t numel(const TensorRef& t) {
    int64_t n = 1;
    for (int d = 0; d < t.ndim; ++d) n *= t.sizes[d];
    return n;
}

Sizes sizes_of(const TensorRef& t) { return Sizes(t.sizes, t.sizes + t.ndim); }
Sizes strides_of(const TensorRef& t) { return Sizes(t.strides, t.strides + t.ndim); }

void check_view(const TensorRef& t, const char* what) {
    TP_AMD_CHECK(t.ndim >= 0 && t.ndim <= TP_AMD_MAX_DIMS, what, ": ", t.ndim,
                 " dimensions (at most ", TP_AMD_MAX_DIMS, ")");
    TP_AMD_CHECK(element_size(t.dtype) > 0, what, ": unknown dtype code ", t.dtype);
    for (int d = 0; d < t.ndim; ++d) TP_AMD_CHECK(t.sizes[d] >= 0, what, ": negative size");
    TP_AMD_CHECK(t.data != nullptr || numel(t) == 0, what, ": null data");
}

bool is_contiguous(const TensorRef& t) {
    int64_t expected = 1;
    for (int d = t.ndim - 1; d >= 0; --d) {
        if (t.sizes[d] == 1) continue;
        if (t.strides[d] != expected) return false;
        expected *= t.sizes[d];
    }
    return true;
}

// Dense: the elements fill one gap-free block of memory in some axis order.
// Sorting the non-unit axes by stride, each stride must equal the number of
// elements the smaller-stride axes span.
bool is_dense(const TensorRef& t) {
    std::vector<std::pair<int64_t, int64_t>> axes;  // (stride, size) of the non-unit axes
    for (int d = 0; d < t.ndim; ++d) {
        if (t.sizes[d] != 1) axes.emplace_back(t.strides[d], t.sizes[d]);
    }
    std::sort(axes.begin(), axes.end());
    int64_t span = 1;
    for (const auto& [stride, size] : axes) {
        if (stride != span) return false;
        span *= size;
    }
    return true;
}

Sizes contiguous_strides(const Sizes& sizes) {
    Sizes strides(sizes.size(), 1);
    for (int64_t i = static_cast<int64_t>(sizes.size()) - 2; i >= 0; --i) {
        strides[i] = strides[i + 1] * std::max<int64_t>(sizes[i + 1], 1);
    }
    return strides;
}

TensorRef make_view(const TensorRef& base, const Sizes& sizes, const Sizes& strides,
                    int64_t element_offset) {
    TP_AMD_CHECK(sizes.size() <= TP_AMD_MAX_DIMS && sizes.size() == strides.size(),
                 "view of ", sizes.size(), " dimensions");
    TensorRef v = base;
    v.ctx = nullptr;
    v.ndim = static_cast<int32_t>(sizes.size());
    for (int d = 0; d < TP_AMD_MAX_DIMS; ++d) {
        v.sizes[d] = d < v.ndim ? sizes[d] : 0;
        v.strides[d] = d < v.ndim ? strides[d] : 0;
    }
    v.data = static_cast<char*>(base.data) + element_offset * element_size(base.dtype);
    return v;
}

Owned empty_on(const Sizes& sizes, int dtype, int device) {
    TP_AMD_CHECK(sizes.size() <= TP_AMD_MAX_DIMS, "at most ", TP_AMD_MAX_DIMS, " dimensions");
    TP_AMD_CHECK(element_size(dtype) > 0, "unknown dtype code ", dtype);
    int64_t n = 1;
    for (int64_t d : sizes) {
        TP_AMD_CHECK(d >= 0, "negative dimension ", d, " in a requested size");
        n *= d;
    }
    TensorRef t{};
    t.ndim = static_cast<int32_t>(sizes.size());
    t.dtype = dtype;
    t.device = resolve_device(device);
    const Sizes strides = contiguous_strides(sizes);
    for (size_t d = 0; d < sizes.size(); ++d) {
        t.sizes[d] = sizes[d];
        t.strides[d] = strides[d];
    }
    if (n > 0) {
        Block* block = device_alloc(static_cast<size_t>(n) * element_size(dtype), t.device);
        t.data = block->ptr;
        t.ctx = block;
    }
    return Owned(t);
}

void strided_copy(const TensorRef& dst, const TensorRef& src) {
    TP_AMD_CHECK(dst.dtype == src.dtype, "strided_copy: dtype mismatch");
    TP_AMD_CHECK(sizes_of(dst) == sizes_of(src), "strided_copy: shape mismatch");
    if (numel(dst) == 0) return;
    TP_AMD_CHECK(dst.device == src.device && dst.device >= 0, "strided_copy: device mismatch");
    const int st = tp_amd_launch_strided_copy(dst.device, element_size(dst.dtype), dst.ndim,
                                              dst.sizes, dst.data, dst.strides, src.data,
                                              src.strides);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
}

MaybeOwned contiguous_on_device(const TensorRef& t) {
    MaybeOwned m;
    if (is_contiguous(t)) {
        m.ref = t;
        m.ref.ctx = nullptr;
        return m;
    }
    m.hold = empty_on(sizes_of(t), t.dtype, t.device);
    strided_copy(m.hold.ref(), t);
    m.ref = m.hold.ref();
    return m;
}

TensorRef expand_to(const TensorRef& t, const Sizes& sizes) {
    const int nd = static_cast<int>(sizes.size());
    TP_AMD_CHECK(nd >= t.ndim, "cannot expand ", t.ndim, "-d to ", nd, "-d");
    Sizes strides(nd, 0);
    for (int i = 0; i < nd; ++i) {
        const int src = i - (nd - t.ndim);
        if (src < 0) continue;
        if (t.sizes[src] == sizes[i]) {
            strides[i] = t.strides[src];
        } else {
            TP_AMD_CHECK(t.sizes[src] == 1, "expand: size ", t.sizes[src], " cannot become ",
                         sizes[i]);
            strides[i] = 0;
        }
    }
    return make_view(t, sizes, strides);
}

// ---- dtype rules -----------------------------------------------------------

namespace {

int category(int dtype) {  // 0 bool, 1 integer, 2 floating
    if (dtype == TP_AMD_BOOL) return 0;
    return is_floating(dtype) ? 2 : 1;
}

}  // namespace

// The usual promotion lattice: a wider category wins; within floats,
// float16 with bfloat16 gives float32 and anything with float64 gives
// float64; within integers the wider type wins and uint8 with a signed type
// goes to the next signed width that holds both.
int promote_types(int a, int b) {
    if (a == b) return a;
    const int ca = category(a), cb = category(b);
    if (ca != cb) return ca > cb ? a : b;
    if (ca == 2) {
        if (a == TP_AMD_FLOAT64 || b == TP_AMD_FLOAT64) return TP_AMD_FLOAT64;
        if (a == TP_AMD_FLOAT32 || b == TP_AMD_FLOAT32) return TP_AMD_FLOAT32;
        return TP_AMD_FLOAT32;  // float16 with bfloat16
    }
    auto width = [](int d) { return element_size(d); };
    if (a == TP_AMD_UINT8 || b == TP_AMD_UINT8) {
        const int other = a == TP_AMD_UINT8 ? b : a;
        if (other == TP_AMD_INT8) return TP_AMD_INT16;
        return other;
    }
    return width(a) >= width(b) ? a : b;
}

// A 0-d operand does not widen a dimensioned one whose category (bool <
// integer < floating) is at least its own: float16 tensor + float64 0-d stays
// float16, int32 tensor + int64 0-d stays int32, float tensor + int 0-d stays
// float.  Otherwise (two dimensioned operands, two 0-d ones, or a 0-d one
// of a higher category) the lattice above decides.
int binary_result_dtype(int a_dtype, int a_ndim, int b_dtype, int b_ndim) {
    if (a_dtype == b_dtype) return a_dtype;
    if ((a_ndim == 0) != (b_ndim == 0)) {
        const int tensor = a_ndim == 0 ? b_dtype : a_dtype;
        const int zero_d = a_ndim == 0 ? a_dtype : b_dtype;
        if (category(tensor) >= category(zero_d)) return tensor;
    }
    return promote_types(a_dtype, b_dtype);
}

// Sizes aligned at the last axis; each pair must agree or one of them be 1,
// and a missing leading axis counts as 1.
Sizes broadcast_shape(const Sizes& a, const Sizes& b) {
    Sizes out(std::max(a.size(), b.size()));
    auto ia = a.rbegin(), ib = b.rbegin();
    for (auto o = out.rbegin(); o != out.rend(); ++o) {
        const int64_t x = ia != a.rend() ? *ia++ : 1;
        const int64_t y = ib != b.rend() ? *ib++ : 1;
        TP_AMD_CHECK(x == y || x == 1 || y == 1, "broadcast: sizes ", x, " and ", y,
                     " in one axis are unequal and neither is 1");
        *o = x == 1 ? y : x;
    }
    return out;
}

// ---- host-side element encodings ---------------------------------------------

uint16_t host_float_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

float host_bf16_to_float(uint16_t b) {
    const uint32_t u = static_cast<uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t host_float_to_f16(float f) {
    const _Float16 h = static_cast<_Float16>(f);  // round to nearest even
    uint16_t bits;
    std::memcpy(&bits, &h, 2);
    return bits;
}

float host_f16_to_float(uint16_t bits) {
    _Float16 h;
    std::memcpy(&h, &bits, 2);
    return static_cast<float>(h);
}

float round_to_dtype(float v, int dtype) {
    if (dtype == TP_AMD_BFLOAT16) return host_bf16_to_float(host_float_to_bf16(v));
    if (dtype == TP_AMD_FLOAT16) return host_f16_to_float(host_float_to_f16(v));
    return v;
}

double host_scalar_value(const TensorRef& t) {
    const void* p = t.data;
    switch (t.dtype) {
        case TP_AMD_FLOAT32: return *static_cast<const float*>(p);
        case TP_AMD_FLOAT64: return *static_cast<const double*>(p);
        case TP_AMD_FLOAT16: return host_f16_to_float(*static_cast<const uint16_t*>(p));
        case TP_AMD_BFLOAT16: return host_bf16_to_float(*static_cast<const uint16_t*>(p));
        case TP_AMD_INT8: return *static_cast<const int8_t*>(p);
        case TP_AMD_INT16: return *static_cast<const int16_t*>(p);
        case TP_AMD_INT32: return *static_cast<const int32_t*>(p);
        case TP_AMD_INT64: return static_cast<double>(*static_cast<const int64_t*>(p));
        case TP_AMD_UINT8: return *static_cast<const uint8_t*>(p);
        case TP_AMD_BOOL: return *static_cast<const uint8_t*>(p) != 0 ? 1.0 : 0.0;
        default: TP_AMD_CHECK(false, "unknown dtype code ", t.dtype);
    }
    return 0.0;
}

// ---- fill --------------------------------------------------------------------

void fill(const TensorRef& self, const tp_amd_scalar& value) {
    if (numel(self) == 0) return;
    TP_AMD_CHECK(on_device(self), "fill_: the tensor is not on a device");
    alignas(16) unsigned char bytes[16] = {};
    const double f = value.f;
    const bool integral = value.kind != TP_AMD_SCALAR_FLOAT;
    // Scalar::to<intN>() of a floating value truncates; an integral value
    // converts exactly (wrapping to the width).
    const int64_t iv = integral ? value.i : static_cast<int64_t>(f);
    switch (self.dtype) {
        case TP_AMD_FLOAT32: { const float v = static_cast<float>(f); std::memcpy(bytes, &v, 4); break; }
        case TP_AMD_FLOAT64: std::memcpy(bytes, &f, 8); break;
        case TP_AMD_FLOAT16: { const uint16_t v = host_float_to_f16(static_cast<float>(f)); std::memcpy(bytes, &v, 2); break; }
        case TP_AMD_BFLOAT16: { const uint16_t v = host_float_to_bf16(static_cast<float>(f)); std::memcpy(bytes, &v, 2); break; }
        case TP_AMD_INT8: { const int8_t v = static_cast<int8_t>(iv); std::memcpy(bytes, &v, 1); break; }
        case TP_AMD_INT16: { const int16_t v = static_cast<int16_t>(iv); std::memcpy(bytes, &v, 2); break; }
        case TP_AMD_INT32: { const int32_t v = static_cast<int32_t>(iv); std::memcpy(bytes, &v, 4); break; }
        case TP_AMD_INT64: std::memcpy(bytes, &iv, 8); break;
        case TP_AMD_UINT8: { const uint8_t v = static_cast<uint8_t>(iv); std::memcpy(bytes, &v, 1); break; }
        case TP_AMD_BOOL: { const uint8_t v = (integral ? value.i != 0 : f != 0.0) ? 1 : 0; std::memcpy(bytes, &v, 1); break; }
        default: TP_AMD_CHECK(false, "fill_: unknown dtype code ", self.dtype);
    }
    const int st = tp_amd_launch_fill(self.device, element_size(self.dtype), bytes, self.ndim,
                                      self.sizes, self.data, self.strides);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
}

// ---- conversions ----------------------------------------------------------------

namespace {

// The pairs the reference converts in one device call
// (CopyKernels.cpp:42-108); other pairs go through float32 when both legs
// are listed (:152-158).
bool direct_cast(int from, int to) {
    static const std::set<std::pair<int, int>> pairs = [] {
        const int F = TP_AMD_FLOAT32, H = TP_AMD_FLOAT16, B = TP_AMD_BFLOAT16, D = TP_AMD_FLOAT64;
        const int I8 = TP_AMD_INT8, I16 = TP_AMD_INT16, I32 = TP_AMD_INT32, I64 = TP_AMD_INT64;
        const int U8 = TP_AMD_UINT8, BO = TP_AMD_BOOL;
        return std::set<std::pair<int, int>>{
            {F, H}, {F, B}, {F, I32}, {F, I64}, {F, I16}, {F, I8}, {F, U8}, {F, BO}, {F, D},
            {H, F}, {H, I32}, {H, I64}, {H, I16}, {H, I8}, {H, U8}, {H, BO},
            {B, F}, {B, I32}, {B, I64}, {B, I16}, {B, I8}, {B, U8}, {B, BO},
            {I32, F}, {I32, H}, {I32, B}, {I32, I64}, {I32, I16}, {I32, I8}, {I32, U8}, {I32, BO},
            {I64, F}, {I64, H}, {I64, B}, {I64, I32}, {I64, I16}, {I64, BO}, {I64, D},
            {I16, F}, {I16, H}, {I16, B}, {I16, I32}, {I16, I64}, {I16, I8},
            {I8, F}, {I8, H}, {I8, B}, {I8, I32}, {I8, I16},
            {U8, F}, {U8, H}, {U8, B}, {U8, I32}, {U8, I64},
            {BO, F}, {BO, H}, {BO, B}, {BO, I32}, {BO, I64},
            {D, F}, {D, I64}};
    }();
    return pairs.count({from, to}) != 0;
}

void launch_cast(const TensorRef& dst, const TensorRef& src) {
    const int st = tp_amd_launch_cast(dst.device, src.dtype, dst.dtype, numel(dst), src.data,
                                      dst.data);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
}

}  // namespace

void cast_dense(const TensorRef& dst, const TensorRef& src) {
    TP_AMD_CHECK(numel(dst) == numel(src), "cast: element count mismatch");
    if (numel(dst) == 0) return;
    const int from = src.dtype, to = dst.dtype;
    if (from == to || direct_cast(from, to) || from == TP_AMD_FLOAT32 || to == TP_AMD_FLOAT32 ||
        !(direct_cast(from, TP_AMD_FLOAT32) && direct_cast(TP_AMD_FLOAT32, to))) {
        // Direct (pairs without a float32 route convert directly, as the
        // host conversion the reference falls back to does).
        launch_cast(dst, src);
        return;
    }
    Owned mid = empty_on(sizes_of(src), TP_AMD_FLOAT32, src.device);
    launch_cast(mid.ref(), src);
    launch_cast(dst, mid.ref());
}

MaybeOwned to_dtype(const TensorRef& t, int dtype) {
    MaybeOwned m;
    if (t.dtype == dtype) {
        m.ref = t;
        m.ref.ctx = nullptr;
        return m;
    }
    m.hold = empty_on(sizes_of(t), dtype, t.device);
    copy_into(m.hold.ref(), t);
    m.ref = m.hold.ref();
    return m;
}

// ---- copy_ routes (CopyKernels.cpp:161-264) --------------------------------------

namespace {

// Gather a strided host view into dense memory (element size ``es``).
void host_gather(void* dst, const TensorRef& src) {
    const int es = element_size(src.dtype);
    const int64_t n = numel(src);
    const char* base = static_cast<const char*>(src.data);
    char* out = static_cast<char*>(dst);
    std::vector<int64_t> idx(src.ndim, 0);
    for (int64_t i = 0; i < n; ++i) {
        int64_t off = 0;
        for (int d = 0; d < src.ndim; ++d) off += idx[d] * src.strides[d];
        std::memcpy(out + i * es, base + off * es, es);
        for (int d = src.ndim - 1; d >= 0; --d) {
            if (++idx[d] < src.sizes[d]) break;
            idx[d] = 0;
        }
    }
}

void host_scatter(const TensorRef& dst, const void* src) {
    const int es = element_size(dst.dtype);
    const int64_t n = numel(dst);
    char* base = static_cast<char*>(dst.data);
    const char* in = static_cast<const char*>(src);
    std::vector<int64_t> idx(dst.ndim, 0);
    for (int64_t i = 0; i < n; ++i) {
        int64_t off = 0;
        for (int d = 0; d < dst.ndim; ++d) off += idx[d] * dst.strides[d];
        std::memcpy(base + off * es, in + i * es, es);
        for (int d = dst.ndim - 1; d >= 0; --d) {
            if (++idx[d] < dst.sizes[d]) break;
            idx[d] = 0;
        }
    }
}

void host_to_device(const TensorRef& self, const TensorRef& src) {
    // Shape is settled on the host; only dense bytes move, then the device
    // converts the dtype (the reference converts on the host, :169-184; the
    // conversion rules are the same).
    const TensorRef host = expand_to(src, sizes_of(self));
    const int64_t n = numel(self);
    const size_t nbytes = static_cast<size_t>(n) * element_size(src.dtype);
    if (is_contiguous(host) && src.dtype == self.dtype && is_contiguous(self)) {
        // The bytes already lie as the destination wants them.
        copy_to_device(self.data, host.data, nbytes, self.device);
        return;
    }
    // Otherwise the host bytes go dense (a gather when the source is strided
    // or broadcast) to a device buffer of the source dtype first.
    std::unique_ptr<char[]> gathered;
    const char* dense = static_cast<const char*>(host.data);
    if (!is_contiguous(host)) {
        gathered.reset(new char[nbytes]);
        host_gather(gathered.get(), host);
        dense = gathered.get();
    }
    Owned staging = empty_on(sizes_of(self), src.dtype, self.device);
    copy_to_device(staging.ref().data, dense, nbytes, self.device);
    if (src.dtype == self.dtype) {
        if (is_contiguous(self)) {
            copy_on_device(self.data, staging.ref().data, nbytes, self.device);
        } else {
            strided_copy(self, staging.ref());
        }
        return;
    }
    if (is_contiguous(self)) {
        cast_dense(self, staging.ref());
    } else {
        Owned conv = empty_on(sizes_of(self), self.dtype, self.device);
        cast_dense(conv.ref(), staging.ref());
        strided_copy(self, conv.ref());
    }
}

void device_to_host(const TensorRef& self, const TensorRef& src) {
    const size_t nbytes = static_cast<size_t>(numel(self)) * element_size(self.dtype);
    if (is_contiguous(self) && is_contiguous(src) && self.dtype == src.dtype &&
        sizes_of(self) == sizes_of(src)) {
        copy_to_host(self.data, src.data, nbytes, src.device);
        return;
    }
    // Convert and densify on the device, then place on the host.
    const TensorRef expanded = expand_to(src, sizes_of(self));
    Owned dense = empty_on(sizes_of(self), self.dtype, src.device);
    if (src.dtype == self.dtype) {
        strided_copy(dense.ref(), expanded);
    } else {
        MaybeOwned packed = contiguous_on_device(expanded);
        cast_dense(dense.ref(), packed.ref);
    }
    if (is_contiguous(self)) {
        copy_to_host(self.data, dense.ref().data, nbytes, src.device);
        return;
    }
    std::unique_ptr<char[]> tmp(new char[nbytes]);
    copy_to_host(tmp.get(), dense.ref().data, nbytes, src.device);
    host_scatter(self, tmp.get());
}

void device_to_device(const TensorRef& self, const TensorRef& src) {
    if (src.device != self.device) {
        // Between devices: through the host (:199-201).
        const size_t nbytes = static_cast<size_t>(numel(src)) * element_size(src.dtype);
        MaybeOwned packed = contiguous_on_device(src);
        std::unique_ptr<char[]> tmp(new char[nbytes]);
        copy_to_host(tmp.get(), packed.ref.data, nbytes, src.device);
        TensorRef host = packed.ref;
        host.data = tmp.get();
        host.device = -1;
        host.ctx = nullptr;
        host_to_device(self, host);
        return;
    }
    const TensorRef source = expand_to(src, sizes_of(self));
    if (source.dtype == self.dtype) {
        strided_copy(self, source);
        return;
    }
    // A dense conversion writes the result once, straight into the
    // destination; anything else converts into a dense copy first.
    if (is_contiguous(source) && is_contiguous(self)) {
        cast_dense(self, source);
        return;
    }
    MaybeOwned packed = contiguous_on_device(source);
    Owned converted = empty_on(sizes_of(self), self.dtype, self.device);
    cast_dense(converted.ref(), packed.ref);
    strided_copy(self, converted.ref());
}

}  // namespace

void copy_into(const TensorRef& self, const TensorRef& src) {
    check_view(self, "copy_ destination");
    check_view(src, "copy_ source");
    if (numel(self) == 0) return;
    const bool self_dev = on_device(self), src_dev = on_device(src);
    if (self_dev && src_dev) {
        device_to_device(self, src);
    } else if (self_dev) {
        host_to_device(self, src);
    } else if (src_dev) {
        device_to_host(self, src);
    } else {
        TP_AMD_CHECK(false, "copy_: neither side is device memory");
    }
}

}  // namespace tp_amd
