// PrivateUse1 allocator, device hooks and the init hook for TensorPlay.
//
// * Allocator (reference MLUAllocator.cpp:61-73, 239-240): allocate() hands
//   out a block of the library's caching allocator (tp_amd_malloc) as
//   DataPtr(ptr, ctx = block, deleter = tp_amd_free, device).  adopt() wraps
//   a result the operator C-ABI already allocated the same way: it parks the
//   block in a thread-local slot that the next allocate() on this thread
//   returns instead of allocating, so the Storage owns exactly that block.
// * Hooks (reference MLUHooks.cpp:14-56): device count, current device,
//   synchronisation, byte copies in every direction, memory information.
// * tp_amd_tensorplay_register (called by tp_mlu_init, reference
//   Module.cpp:15-22): every operator without a device kernel runs through
//   TensorPlay's host fallback.

#include <cstdlib>
#include <cstring>
#include <utility>

#include "Adapter.h"
#include "PrivateUse1Hooks.h"

namespace tensorplay {
namespace amd {

namespace {

struct Parked {
    bool set = false;
    void* ptr = nullptr;
    void* ctx = nullptr;
};
thread_local Parked t_parked;

class DeviceAllocator final : public Allocator {
public:
    DataPtr allocate(size_t nbytes) const override {
        int index = 0;
        if (tp_amd_current_device(&index) != TP_AMD_OK) raise("allocate");
        return allocate(nbytes, Device(DeviceType::PrivateUse1, index));
    }

    DataPtr allocate(size_t nbytes, const Device& device) const override {
        const Device placed(DeviceType::PrivateUse1, index_of(device));
        if (t_parked.set) {
            Parked parked = std::exchange(t_parked, Parked{});
            return DataPtr(parked.ptr, parked.ctx, &tp_amd_free, placed);
        }
        void* ptr = nullptr;
        void* ctx = nullptr;
        if (tp_amd_malloc(nbytes, static_cast<int>(placed.index()), &ptr, &ctx) != TP_AMD_OK) {
            raise("allocate");
        }
        return DataPtr(ptr, ctx, &tp_amd_free, placed);
    }
};

DeviceAllocator g_allocator;
static ::tensorplay::detail::AllocatorRegisterer g_register_allocator(DeviceType::PrivateUse1,
                                                                      &g_allocator);

void check(int status, const char* what) {
    if (status != TP_AMD_OK) raise(what);
}

struct Hooks final : PrivateUse1HooksInterface {
    bool is_available() const override { return tp_amd_is_available() != 0; }
    int64_t device_count() const override { return tp_mlu_device_count(); }
    int64_t current_device() const override {
        int index = 0;
        check(tp_amd_current_device(&index), "current_device");
        return index;
    }
    void set_device(int64_t index) const override {
        check(tp_amd_set_device(static_cast<int>(index)), "set_device");
    }
    void synchronize(int64_t index) const override {
        check(tp_amd_synchronize(static_cast<int>(index)), "synchronize");
    }
    // Host <-> device copies synchronise; device <-> device is ordered on the
    // stream; between two GPUs the runtime copies peer to peer.
    void copy_bytes(void* dst, const Device& dst_device, const void* src,
                    const Device& src_device, size_t nbytes) const override {
        const int dst_index = dst_device.is_privateuse1() ? index_of(dst_device) : -1;
        const int src_index = src_device.is_privateuse1() ? index_of(src_device) : -1;
        if (dst_index < 0 && src_index < 0) {
            std::memcpy(dst, src, nbytes);
            return;
        }
        check(tp_amd_copy_bytes(dst, dst_index, src, src_index, nbytes), "copy_bytes");
    }
    std::pair<size_t, size_t> memory_info(int64_t index) const override {
        size_t free_bytes = 0, total_bytes = 0;
        check(tp_amd_mem_get_info(static_cast<int>(index), &free_bytes, &total_bytes),
              "memory_info");
        return {free_bytes, total_bytes};
    }
};

Hooks g_hooks;
REGISTER_PRIVATEUSE1_HOOKS(&g_hooks);

}  // namespace

Allocator* allocator() { return &g_allocator; }

int index_of(const Device& device) {
    if (device.index() >= 0) return static_cast<int>(device.index());
    int index = 0;
    check(tp_amd_current_device(&index), "current_device");
    return index;
}

int dtype_code(DType dtype) {
    switch (dtype) {
        case DType::Float32: return TP_AMD_FLOAT32;
        case DType::Float16: return TP_AMD_FLOAT16;
        case DType::BFloat16: return TP_AMD_BFLOAT16;
        case DType::Float64: return TP_AMD_FLOAT64;
        case DType::Int8: return TP_AMD_INT8;
        case DType::Int16: return TP_AMD_INT16;
        case DType::Int32: return TP_AMD_INT32;
        case DType::Int64: return TP_AMD_INT64;
        case DType::UInt8: return TP_AMD_UINT8;
        case DType::Bool: return TP_AMD_BOOL;
        default: return TP_AMD_UNDEFINED;
    }
}

DType dtype_of(int code) {
    switch (code) {
        case TP_AMD_FLOAT32: return DType::Float32;
        case TP_AMD_FLOAT16: return DType::Float16;
        case TP_AMD_BFLOAT16: return DType::BFloat16;
        case TP_AMD_FLOAT64: return DType::Float64;
        case TP_AMD_INT8: return DType::Int8;
        case TP_AMD_INT16: return DType::Int16;
        case TP_AMD_INT32: return DType::Int32;
        case TP_AMD_INT64: return DType::Int64;
        case TP_AMD_UINT8: return DType::UInt8;
        case TP_AMD_BOOL: return DType::Bool;
        default: return DType::Undefined;
    }
}

bool view(const Tensor& t, tp_amd_tensor* out) {
    *out = tp_amd_tensor{};
    const int code = dtype_code(t.dtype());
    if (code == TP_AMD_UNDEFINED || t.dim() > TP_AMD_MAX_DIMS) return false;
    const auto sizes = t.sizes().vec();
    const auto strides = t.strides();
    out->data = t.data_ptr();
    out->ndim = static_cast<int32_t>(sizes.size());
    for (size_t i = 0; i < sizes.size(); ++i) {
        out->sizes[i] = sizes[i];
        out->strides[i] = strides[i];
    }
    out->dtype = code;
    out->device = t.device().is_privateuse1() ? index_of(t.device()) : -1;
    return true;
}

tp_amd_scalar scalar(const Scalar& s) {
    tp_amd_scalar out{};
    if (s.isFloatingPoint()) {
        out.kind = TP_AMD_SCALAR_FLOAT;
        out.f = s.toDouble();
    } else if (s.isIntegral(false)) {
        out.kind = TP_AMD_SCALAR_INT;
        out.i = s.to<int64_t>();
        out.f = static_cast<double>(out.i);
    } else {
        out.kind = TP_AMD_SCALAR_BOOL;
        out.i = s.to<bool>() ? 1 : 0;
        out.f = static_cast<double>(out.i);
    }
    return out;
}

Scalar to_scalar(const tp_amd_scalar& s) {
    switch (s.kind) {
        case TP_AMD_SCALAR_INT: return Scalar(static_cast<int64_t>(s.i));
        case TP_AMD_SCALAR_BOOL: return Scalar(s.i != 0);
        default: return Scalar(s.f);
    }
}

Tensor adopt(const tp_amd_tensor& result) {
    std::vector<int64_t> sizes(result.sizes, result.sizes + result.ndim);
    const DType dtype = dtype_of(result.dtype);
    int64_t numel = 1;
    for (int64_t d : sizes) numel *= d;
    t_parked = Parked{true, result.data, result.ctx};
    Storage storage(static_cast<size_t>(numel) * elementSize(dtype), allocator(),
                    Device(DeviceType::PrivateUse1, result.device));
    TP_CHECK(!t_parked.set, "tensorplay-mlu_amd: storage did not take the result block");
    return Tensor(std::move(storage), sizes, dtype);
}

void raise(const char* op) {
    const char* message = tp_mlu_last_error();
    TP_CHECK(false, "tensorplay-mlu_amd: ", op, ": ", message ? message : "unknown error");
    std::abort();  // not reached: a failed TP_CHECK throws
}

}  // namespace amd
}  // namespace tensorplay

extern "C" int tp_amd_tensorplay_register(void) {
    try {
        ::tensorplay::cpu_fallback::register_host_fallbacks(
            ::tensorplay::DispatchKey::PrivateUse1);
        return 0;
    } catch (...) {
        return 1;
    }
}
