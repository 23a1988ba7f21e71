// Declarations of the TensorPlay C++ API as the reference backend uses it
// (tensorplay_mlu/csrc/*.cpp), for a syntax check of the PrivateUse1
// adapter (tensorplay-mlu_amd/csrc/tensorplay/) on a machine without
// TensorPlay's headers.  Declarations only: nothing here is linked or run.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace tensorplay {

enum class DeviceType { CPU, PrivateUse1 };

class Device {
public:
    Device(DeviceType type, int64_t index = -1);
    int64_t index() const;
    bool is_privateuse1() const;
};

enum class DType {
    Undefined, Float32, Float16, BFloat16, Float64, Int8, Int16, Int32, Int64, UInt8, Bool,
    ComplexFloat
};
size_t elementSize(DType dtype);

enum class DispatchKey { CPU, PrivateUse1 };

template <typename... Args>
[[noreturn]] void throw_error(const Args&... args);

#define TP_CHECK(cond, ...)                                               \
    do {                                                                  \
        if (!(cond)) ::tensorplay::throw_error(__VA_ARGS__);             \
    } while (0)

class Scalar {
public:
    Scalar(double v);
    Scalar(int64_t v);
    Scalar(bool v);
    bool isFloatingPoint() const;
    bool isIntegral(bool include_bool) const;
    double toDouble() const;
    template <typename T>
    T to() const;
};

class DataPtr {
public:
    DataPtr();
    DataPtr(void* ptr, void* ctx, void (*deleter)(void*), Device device);
};

class Allocator {
public:
    virtual ~Allocator() = default;
    virtual DataPtr allocate(size_t nbytes) const = 0;
    virtual DataPtr allocate(size_t nbytes, const Device& device) const = 0;
};

namespace detail {
struct AllocatorRegisterer {
    AllocatorRegisterer(DeviceType type, Allocator* allocator);
};
}  // namespace detail

class Storage {
public:
    Storage(size_t nbytes, Allocator* allocator, Device device);
};

class IntArrayRef {
public:
    std::vector<int64_t> vec() const;
};

class Tensor {
public:
    Tensor();
    Tensor(Storage storage, const std::vector<int64_t>& sizes, DType dtype);
    Tensor(const std::vector<int64_t>& sizes, DType dtype, Device device);
    IntArrayRef sizes() const;
    std::vector<int64_t> strides() const;
    DType dtype() const;
    Device device() const;
    void* data_ptr() const;
    int64_t numel() const;
    int64_t dim() const;
    bool is_contiguous() const;
    bool defined() const;
    Tensor& fill_(const Scalar& value);
};

class Library {
public:
    template <typename F>
    void impl(const char* name, F* fn);
};

#define TENSORPLAY_LIBRARY_IMPL(key, name)                                 \
    static void name##_define(::tensorplay::Library& m);                  \
    static void name##_define(::tensorplay::Library& m)

template <size_t N>
struct FixedString {
    constexpr FixedString(const char (&s)[N]) {
        for (size_t i = 0; i < N; ++i) text[i] = s[i];
    }
    char text[N];
};

namespace cpu_fallback {
template <FixedString Name, typename Sig>
struct Kernel;
template <FixedString Name, typename R, typename... Args>
struct Kernel<Name, R(Args...)> {
    static R call(Args... args);
};
void register_host_fallbacks(DispatchKey key);
}  // namespace cpu_fallback

struct PrivateUse1HooksInterface {
    virtual ~PrivateUse1HooksInterface() = default;
    virtual bool is_available() const = 0;
    virtual int64_t device_count() const = 0;
    virtual int64_t current_device() const = 0;
    virtual void set_device(int64_t index) const = 0;
    virtual void synchronize(int64_t index) const = 0;
    virtual void copy_bytes(void* dst, const Device& dst_device, const void* src,
                            const Device& src_device, size_t nbytes) const = 0;
    virtual std::pair<size_t, size_t> memory_info(int64_t index) const = 0;
};
int register_privateuse1_hooks(PrivateUse1HooksInterface* hooks);
#define REGISTER_PRIVATEUSE1_HOOKS(ptr) \
    static int tp_hooks_registered = ::tensorplay::register_privateuse1_hooks(ptr)

}  // namespace tensorplay
