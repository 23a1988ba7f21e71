#include "runtime.h"

#include <array>
#include <atomic>
#include <cstring>
#include <memory>
#include <mutex>

#include "tp_amd_runtime.h"

namespace tp_amd {

namespace {

std::array<std::atomic<hipStream_t>, kMaxDevices> g_streams{};
std::array<std::atomic<int>, kMaxDevices> g_cu_counts{};
std::mutex g_stream_lock;

thread_local std::string t_last_error;

}  // namespace

void set_last_error(const std::string& message) { t_last_error = message; }
const char* last_error() { return t_last_error.c_str(); }

const char* dtype_name(int dtype) {
    switch (dtype) {
        case TP_AMD_FLOAT32: return "float32";
        case TP_AMD_FLOAT16: return "float16";
        case TP_AMD_BFLOAT16: return "bfloat16";
        case TP_AMD_FLOAT64: return "float64";
        case TP_AMD_INT8: return "int8";
        case TP_AMD_INT16: return "int16";
        case TP_AMD_INT32: return "int32";
        case TP_AMD_INT64: return "int64";
        case TP_AMD_UINT8: return "uint8";
        case TP_AMD_BOOL: return "bool";
        case TP_AMD_UNDEFINED: return "undefined";
        default: return "unknown";
    }
}

int device_count() noexcept {
    static const int count = [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            return 0;
        }
        return n < kMaxDevices ? n : kMaxDevices;
    }();
    return count;
}

int current_device() {
    int index = 0;
    TP_AMD_HIP_CHECK(hipGetDevice(&index));
    return index;
}

static void check_index(int index) {
    const int count = device_count();
    TP_AMD_CHECK(index >= 0 && index < count, "invalid device index ", index, " (", count,
                 " device(s) visible)");
}

void set_device(int index) {
    check_index(index);
    TP_AMD_HIP_CHECK(hipSetDevice(index));
}

int resolve_device(int index) {
    TP_AMD_CHECK(device_count() > 0, "no GPU device is visible");
    if (index < 0) index = current_device();
    check_index(index);
    return index;
}

DeviceGuard::DeviceGuard(int index) : previous_(current_device()), current_(index) {
    if (current_ != previous_) set_device(current_);
}

DeviceGuard::~DeviceGuard() {
    if (current_ != previous_) (void)hipSetDevice(previous_);
}

hipStream_t stream(int index) {
    check_index(index);
    hipStream_t s = g_streams[index].load(std::memory_order_acquire);
    if (s != nullptr) return s;
    std::lock_guard<std::mutex> lock(g_stream_lock);
    s = g_streams[index].load(std::memory_order_relaxed);
    if (s == nullptr) {
        DeviceGuard guard(index);
        TP_AMD_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        g_streams[index].store(s, std::memory_order_release);
    }
    return s;
}

namespace {

// Host copies and synchronisation cannot be part of a recorded sequence
// (the recording holds device work only): refuse them while the stream is
// being recorded, before anything reaches the runtime.
void refuse_while_recording(hipStream_t s, const char* what) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    TP_AMD_HIP_CHECK(hipStreamIsCapturing(s, &status));
    TP_AMD_CHECK(status == hipStreamCaptureStatusNone, what,
                 " while the stream is being recorded: a recorded step may only queue "
                 "device work");
}

}  // namespace

void synchronize(int index) {
    DeviceGuard guard(index);
    refuse_while_recording(stream(index), "synchronisation");
    TP_AMD_HIP_CHECK(hipStreamSynchronize(stream(index)));
}

void copy_to_device(void* device_dst, const void* host_src, size_t nbytes, int index) {
    if (nbytes == 0) return;
    DeviceGuard guard(index);
    hipStream_t s = stream(index);
    refuse_while_recording(s, "a host-to-device copy");
    TP_AMD_HIP_CHECK(hipMemcpyAsync(device_dst, host_src, nbytes, hipMemcpyHostToDevice, s));
    TP_AMD_HIP_CHECK(hipStreamSynchronize(s));
}

void copy_to_host(void* host_dst, const void* device_src, size_t nbytes, int index) {
    if (nbytes == 0) return;
    DeviceGuard guard(index);
    hipStream_t s = stream(index);
    refuse_while_recording(s, "a device-to-host copy");
    TP_AMD_HIP_CHECK(hipMemcpyAsync(host_dst, device_src, nbytes, hipMemcpyDeviceToHost, s));
    TP_AMD_HIP_CHECK(hipStreamSynchronize(s));
}

void copy_on_device(void* dst, const void* src, size_t nbytes, int index) {
    if (nbytes == 0 || dst == src) return;
    DeviceGuard guard(index);
    TP_AMD_HIP_CHECK(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, stream(index)));
}

int cu_count(int index) {
    check_index(index);
    int n = g_cu_counts[index].load(std::memory_order_relaxed);
    if (n == 0) {
        TP_AMD_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, index));
        g_cu_counts[index].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace tp_amd

using namespace tp_amd;

extern "C" {

const char* tp_mlu_last_error(void) { return last_error(); }

int tp_mlu_device_count(void) { return device_count(); }

int tp_amd_is_available(void) { return device_count() > 0 ? 1 : 0; }

int tp_amd_current_device(int* index) {
    return guarded([&] {
        TP_AMD_CHECK(index != nullptr, "tp_amd_current_device: null output");
        TP_AMD_CHECK(device_count() > 0, "no GPU device is visible");
        *index = current_device();
    });
}

int tp_amd_set_device(int index) {
    return guarded([&] { set_device(index); });
}

int tp_amd_synchronize(int index) {
    return guarded([&] { synchronize(resolve_device(index)); });
}

int tp_amd_mem_get_info(int index, size_t* free_bytes, size_t* total_bytes) {
    return guarded([&] {
        TP_AMD_CHECK(free_bytes != nullptr && total_bytes != nullptr,
                     "tp_amd_mem_get_info: null output");
        DeviceGuard guard(resolve_device(index));
        TP_AMD_HIP_CHECK(hipMemGetInfo(free_bytes, total_bytes));
    });
}

int tp_amd_copy_bytes(void* dst, int dst_device, const void* src, int src_device,
                      size_t nbytes) {
    return guarded([&] {
        if (nbytes == 0) return;
        TP_AMD_CHECK(dst != nullptr && src != nullptr, "tp_amd_copy_bytes: null pointer");
        const bool dst_dev = dst_device >= 0, src_dev = src_device >= 0;
        if (dst_dev && src_dev) {
            if (dst_device == src_device) {
                copy_on_device(dst, src, nbytes, dst_device);
                return;
            }
            // Between two devices: through the host (MLUHooks.cpp:34-37).
            std::unique_ptr<char[]> bounce(new char[nbytes]);
            copy_to_host(bounce.get(), src, nbytes, src_device);
            copy_to_device(dst, bounce.get(), nbytes, dst_device);
        } else if (dst_dev) {
            copy_to_device(dst, src, nbytes, dst_device);
        } else if (src_dev) {
            copy_to_host(dst, src, nbytes, src_device);
        } else {
            std::memcpy(dst, src, nbytes);
        }
    });
}

int tp_amd_stream(int index, void** out) {
    return guarded([&] {
        TP_AMD_CHECK(out != nullptr, "tp_amd_stream: null output");
        *out = static_cast<void*>(stream(resolve_device(index)));
    });
}

int tp_amd_event_create(void** event) {
    return guarded([&] {
        TP_AMD_CHECK(event != nullptr, "tp_amd_event_create: null output");
        hipEvent_t e = nullptr;
        TP_AMD_HIP_CHECK(hipEventCreate(&e));
        *event = static_cast<void*>(e);
    });
}

int tp_amd_event_record(void* event, int device) {
    return guarded([&] {
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        TP_AMD_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), stream(index)));
    });
}

int tp_amd_event_elapsed_ms(void* start, void* stop, float* ms) {
    return guarded([&] {
        TP_AMD_CHECK(ms != nullptr, "tp_amd_event_elapsed_ms: null output");
        TP_AMD_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
        TP_AMD_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                             static_cast<hipEvent_t>(stop)));
    });
}

int tp_amd_event_destroy(void* event) {
    return guarded([&] { TP_AMD_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event))); });
}

}  // extern "C"
