// HIP device layer: device count, current device, one stream per device and
// byte copies ordered on it.  MI355X-native replacement of the reference's
// CNRT runtime glue (tensorplay_mlu/csrc/MLURuntime.h:54-96,
// MLURuntime.cpp:34-136).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "common.h"

namespace tp_amd {

constexpr int kMaxDevices = 64;

// Visible devices, 0 when the driver or GPU is absent (MLURuntime.cpp:34-41).
int device_count() noexcept;
int current_device();
void set_device(int index);
// ``index`` itself when >= 0, else the current device; checked.
int resolve_device(int index);

// Makes ``index`` current for the guard's lifetime (MLURuntime.cpp:73-79).
class DeviceGuard {
public:
    explicit DeviceGuard(int index);
    ~DeviceGuard();
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;

private:
    int previous_;
    int current_;
};

// The single stream all work on ``index`` is issued to, created on first use
// with default priority and no implicit synchronization with the null
// stream (MLURuntime.cpp:81-93).
hipStream_t stream(int index);

// Wait for the device's stream (MLURuntime.cpp:107-110).
void synchronize(int index);

// Host copies return once the bytes have landed: the host side may be
// pageable memory the caller frees right after (MLURuntime.cpp:112-129).
void copy_to_device(void* device_dst, const void* host_src, size_t nbytes, int index);
void copy_to_host(void* host_dst, const void* device_src, size_t nbytes, int index);
// Ordered on the stream, asynchronous (MLURuntime.cpp:131-136).
void copy_on_device(void* dst, const void* src, size_t nbytes, int index);

// Number of compute units of ``index`` (cached), used to size grids.
int cu_count(int index);

}  // namespace tp_amd
