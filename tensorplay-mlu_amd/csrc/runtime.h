// HIP device layer: which GPUs exist, one work stream per GPU, and byte
// copies ordered on that stream.  It stands where the reference's CNRT glue
// stands (tensorplay_mlu/csrc/MLURuntime.h:54-96): the same contract -- one
// queue per device shared by every thread, host copies that return once the
// bytes have landed, device copies that are only queued -- on a design of
// its own: a table with one slot per GPU, filled once per GPU, and a scope
// object that is the only way code here switches the current GPU.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "common.h"

namespace tp_amd {

constexpr int kMaxDevices = 64;

// GPUs this process sees (at most kMaxDevices; 0 without a driver or GPU).
int device_count() noexcept;
int current_device();
void set_device(int index);
// ``index`` when >= 0, else the current GPU; throws unless it names a
// visible GPU.
int resolve_device(int index);

// Opens every visible GPU's slot now (tp_mlu_init), so the first operator
// does not pay for stream creation.
void open_all_devices();

// For its lifetime, makes a GPU current (``index`` < 0: the current one) and
// hands out that GPU's slot; the previous GPU is made current again at the
// end of the scope, if the scope changed it.
class OnDevice {
public:
    explicit OnDevice(int index);
    ~OnDevice();
    OnDevice(const OnDevice&) = delete;
    OnDevice& operator=(const OnDevice&) = delete;

    int index() const { return index_; }
    hipStream_t stream() const;

private:
    int index_;
    int restore_;  // the GPU to make current again, or -1
};

// The stream every piece of work on GPU ``index`` is queued on: default
// priority, no implicit synchronisation with the null stream.
hipStream_t stream(int index);

// Number of compute units of GPU ``index``, used to size grids.
int cu_count(int index);

// Wait until GPU ``index``'s stream has drained.
void synchronize(int index);

// Host copies return once the bytes have landed: the host side may be
// pageable memory the caller frees right after.
void copy_to_device(void* device_dst, const void* host_src, size_t nbytes, int index);
void copy_to_host(void* host_dst, const void* device_src, size_t nbytes, int index);
// Queued on the stream; returns at once.
void copy_on_device(void* dst, const void* src, size_t nbytes, int index);

}  // namespace tp_amd
