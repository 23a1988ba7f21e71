#include "runtime.h"

#include <algorithm>
#include <array>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <memory>
#include <mutex>
#include <thread>

#include "tp_amd_runtime.h"

namespace tp_amd {

namespace {

thread_local std::string t_last_error;

// One GPU's state.  ``opened`` guards the one-time set-up; a set-up that
// throws leaves the slot closed and the next use tries again.
struct DeviceSlot {
    std::once_flag opened;
    hipStream_t stream = nullptr;
    int compute_units = 0;
};

// Every GPU the process sees, enumerated once.  The table is never
// destroyed: streams stay valid until the process ends, also for work
// queued from static destructors.
class DeviceTable {
public:
    static DeviceTable& get() {
        static DeviceTable* table = new DeviceTable();
        return *table;
    }

    int size() const { return visible_; }

    void require(int index) const {
        if (index >= 0 && index < visible_) return;
        throw Error(concat("GPU index ", index, " is out of range: this process sees ", visible_,
                           visible_ == 1 ? " GPU" : " GPUs"));
    }

    const DeviceSlot& slot(int index) {
        require(index);
        DeviceSlot& s = slots_[index];
        std::call_once(s.opened, [&] { open(index, s); });
        return s;
    }

private:
    DeviceTable() {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();  // no driver or no GPU: an empty table
            n = 0;
        }
        visible_ = std::min(n, kMaxDevices);
    }

    static void open(int index, DeviceSlot& s) {
        const OnDevice scope(index);
        TP_AMD_HIP_CHECK(hipDeviceGetAttribute(&s.compute_units, hipDeviceAttributeMultiprocessorCount, index));
        TP_AMD_HIP_CHECK(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
    }

    int visible_ = 0;
    std::array<DeviceSlot, kMaxDevices> slots_;
};

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
    try {
        return DeviceTable::get().size();
    } catch (...) {
        return 0;
    }
}

int current_device() {
    int index = 0;
    TP_AMD_HIP_CHECK(hipGetDevice(&index));
    return index;
}

void set_device(int index) {
    DeviceTable::get().require(index);
    TP_AMD_HIP_CHECK(hipSetDevice(index));
}

int resolve_device(int index) {
    DeviceTable& table = DeviceTable::get();
    TP_AMD_CHECK(table.size() > 0, "no GPU is visible to this process");
    const int resolved = index < 0 ? current_device() : index;
    table.require(resolved);
    return resolved;
}

void open_all_devices() {
    DeviceTable& table = DeviceTable::get();
    for (int d = 0; d < table.size(); ++d) (void)table.slot(d);
}

OnDevice::OnDevice(int index) : index_(resolve_device(index)), restore_(-1) {
    const int now = current_device();
    if (now != index_) {
        TP_AMD_HIP_CHECK(hipSetDevice(index_));
        restore_ = now;
    }
}

OnDevice::~OnDevice() {
    if (restore_ >= 0) (void)hipSetDevice(restore_);
}

hipStream_t OnDevice::stream() const { return DeviceTable::get().slot(index_).stream; }

hipStream_t stream(int index) { return DeviceTable::get().slot(index).stream; }

int cu_count(int index) { return DeviceTable::get().slot(index).compute_units; }

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
    const OnDevice scope(index);
    refuse_while_recording(stream(index), "synchronisation");
    TP_AMD_HIP_CHECK(hipStreamSynchronize(stream(index)));
}

namespace {

// Host memcpy spread over a few threads: the caller takes the first part,
// kCopyParts - 1 workers the rest.  The pool is created on first use and
// never destroyed (its threads would otherwise be torn down during static
// destruction while idle workers still wait on it).
constexpr int kCopyParts = 8;
constexpr size_t kSplitFrom = size_t{256} << 10;  // smaller copies stay on one thread

class CopyPool {
public:
    static CopyPool& instance() {
        static CopyPool* pool = new CopyPool();
        return *pool;
    }

    void copy(void* dst, const void* src, size_t n) {
        if (parts_ == 1 || n < kSplitFrom) {
            std::memcpy(dst, src, n);
            return;
        }
        std::lock_guard<std::mutex> job(job_lock_);  // one copy at a time
        {
            std::lock_guard<std::mutex> lock(m_);
            dst_ = static_cast<char*>(dst);
            src_ = static_cast<const char*>(src);
            n_ = n;
            pending_ = parts_ - 1;
            ++generation_;
        }
        start_.notify_all();
        copy_part(0);
        std::unique_lock<std::mutex> lock(m_);
        finish_.wait(lock, [&] { return pending_ == 0; });
    }

private:
    CopyPool() {
        const unsigned hw = std::thread::hardware_concurrency();
        parts_ = static_cast<int>(std::min<unsigned>(kCopyParts, hw > 1 ? hw : 1));
        for (int id = 1; id < parts_; ++id) std::thread([this, id] { work(id); }).detach();
    }

    // Part `id` of the current copy, in 64-byte multiples; the parts cover
    // all n_ bytes (per >= ceil(n_ / parts_)).  dst_, src_ and n_ were
    // written under m_ before the generation moved on, and a worker reads
    // them after seeing the new generation under m_.
    void copy_part(int id) const {
        const size_t per = ((n_ + parts_ - 1) / parts_ + 63) & ~size_t{63};
        const size_t lo = std::min(n_, per * id), hi = std::min(n_, lo + per);
        if (hi > lo) std::memcpy(dst_ + lo, src_ + lo, hi - lo);
    }

    void work(int id) {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lock(m_);
                start_.wait(lock, [&] { return generation_ != seen; });
                seen = generation_;
            }
            copy_part(id);
            std::lock_guard<std::mutex> lock(m_);
            if (--pending_ == 0) finish_.notify_one();
        }
    }

    int parts_ = 1;
    std::mutex job_lock_, m_;
    std::condition_variable start_, finish_;
    uint64_t generation_ = 0;
    int pending_ = 0;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t n_ = 0;
};

// Large copies between pageable host memory and a device go through
// kStages pinned chunks of kStageBytes per device (allocated on first use,
// kept until the process ends): the host copy of one chunk overlaps the DMA
// of the one before, and an event per chunk says when its buffer is free
// (to device) or filled (to host).
constexpr size_t kStageBytes = size_t{4} << 20;
constexpr int kStages = 4;
constexpr size_t kStageFrom = size_t{8} << 20;  // smaller copies take the runtime's own path

struct Staging {
    std::mutex lock;  // one staged copy at a time per device
    std::array<char*, kStages> buf{};
    std::array<hipEvent_t, kStages> ready{};
    bool allocated = false;
};
std::array<Staging, kMaxDevices> g_staging;

// The device's staging buffers, allocated on first use; the caller holds
// st.lock with the device current.
Staging& staging(int index) {
    Staging& st = g_staging[index];
    if (!st.allocated) {
        for (int b = 0; b < kStages; ++b) {
            if (st.buf[b] == nullptr) {
                TP_AMD_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&st.buf[b]), kStageBytes, hipHostMallocDefault));
            }
            if (st.ready[b] == nullptr) TP_AMD_HIP_CHECK(hipEventCreateWithFlags(&st.ready[b], hipEventDisableTiming));
        }
        st.allocated = true;
    }
    return st;
}

void staged_to_device(char* dst, const char* src, size_t n, hipStream_t s, int index) {
    Staging& st = g_staging[index];
    std::lock_guard<std::mutex> lock(st.lock);
    staging(index);
    for (size_t off = 0, c = 0; off < n; off += kStageBytes, ++c) {
        const int b = static_cast<int>(c % kStages);
        const size_t len = std::min(kStageBytes, n - off);
        TP_AMD_HIP_CHECK(hipEventSynchronize(st.ready[b]));  // the chunk's last DMA out of it is done
        CopyPool::instance().copy(st.buf[b], src + off, len);
        TP_AMD_HIP_CHECK(hipMemcpyAsync(dst + off, st.buf[b], len, hipMemcpyHostToDevice, s));
        TP_AMD_HIP_CHECK(hipEventRecord(st.ready[b], s));
    }
    TP_AMD_HIP_CHECK(hipStreamSynchronize(s));
}

void staged_to_host(char* dst, const char* src, size_t n, hipStream_t s, int index) {
    Staging& st = g_staging[index];
    std::lock_guard<std::mutex> lock(st.lock);
    staging(index);
    const size_t chunks = (n + kStageBytes - 1) / kStageBytes;
    auto fill = [&](size_t c) {  // DMA chunk c into its buffer, after the work queued before it
        const int b = static_cast<int>(c % kStages);
        const size_t off = c * kStageBytes;
        TP_AMD_HIP_CHECK(hipMemcpyAsync(st.buf[b], src + off, std::min(kStageBytes, n - off),
                                        hipMemcpyDeviceToHost, s));
        TP_AMD_HIP_CHECK(hipEventRecord(st.ready[b], s));
    };
    for (size_t c = 0; c < chunks && c < static_cast<size_t>(kStages); ++c) fill(c);
    for (size_t c = 0; c < chunks; ++c) {
        const int b = static_cast<int>(c % kStages);
        const size_t off = c * kStageBytes;
        TP_AMD_HIP_CHECK(hipEventSynchronize(st.ready[b]));
        CopyPool::instance().copy(dst + off, st.buf[b], std::min(kStageBytes, n - off));
        if (c + kStages < chunks) fill(c + kStages);
    }
}

}  // namespace

void copy_to_device(void* device_dst, const void* host_src, size_t nbytes, int index) {
    if (nbytes == 0) return;
    const OnDevice scope(index);
    hipStream_t s = stream(index);
    refuse_while_recording(s, "a host-to-device copy");
    if (nbytes >= kStageFrom) {
        staged_to_device(static_cast<char*>(device_dst), static_cast<const char*>(host_src), nbytes, s, index);
        return;
    }
    TP_AMD_HIP_CHECK(hipMemcpyAsync(device_dst, host_src, nbytes, hipMemcpyHostToDevice, s));
    TP_AMD_HIP_CHECK(hipStreamSynchronize(s));
}

void copy_to_host(void* host_dst, const void* device_src, size_t nbytes, int index) {
    if (nbytes == 0) return;
    const OnDevice scope(index);
    hipStream_t s = stream(index);
    refuse_while_recording(s, "a device-to-host copy");
    if (nbytes >= kStageFrom) {
        staged_to_host(static_cast<char*>(host_dst), static_cast<const char*>(device_src), nbytes, s, index);
        return;
    }
    TP_AMD_HIP_CHECK(hipMemcpyAsync(host_dst, device_src, nbytes, hipMemcpyDeviceToHost, s));
    TP_AMD_HIP_CHECK(hipStreamSynchronize(s));
}

void copy_on_device(void* dst, const void* src, size_t nbytes, int index) {
    if (nbytes == 0 || dst == src) return;
    const OnDevice scope(index);
    TP_AMD_HIP_CHECK(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, stream(index)));
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
        const OnDevice scope(index);
        TP_AMD_HIP_CHECK(hipMemGetInfo(free_bytes, total_bytes));
    });
}

int tp_amd_compute_units(int index, int* units) {
    return guarded([&] {
        TP_AMD_CHECK(units != nullptr, "tp_amd_compute_units: null output");
        *units = cu_count(resolve_device(index));
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
        const OnDevice scope(device);
        const int index = scope.index();
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
