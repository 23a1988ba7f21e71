// Device time for TensorPlay's profiler (reference MLUProfiler.cpp:20-80 and
// MLUActivity.cpp:87-258) over the library's profiler entries:
//
// * Timer hooks: a pooled HIP event on the device's stream before and after
//   each operation (tp_amd_timer_*), so profile(use_device="mlu") reports
//   per-operation device time.
// * Activity hooks: the kernels and copies of a session from rocprofiler-sdk
//   (tp_amd_activity_*), each joined to its operation through the record
//   slot the dispatcher pushes as the external correlation id.  Tracing is
//   there when the process starts with TP_AMD_DEVICE_TRACE=1; otherwise
//   start() fails with the reason and a session reports per-operation
//   device time only, as the reference does without its activity library.

#include <mutex>
#include <string>
#include <vector>

#include "Adapter.h"
#include "Profiler.h"

namespace tensorplay {
namespace amd {

namespace {

class EventTimer final : public prof::DeviceTimerHooks {
public:
    int current_device() const override {
        int index = 0;
        return tp_amd_current_device(&index) == TP_AMD_OK ? index : 0;
    }

    void* record(int device) const override {
        void* marker = nullptr;
        return tp_amd_timer_record(device, &marker) == TP_AMD_OK ? marker : nullptr;
    }

    bool elapsed_ms(void* start, void* end, float* ms) const override {
        return tp_amd_timer_elapsed_ms(start, end, ms) == TP_AMD_OK;
    }

    void release(void* event) const override { tp_amd_timer_release(event); }
};

class RocprofilerCollector final : public prof::DeviceActivityHooks {
public:
    bool start() override {
        std::lock_guard<std::mutex> lock(mutex_);
        if (tp_amd_activity_start() == TP_AMD_OK) return true;
        error_ = tp_mlu_last_error();
        return false;
    }

    void stop_and_collect(std::vector<prof::GpuActivity>& out) override {
        std::lock_guard<std::mutex> lock(mutex_);
        const tp_amd_activity* records = nullptr;
        size_t count = 0;
        if (tp_amd_activity_stop(&records, &count) != TP_AMD_OK) {
            error_ = tp_mlu_last_error();
            return;
        }
        // The names stay valid until the next start(), as the profiler
        // expects of kernel names.
        for (size_t i = 0; i < count; ++i) {
            const tp_amd_activity& r = records[i];
            prof::GpuActivity a{};
            a.name = r.name;
            a.kind = r.kind;
            a.start_ns = r.start_ns;
            a.end_ns = r.end_ns;
            a.external_id = r.external_id == TP_AMD_NO_EXTERNAL ? prof::GpuActivity::kNoExt : r.external_id;
            a.device = r.device;
            a.stream = r.stream;
            a.bytes = r.bytes;
            a.copy_kind = r.copy_kind;
            a.correlation = r.correlation;
            out.push_back(a);
        }
    }

    void push_external_id(uint64_t id) override { tp_amd_activity_push_external(id); }

    void pop_external_id() override { tp_amd_activity_pop_external(); }

    std::string last_error() const override {
        std::lock_guard<std::mutex> lock(mutex_);
        return error_.empty() ? std::string(tp_amd_activity_error()) : error_;
    }

private:
    mutable std::mutex mutex_;
    std::string error_;
};

// Leaked: the profiler may still hold them while the process exits.
[[maybe_unused]] const bool registered = [] {
    prof::register_privateuse1_timer_hooks(new EventTimer);
    prof::register_privateuse1_activity_hooks(new RocprofilerCollector);
    return true;
}();

}  // namespace

}  // namespace amd
}  // namespace tensorplay
