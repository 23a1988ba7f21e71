#pragma once
// Declarations of TensorPlay's profiler hooks as the reference uses them
// (tensorplay_mlu/csrc/MLUProfiler.cpp:20-80, MLUActivity.cpp:87-258), for
// the adapter's syntax check; nothing here is linked.
#include <cstdint>
#include <string>
#include <vector>

namespace tensorplay {
namespace prof {

class DeviceTimerHooks {
public:
    virtual ~DeviceTimerHooks() = default;
    virtual int current_device() const = 0;
    virtual void* record(int device) const = 0;
    virtual bool elapsed_ms(void* start, void* end, float* ms) const = 0;
    virtual void release(void* event) const = 0;
};
void register_privateuse1_timer_hooks(const DeviceTimerHooks* hooks);

struct GpuActivity {
    static constexpr uint64_t kNoExt = ~uint64_t{0};
    const char* name;
    char kind;
    uint64_t start_ns;
    uint64_t end_ns;
    uint64_t external_id;
    int32_t device;
    int32_t stream;
    uint64_t bytes;
    uint8_t copy_kind;
    uint32_t correlation;
};

class DeviceActivityHooks {
public:
    virtual ~DeviceActivityHooks() = default;
    virtual bool start() = 0;
    virtual void stop_and_collect(std::vector<GpuActivity>& out) = 0;
    virtual void push_external_id(uint64_t id) = 0;
    virtual void pop_external_id() = 0;
    virtual std::string last_error() const = 0;
};
void register_privateuse1_activity_hooks(DeviceActivityHooks* hooks);

}  // namespace prof
}  // namespace tensorplay
