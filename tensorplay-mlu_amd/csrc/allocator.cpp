// hipMalloc-backed instance of the caching allocator and its C entry points
// (replaces tensorplay_mlu/csrc/MLUAllocator.cpp and the allocator part of
// Module.cpp:24-37).

#include "allocator.h"

#include "runtime.h"
#include "tp_amd_runtime.h"

namespace tp_amd {

namespace {

void* hip_allocate(int device, size_t nbytes, void*) {
    DeviceGuard guard(device);
    void* ptr = nullptr;
    const hipError_t status = hipMalloc(&ptr, nbytes);
    if (status == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        return nullptr;
    }
    TP_AMD_HIP_CHECK(status);
    return ptr;
}

void hip_release(int device, void* ptr, void*) {
    DeviceGuard guard(device);
    (void)hipFree(ptr);
}

void hip_wait(int device, void*) { synchronize(device); }

using DeviceAllocator = CachingAllocatorCore<kMaxDevices>;

DeviceAllocator& instance() {
    // Never destroyed: blocks released during process teardown still come
    // back here (MLUAllocator.cpp:222-227).
    static auto* allocator =
        new DeviceAllocator(AllocatorBackend{&hip_allocate, &hip_release, &hip_wait, nullptr});
    return *allocator;
}

}  // namespace

Block* device_alloc(size_t nbytes, int device) {
    const int index = resolve_device(device);
    return instance().take<Error>(index, nbytes);
}

void device_free(Block* block) { instance().give_back(block); }

MemoryStats memory_stats(int device) { return instance().stats(resolve_device(device)); }

void reset_peak_memory_stats(int device) { instance().reset_peak(resolve_device(device)); }

void empty_cache() { instance().empty_cache(device_count()); }

void set_capture_holding(bool on) { instance().set_capture_holding(on); }
void freeze_capture_blocks() { instance().freeze_capture_blocks(); }
void drop_capture_blocks() { instance().drop_capture_blocks(device_count()); }
int64_t capture_allocations() { return instance().capture_allocations(); }
int64_t capture_blocks() { return instance().capture_blocks(); }

}  // namespace tp_amd

using namespace tp_amd;

// Defined by the TensorPlay adapter when it is linked in (csrc/tensorplay/,
// make TENSORPLAY_INCLUDE=...); null otherwise.
extern "C" int tp_amd_tensorplay_register(void) __attribute__((weak));

extern "C" {

void tp_mlu_memory_stats(int index, int64_t* out) {
    const int status = guarded([&] {
        const MemoryStats s = memory_stats(index);
        out[0] = s.allocated;
        out[1] = s.reserved;
        out[2] = s.peak_allocated;
        out[3] = s.peak_reserved;
    });
    if (status != TP_AMD_OK && out != nullptr) out[0] = out[1] = out[2] = out[3] = 0;
}

void tp_mlu_reset_peak_memory_stats(int index) {
    (void)guarded([&] { reset_peak_memory_stats(index); });
}

void tp_mlu_empty_cache(void) {
    (void)guarded([&] { empty_cache(); });
}

int tp_amd_malloc(size_t nbytes, int device, void** ptr, void** ctx) {
    return guarded([&] {
        TP_AMD_CHECK(ptr != nullptr && ctx != nullptr, "tp_amd_malloc: null output");
        *ptr = nullptr;
        *ctx = nullptr;
        if (nbytes == 0) {
            resolve_device(device);
            return;
        }
        Block* block = device_alloc(nbytes, device);
        *ptr = block->ptr;
        *ctx = block;
    });
}

void tp_amd_free(void* ctx) { device_free(static_cast<Block*>(ctx)); }

size_t tp_amd_block_size(void* ctx) {
    return ctx == nullptr ? 0 : static_cast<Block*>(ctx)->size;
}

int tp_mlu_init(void) {
    const int status = guarded([&] {
        // Make the runtime usable and create the streams up front, so the
        // first operator does not pay for it.
        for (int d = 0; d < device_count(); ++d) (void)stream(d);
    });
    if (status != TP_AMD_OK) return 1;
    // Built with the TensorPlay adapter (csrc/tensorplay/), the operators
    // without a device kernel are routed to TensorPlay's host kernels here,
    // as the reference's tp_mlu_init does (Module.cpp:15-22).
    if (tp_amd_tensorplay_register != nullptr && tp_amd_tensorplay_register() != 0) return 1;
    return 0;
}

}  // extern "C"
