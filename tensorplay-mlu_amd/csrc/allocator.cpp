// The hipMalloc-backed block cache and its C entry points (replaces
// tensorplay_mlu/csrc/MLUAllocator.cpp and the allocator part of
// Module.cpp:24-37).

#include "allocator.h"

#include "runtime.h"
#include "tp_amd_runtime.h"

namespace tp_amd {

namespace {

void* hip_acquire(int device, size_t nbytes, void*) {
    const OnDevice scope(device);
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
    const OnDevice scope(device);
    (void)hipFree(ptr);
}

void hip_drain(int device, void*) { synchronize(device); }

using DeviceCache = BlockCache<kMaxDevices>;

DeviceCache& cache() {
    // Never destroyed: tensors that die during process teardown still give
    // their blocks back to it.
    static auto* c = new DeviceCache(MemoryBackend{&hip_acquire, &hip_release, &hip_drain, nullptr});
    return *c;
}

}  // namespace

Block* device_alloc(size_t nbytes, int device) {
    const int index = resolve_device(device);
    return cache().obtain<Error>(index, nbytes);
}

void device_free(Block* block) { cache().recycle(block); }

MemoryStats device_memory(int device) { return cache().ledger(resolve_device(device)); }

void restart_device_peaks(int device) { cache().restart_peaks(resolve_device(device)); }

void return_idle_memory() { cache().trim(device_count()); }

void stamp_recorded_blocks(bool on) {
    if (on) {
        cache().begin_stamping();
    } else {
        cache().end_stamping();
    }
}
void pin_recorded_blocks() { cache().pin_epoch(); }
void release_recorded_blocks() { cache().retire_epoch(device_count()); }
int64_t recorded_grants() { return cache().grants(); }
int64_t pinned_blocks() { return cache().pinned(); }

}  // namespace tp_amd

using namespace tp_amd;

// Defined by the TensorPlay adapter when it is linked in (csrc/tensorplay/,
// make TENSORPLAY_INCLUDE=...); null otherwise.
extern "C" int tp_amd_tensorplay_register(void) __attribute__((weak));

extern "C" {

void tp_mlu_memory_stats(int index, int64_t* out) {
    const int status = guarded([&] {
        const MemoryStats s = device_memory(index);
        out[0] = s.allocated;
        out[1] = s.reserved;
        out[2] = s.peak_allocated;
        out[3] = s.peak_reserved;
    });
    if (status != TP_AMD_OK && out != nullptr) out[0] = out[1] = out[2] = out[3] = 0;
}

void tp_mlu_reset_peak_memory_stats(int index) {
    (void)guarded([&] { restart_device_peaks(index); });
}

void tp_mlu_empty_cache(void) {
    (void)guarded([&] { return_idle_memory(); });
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
        // Open every GPU's slot (its stream and properties) up front, so the
        // first operator does not pay for it.
        open_all_devices();
    });
    if (status != TP_AMD_OK) return 1;
    // Built with the TensorPlay adapter (csrc/tensorplay/), the operators
    // without a device kernel are routed to TensorPlay's host kernels here,
    // as the reference's tp_mlu_init does (Module.cpp:15-22).
    if (tp_amd_tensorplay_register != nullptr && tp_amd_tensorplay_register() != 0) return 1;
    return 0;
}

}  // extern "C"
