// Host-memory instance of the device block cache, for the CPU tests: the
// same code (block_cache.h) over malloc with an injectable capacity, so
// quantization, reuse, statistics, the out-of-memory retry and the
// recording epochs can be checked without a GPU.
#include <cstdlib>
#include <map>
#include <stdexcept>

#include "../../tensorplay-mlu_amd/csrc/block_cache.h"

namespace {

struct HostState {
    size_t cap = 0;       // bytes the fake device holds
    size_t used = 0;
    long allocs = 0, frees = 0, waits = 0;
    std::map<void*, size_t> live;
};

HostState g_state;

void* host_alloc(int, size_t n, void* s) {
    HostState* st = static_cast<HostState*>(s);
    if (st->used + n > st->cap) return nullptr;
    st->used += n;
    ++st->allocs;
    void* p = std::malloc(n);
    st->live[p] = n;
    return p;
}

void host_release(int, void* p, void* s) {
    HostState* st = static_cast<HostState*>(s);
    ++st->frees;
    st->used -= st->live[p];
    st->live.erase(p);
    std::free(p);
}

void host_wait(int, void* s) { ++static_cast<HostState*>(s)->waits; }

using Core = tp_amd::BlockCache<4>;
Core* g_core = nullptr;

struct Oom : std::runtime_error {
    explicit Oom(const std::string& m) : std::runtime_error(m) {}
};

}  // namespace

extern "C" {

void shim_reset(size_t cap) {
    delete g_core;
    g_state = HostState{};
    g_state.cap = cap;
    g_core = new Core(tp_amd::MemoryBackend{&host_alloc, &host_release, &host_wait, &g_state});
}

size_t shim_round(size_t n) { return tp_amd::quantize(n); }

// Returns the block (or NULL after an out-of-memory error).
void* shim_take(int dev, size_t n) {
    try {
        return g_core->obtain<Oom>(dev, n);
    } catch (const Oom&) {
        return nullptr;
    }
}

size_t shim_block_size(void* b) { return static_cast<tp_amd::Block*>(b)->size; }
void* shim_block_ptr(void* b) { return static_cast<tp_amd::Block*>(b)->ptr; }
void shim_give(void* b) { g_core->recycle(static_cast<tp_amd::Block*>(b)); }

void shim_stats(int dev, long long* out) {
    const tp_amd::MemoryStats s = g_core->ledger(dev);
    out[0] = s.allocated;
    out[1] = s.reserved;
    out[2] = s.peak_allocated;
    out[3] = s.peak_reserved;
}

void shim_reset_peak(int dev) { g_core->restart_peaks(dev); }
void shim_empty(void) { g_core->trim(4); }
size_t shim_cached(int dev) { return g_core->idle_count(dev); }

void shim_capture_holding(int on) {
    if (on) {
        g_core->begin_stamping();
    } else {
        g_core->end_stamping();
    }
}
void shim_freeze(void) { g_core->pin_epoch(); }
void shim_drop(void) { g_core->retire_epoch(4); }
void shim_capture_stats(long long* out) {
    out[0] = g_core->grants();
    out[1] = g_core->pinned();
}

void shim_counts(long* out) {
    out[0] = g_state.allocs;
    out[1] = g_state.frees;
    out[2] = g_state.waits;
    out[3] = static_cast<long>(g_state.used);
}

}  // extern "C"
