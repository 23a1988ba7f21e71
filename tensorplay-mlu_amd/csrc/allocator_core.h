// Size-bucketed caching allocator, independent of the memory it manages.
//
// Restates the policy of the reference's CNRT caching allocator
// (tensorplay_mlu/csrc/MLUAllocator.cpp:37-236) over a pluggable backend, so
// the HIP instance (allocator.cpp) and a host-memory instance used by the
// CPU tests share one implementation:
//   * sizes round up to 512 B at or below 1 MiB and to 2 MiB above (:42-45);
//   * a free block is reused when it is the smallest one at least the
//     rounded size and no more than a quarter larger (:98-106);
//   * when the backend is out of memory the device's cache is released and
//     the allocation retried once; a second failure is an error carrying
//     the device's statistics (:111-121);
//   * allocated / reserved bytes and their peaks per device (:75-85).
// Blocks are reused without events: every user of a device's memory orders
// its work on that device's single stream (:1-6), so a block freed by the
// host may be handed out at once.  Releasing cached blocks to the backend
// first waits for the stream (:208-219).
#pragma once

#include <algorithm>
#include <array>
#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>

namespace tp_amd {

struct MemoryStats {
    int64_t allocated = 0;  // bytes held by live blocks
    int64_t reserved = 0;   // bytes obtained from the backend (live + cached)
    int64_t peak_allocated = 0;
    int64_t peak_reserved = 0;
};

constexpr size_t kSmallLimit = size_t(1) << 20;
constexpr size_t kSmallRound = 512;
constexpr size_t kLargeRound = size_t(2) << 20;

inline size_t round_size(size_t nbytes) {
    if (nbytes <= kSmallLimit) return (nbytes + kSmallRound - 1) / kSmallRound * kSmallRound;
    return (nbytes + kLargeRound - 1) / kLargeRound * kLargeRound;
}

// Backend contract: ``allocate`` returns nullptr when out of memory (other
// failures throw), ``release`` returns memory, ``wait`` blocks until the
// device's queued work is done.
struct AllocatorBackend {
    void* (*allocate)(int device, size_t nbytes, void* state);
    void (*release)(int device, void* ptr, void* state);
    void (*wait)(int device, void* state);
    void* state;
};

struct Block {
    void* ptr;
    size_t size;
    int device;
};

template <int MaxDevices>
class CachingAllocatorCore {
public:
    explicit CachingAllocatorCore(AllocatorBackend backend) : backend_(backend) {}

    // A block of at least ``nbytes`` (nbytes > 0) on ``device``.  Throws
    // ``OomError`` (constructed from a message) when the retry fails too.
    template <typename OomError>
    Block* take(int device, size_t nbytes) {
        const size_t size = round_size(nbytes);
        std::lock_guard<std::mutex> lock(mutex_);
        Pool& pool = pools_.at(device);
        auto it = pool.free_blocks.lower_bound(size);
        if (it != pool.free_blocks.end() && it->first <= size + size / 4) {
            Block* block = it->second;
            pool.free_blocks.erase(it);
            note_allocated(pool, block->size);
            return block;
        }
        void* ptr = backend_.allocate(device, size, backend_.state);
        if (ptr == nullptr) {
            release_cached_locked(device);
            ptr = backend_.allocate(device, size, backend_.state);
            if (ptr == nullptr) {
                throw OomError("out of memory allocating " + std::to_string(size) +
                               " bytes on device " + std::to_string(device) + " (" +
                               std::to_string(pool.stats.allocated) + " bytes allocated, " +
                               std::to_string(pool.stats.reserved) +
                               " reserved by the cache)");
            }
        }
        pool.stats.reserved += static_cast<int64_t>(size);
        pool.stats.peak_reserved = std::max(pool.stats.peak_reserved, pool.stats.reserved);
        Block* block = new Block{ptr, size, device};
        note_allocated(pool, size);
        return block;
    }

    void give_back(Block* block) {
        if (block == nullptr) return;
        std::lock_guard<std::mutex> lock(mutex_);
        Pool& pool = pools_.at(block->device);
        pool.stats.allocated -= static_cast<int64_t>(block->size);
        pool.free_blocks.emplace(block->size, block);
    }

    MemoryStats stats(int device) {
        std::lock_guard<std::mutex> lock(mutex_);
        return pools_.at(device).stats;
    }

    void reset_peak(int device) {
        std::lock_guard<std::mutex> lock(mutex_);
        MemoryStats& s = pools_.at(device).stats;
        s.peak_allocated = s.allocated;
        s.peak_reserved = s.reserved;
    }

    // Return every cached block of devices [0, ndevices) to the backend.
    void empty_cache(int ndevices) {
        std::lock_guard<std::mutex> lock(mutex_);
        for (int d = 0; d < ndevices && d < MaxDevices; ++d) release_cached_locked(d);
    }

    size_t cached_blocks(int device) {
        std::lock_guard<std::mutex> lock(mutex_);
        return pools_.at(device).free_blocks.size();
    }

private:
    struct Pool {
        std::multimap<size_t, Block*> free_blocks;
        MemoryStats stats;
    };

    static void note_allocated(Pool& pool, size_t size) {
        pool.stats.allocated += static_cast<int64_t>(size);
        pool.stats.peak_allocated = std::max(pool.stats.peak_allocated, pool.stats.allocated);
    }

    // Caller holds mutex_.  Waits for the device first so no queued kernel
    // still touches a block that goes back to the backend.
    void release_cached_locked(int device) {
        Pool& pool = pools_.at(device);
        if (pool.free_blocks.empty()) return;
        backend_.wait(device, backend_.state);
        for (auto& entry : pool.free_blocks) {
            backend_.release(device, entry.second->ptr, backend_.state);
            pool.stats.reserved -= static_cast<int64_t>(entry.first);
            delete entry.second;
        }
        pool.free_blocks.clear();
    }

    AllocatorBackend backend_;
    std::mutex mutex_;
    std::array<Pool, MaxDevices> pools_;
};

}  // namespace tp_amd
