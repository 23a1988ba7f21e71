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
#include <vector>
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
    // Handed out while recording number ``recorded`` (0: none) of device
    // work ran: that recording may read or write it on every replay.
    uint64_t recorded = 0;
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
            return note_recorded(block);
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
        return note_recorded(block);
    }

    // A block whose last user is gone.  One handed out during a recording
    // that has ended is set aside instead: the recording still touches it on
    // every replay.  While the recording runs it may be reused, because the
    // recorded work keeps its order.
    void give_back(Block* block) {
        if (block == nullptr) return;
        std::lock_guard<std::mutex> lock(mutex_);
        Pool& pool = pools_.at(block->device);
        pool.stats.allocated -= static_cast<int64_t>(block->size);
        if (block->recorded == generation_ && !holding_) {
            held_.push_back(block);
            return;
        }
        pool.free_blocks.emplace(block->size, block);
    }

    // ---- recording support (the reference's MLUAllocator.cpp:144-201) ----

    // Start (on) or stop marking the blocks handed out.
    void set_capture_holding(bool on) {
        std::lock_guard<std::mutex> lock(mutex_);
        if (on) capture_allocations_ = 0;
        holding_ = on;
    }

    // At the end of a recording: the recorded blocks sitting free in the
    // pools leave them, so nothing else is handed memory the replays use.
    void freeze_capture_blocks() {
        std::lock_guard<std::mutex> lock(mutex_);
        for (Pool& pool : pools_) {
            for (auto it = pool.free_blocks.begin(); it != pool.free_blocks.end();) {
                if (it->second->recorded == generation_) {
                    held_.push_back(it->second);
                    it = pool.free_blocks.erase(it);
                } else {
                    ++it;
                }
            }
        }
    }

    // After the recording is dropped: the blocks set aside go back to the
    // backend (once the devices [0, ndevices) are idle), and blocks of that
    // recording still in use return to the pool as usual when freed.
    void drop_capture_blocks(int ndevices) {
        std::lock_guard<std::mutex> lock(mutex_);
        ++generation_;
        if (held_.empty()) return;
        for (int d = 0; d < ndevices && d < MaxDevices; ++d) backend_.wait(d, backend_.state);
        for (Block* block : held_) {
            backend_.release(block->device, block->ptr, backend_.state);
            pools_.at(block->device).stats.reserved -= static_cast<int64_t>(block->size);
            delete block;
        }
        held_.clear();
    }

    // Blocks handed out since the last set_capture_holding(true).
    int64_t capture_allocations() {
        std::lock_guard<std::mutex> lock(mutex_);
        return capture_allocations_;
    }

    // Blocks set aside for a recording.
    int64_t capture_blocks() {
        std::lock_guard<std::mutex> lock(mutex_);
        return static_cast<int64_t>(held_.size());
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

    // Caller holds mutex_.
    Block* note_recorded(Block* block) {
        if (holding_) {
            block->recorded = generation_;
            ++capture_allocations_;
        }
        return block;
    }

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
    bool holding_ = false;
    uint64_t generation_ = 1;  // number of the current (or next) recording
    int64_t capture_allocations_ = 0;
    std::vector<Block*> held_;
};

}  // namespace tp_amd
