// Per-device cache of device-memory blocks over a pluggable backend.
//
// The sizing and reuse policy is the one the reference's CNRT allocator
// applies (tensorplay_mlu/csrc/MLUAllocator.cpp:42-45, 98-128, 208-219):
//   * a request is quantized to a multiple of 512 B up to 1 MiB and of
//     2 MiB above;
//   * an idle block is handed out again when it is the smallest idle block
//     of at least the quantized size and at most a quarter larger;
//   * when the backend has no memory left, the device's idle blocks are
//     returned to it (after its queued work has finished) and the request is
//     tried once more;
//   * bytes in use and bytes obtained from the backend, with their peaks,
//     are kept per device.
// The data structure is this file's own: each device keeps its idle blocks
// in size classes -- 2048 fine classes of 512 B, each a LIFO stack, with a
// bitmap of the non-empty ones, and one LIFO stack per 2 MiB multiple above
// 1 MiB in an ordered map -- so a best-fit lookup is a bitmap scan or one
// ordered-map probe.
//
// Every user of a device's memory orders its work on that device's single
// stream, so a block given back by the host may be handed out again at once
// without events.
//
// Recording support: while a recording runs, blocks handed out are stamped
// with the recording's epoch.  Once it has ended, the stamped blocks that are
// idle, and any stamped block given back later, are pinned -- kept out of
// circulation, since every replay still reads and writes them -- until the
// recording is discarded, when the pinned blocks go back to the backend
// and a new epoch starts.  Blocks given back while the recording still runs
// may be handed out again within it: the recorded work keeps its order.
#pragma once

#include <algorithm>
#include <array>
#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace tp_amd {

struct MemoryStats {
    int64_t allocated = 0;  // bytes in blocks handed out
    int64_t reserved = 0;   // bytes obtained from the backend (handed out + idle + pinned)
    int64_t peak_allocated = 0;
    int64_t peak_reserved = 0;
};

constexpr size_t kFineStep = 512;
constexpr size_t kFineLimit = size_t(1) << 20;
constexpr size_t kCoarseStep = size_t(2) << 20;

// The size a request of ``nbytes`` is served with.
inline size_t quantize(size_t nbytes) {
    const size_t step = nbytes <= kFineLimit ? kFineStep : kCoarseStep;
    return (nbytes + step - 1) / step * step;
}

// Where the memory comes from.  ``acquire`` returns nullptr when the device
// is out of memory (any other failure throws); ``drain`` waits until the
// device's queued work has finished.
struct MemoryBackend {
    void* (*acquire)(int device, size_t nbytes, void* ctx);
    void (*release)(int device, void* ptr, void* ctx);
    void (*drain)(int device, void* ctx);
    void* ctx;
};

struct Block {
    void* ptr;
    size_t size;  // quantized
    int device;
    uint64_t epoch = 0;  // recording epoch it was handed out in (0: none)
};

// The idle blocks of one device, by size class.
class IdleBlocks {
public:
    void put(Block* b) {
        if (b->size <= kFineLimit) {
            const size_t c = b->size / kFineStep;
            fine_[c].push_back(b);
            occupied_[c / 64] |= uint64_t(1) << (c % 64);
        } else {
            coarse_[b->size].push_back(b);
        }
        ++count_;
    }

    // The most recently idled block of the smallest class in
    // [size, limit], removed; nullptr when that range is empty.
    Block* pop_fit(size_t size, size_t limit) {
        if (size <= kFineLimit) {
            const size_t last = std::min(limit, kFineLimit) / kFineStep;
            for (size_t c = size / kFineStep; c <= last;) {
                const uint64_t word = occupied_[c / 64] >> (c % 64);
                if (word == 0) {
                    c = (c / 64 + 1) * 64;
                    continue;
                }
                c += static_cast<size_t>(__builtin_ctzll(word));
                if (c > last) break;
                return pop_fine(c);
            }
            if (limit <= kFineLimit) return nullptr;
        }
        auto it = coarse_.lower_bound(std::max(size, kFineLimit + 1));
        if (it == coarse_.end() || it->first > limit) return nullptr;
        Block* b = it->second.back();
        it->second.pop_back();
        if (it->second.empty()) coarse_.erase(it);
        --count_;
        return b;
    }

    // Remove every block for which ``pick(b)`` holds, handing each to
    // ``take(b)``.
    template <typename Pick, typename Take>
    void remove_if(Pick&& pick, Take&& take) {
        for (size_t c = 0; c < fine_.size(); ++c) {
            auto& stack = fine_[c];
            if (stack.empty()) continue;
            sweep(stack, pick, take);
            if (stack.empty()) occupied_[c / 64] &= ~(uint64_t(1) << (c % 64));
        }
        for (auto it = coarse_.begin(); it != coarse_.end();) {
            sweep(it->second, pick, take);
            it = it->second.empty() ? coarse_.erase(it) : std::next(it);
        }
    }

    size_t count() const { return count_; }

private:
    static constexpr size_t kFineClasses = kFineLimit / kFineStep + 1;  // index = size / 512

    Block* pop_fine(size_t c) {
        auto& stack = fine_[c];
        Block* b = stack.back();
        stack.pop_back();
        if (stack.empty()) occupied_[c / 64] &= ~(uint64_t(1) << (c % 64));
        --count_;
        return b;
    }

    template <typename Pick, typename Take>
    void sweep(std::vector<Block*>& stack, Pick& pick, Take& take) {
        size_t kept = 0;
        for (Block* b : stack) {
            if (pick(b)) {
                take(b);
                --count_;
            } else {
                stack[kept++] = b;
            }
        }
        stack.resize(kept);
    }

    std::array<std::vector<Block*>, kFineClasses> fine_;
    std::array<uint64_t, (kFineClasses + 63) / 64> occupied_{};
    std::map<size_t, std::vector<Block*>> coarse_;
    size_t count_ = 0;
};

template <int MaxDevices>
class BlockCache {
public:
    explicit BlockCache(MemoryBackend backend) : backend_(backend) {}

    // A block of at least ``nbytes`` (> 0) on ``device``.  When even a
    // second try at the backend (after its idle blocks went back) finds no
    // memory, throws ``Failure`` built from a message.
    template <typename Failure>
    Block* obtain(int device, size_t nbytes) {
        const size_t size = quantize(nbytes);
        std::lock_guard<std::mutex> lock(mutex_);
        Device& d = devices_.at(device);
        Block* b = d.idle.pop_fit(size, size + size / 4);
        if (b == nullptr) {
            void* ptr = backend_.acquire(device, size, backend_.ctx);
            if (ptr == nullptr) {
                return_idle(device, d);
                ptr = backend_.acquire(device, size, backend_.ctx);
            }
            if (ptr == nullptr) {
                throw Failure("device " + std::to_string(device) + " has no memory left for a " +
                              std::to_string(size) + "-byte block (" + std::to_string(d.ledger.allocated) +
                              " bytes in use, " + std::to_string(d.ledger.reserved - d.ledger.allocated) +
                              " more reserved, cached blocks already returned)");
            }
            b = new Block{ptr, size, device};
            d.ledger.reserved += static_cast<int64_t>(size);
            d.ledger.peak_reserved = std::max(d.ledger.peak_reserved, d.ledger.reserved);
        }
        d.ledger.allocated += static_cast<int64_t>(b->size);
        d.ledger.peak_allocated = std::max(d.ledger.peak_allocated, d.ledger.allocated);
        b->epoch = 0;
        if (stamping_) {
            b->epoch = epoch_;
            ++grants_;
        }
        return b;
    }

    // A block whose last user is gone (nullptr is ignored).
    void recycle(Block* b) {
        if (b == nullptr) return;
        std::lock_guard<std::mutex> lock(mutex_);
        Device& d = devices_.at(b->device);
        d.ledger.allocated -= static_cast<int64_t>(b->size);
        if (b->epoch == epoch_ && !stamping_) {
            pinned_.push_back(b);  // a finished recording still uses it
        } else {
            d.idle.put(b);
        }
    }

    // ---- recording ------------------------------------------------------

    // Start stamping the blocks handed out (with a fresh grant count).
    void begin_stamping() {
        std::lock_guard<std::mutex> lock(mutex_);
        grants_ = 0;
        stamping_ = true;
    }

    void end_stamping() {
        std::lock_guard<std::mutex> lock(mutex_);
        stamping_ = false;
    }

    // Take this epoch's idle blocks out of circulation.
    void pin_epoch() {
        std::lock_guard<std::mutex> lock(mutex_);
        const uint64_t e = epoch_;
        for (Device& d : devices_) {
            d.idle.remove_if([e](const Block* b) { return b->epoch == e; },
                             [this](Block* b) { pinned_.push_back(b); });
        }
    }

    // The recording is gone: once devices [0, ndevices) are idle, the pinned
    // blocks go back to the backend, and a new epoch starts (blocks of the
    // old one still in use return to circulation when given back).
    void retire_epoch(int ndevices) {
        std::lock_guard<std::mutex> lock(mutex_);
        ++epoch_;
        if (pinned_.empty()) return;
        for (int d = 0; d < ndevices && d < MaxDevices; ++d) backend_.drain(d, backend_.ctx);
        for (Block* b : pinned_) {
            backend_.release(b->device, b->ptr, backend_.ctx);
            devices_.at(b->device).ledger.reserved -= static_cast<int64_t>(b->size);
            delete b;
        }
        pinned_.clear();
    }

    int64_t grants() {
        std::lock_guard<std::mutex> lock(mutex_);
        return grants_;
    }

    int64_t pinned() {
        std::lock_guard<std::mutex> lock(mutex_);
        return static_cast<int64_t>(pinned_.size());
    }

    // ---- accounting -----------------------------------------------------

    MemoryStats ledger(int device) {
        std::lock_guard<std::mutex> lock(mutex_);
        return devices_.at(device).ledger;
    }

    void restart_peaks(int device) {
        std::lock_guard<std::mutex> lock(mutex_);
        MemoryStats& l = devices_.at(device).ledger;
        l.peak_allocated = l.allocated;
        l.peak_reserved = l.reserved;
    }

    // Give every idle block of devices [0, ndevices) back to the backend.
    void trim(int ndevices) {
        std::lock_guard<std::mutex> lock(mutex_);
        for (int d = 0; d < ndevices && d < MaxDevices; ++d) return_idle(d, devices_[d]);
    }

    size_t idle_count(int device) {
        std::lock_guard<std::mutex> lock(mutex_);
        return devices_.at(device).idle.count();
    }

private:
    struct Device {
        IdleBlocks idle;
        MemoryStats ledger;
    };

    // Caller holds mutex_.  Queued kernels may still use an idle block, so
    // the device drains first.
    void return_idle(int device, Device& d) {
        if (d.idle.count() == 0) return;
        backend_.drain(device, backend_.ctx);
        d.idle.remove_if([](const Block*) { return true; }, [&](Block* b) {
            backend_.release(device, b->ptr, backend_.ctx);
            d.ledger.reserved -= static_cast<int64_t>(b->size);
            delete b;
        });
    }

    MemoryBackend backend_;
    std::mutex mutex_;
    std::array<Device, MaxDevices> devices_;
    bool stamping_ = false;
    uint64_t epoch_ = 1;
    int64_t grants_ = 0;
    std::vector<Block*> pinned_;
};

}  // namespace tp_amd
