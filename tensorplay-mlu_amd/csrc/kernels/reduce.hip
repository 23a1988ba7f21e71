// Reductions for gfx950: sum, mean, amax, amin of a dense [outer, r, inner]
// array along the middle axis (the reference's cnnlReduce_v2,
// tensorplay_mlu/csrc/ReduceKernels.cpp:21-44).
//
// * inner == 1 (row reductions): a wavefront (or, for long rows, a whole
//   block) reduces one row segment with 16-byte packet loads, then combines
//   across lanes with DPP/shuffle steps and across waves in LDS.  When there
//   are too few rows to fill 256 CUs (a whole-tensor sum), rows are split
//   into segments of one block each, and the last block of a row to finish
//   folds the row's float32 partials in the same launch.
// * inner > 1 (column reductions, e.g. dim 0 of [32768, 4096]): lanes walk
//   the contiguous inner axis with packets, four row groups per block share
//   the rows of a chunk, and chunks of rows are spread over the grid; the
//   last block of a column range folds the chunk partials in the same launch.
// Arithmetic is float32.  amax/amin skip NaN inputs and order -0 below +0,
// so every evaluation order gives the same bits.

#include <cmath>

#include <climits>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "device_common.h"
#include "../allocator.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kBlock = 256;

template <int OP>
struct Combine;

template <>
struct Combine<TP_AMD_REDUCE_SUM> {
    __device__ __forceinline__ static float identity() { return 0.0f; }
    __device__ __forceinline__ static float apply(float a, float b) { return a + b; }
};
template <>
struct Combine<TP_AMD_REDUCE_MEAN> : Combine<TP_AMD_REDUCE_SUM> {};
template <>
struct Combine<TP_AMD_REDUCE_AMAX> {
    __device__ __forceinline__ static float identity() { return __uint_as_float(0x7fc00000u); }
    __device__ __forceinline__ static float apply(float a, float b) {
        if (a != a) return b;
        if (b != b) return a;
        if (a == b) return (__float_as_uint(a) & 0x80000000u) ? b : a;  // +0 over -0
        return a > b ? a : b;
    }
};
template <>
struct Combine<TP_AMD_REDUCE_AMIN> {
    __device__ __forceinline__ static float identity() { return __uint_as_float(0x7fc00000u); }
    __device__ __forceinline__ static float apply(float a, float b) {
        if (a != a) return b;
        if (b != b) return a;
        if (a == b) return (__float_as_uint(a) & 0x80000000u) ? a : b;  // -0 over +0
        return a < b ? a : b;
    }
};

template <int OP>
__device__ __forceinline__ float wave_reduce(float v) {
    return wave_allreduce(v, [](float a, float b) { return Combine<OP>::apply(a, b); });
}

// ---- amax / amin on order-preserving integer keys -------------------------------
//
// Flipping the magnitude bits of negative values maps the float order
// (with -0 below +0) onto the signed integer order: key(u) = u ^ ((u >> 31) &
// 0x7fff...), an involution.  NaNs map beyond +-inf, so an integer max / min
// gives the exact amax / amin unless a NaN wins; a thread whose result comes
// out NaN (a NaN among its elements, or no elements) recomputes its elements
// with the NaN-skipping float combine.  For 16-bit storage two keys share a
// register and one packed v_pk_max_i16 / v_pk_min_i16 covers both.
template <int OP>
constexpr bool kMinMax = OP == TP_AMD_REDUCE_AMAX || OP == TP_AMD_REDUCE_AMIN;

typedef short short2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int32_t key32(uint32_t u) {
    return static_cast<int32_t>(u ^ (static_cast<uint32_t>(static_cast<int32_t>(u) >> 31) &
                                     0x7fffffffu));
}
__device__ __forceinline__ short2_t key16x2(uint32_t w) {
    short2_t h;
    __builtin_memcpy(&h, &w, 4);
    const short2_t m = (h >> static_cast<short>(15)) & static_cast<short>(0x7fff);
    return h ^ m;
}

template <int OP>
struct KeyOps {
    static constexpr bool kMax = OP == TP_AMD_REDUCE_AMAX;
    // The identity is the key no value beats; it decodes to a NaN, so an
    // empty thread falls back to the float combine (which returns NaN too).
    __device__ __forceinline__ static int32_t id32() { return kMax ? INT32_MIN : INT32_MAX; }
    __device__ __forceinline__ static short id16() {
        return kMax ? static_cast<short>(-32768) : static_cast<short>(32767);
    }
    __device__ __forceinline__ static int32_t pick(int32_t a, int32_t b) {
        return kMax ? (a > b ? a : b) : (a < b ? a : b);
    }
    __device__ __forceinline__ static short2_t pick(short2_t a, short2_t b) {
        return kMax ? __builtin_elementwise_max(a, b) : __builtin_elementwise_min(a, b);
    }
    // Float value of a 32-bit key.
    __device__ __forceinline__ static float value32(int32_t k) {
        const uint32_t u = static_cast<uint32_t>(k);
        return __uint_as_float(u ^ (static_cast<uint32_t>(k >> 31) & 0x7fffffffu));
    }
    // Float value of the better of a pair of 16-bit keys.
    template <typename Tin>
    __device__ __forceinline__ static float value16(short2_t k) {
        const short b = kMax ? (k.x > k.y ? k.x : k.y) : (k.x < k.y ? k.x : k.y);
        const uint16_t u = static_cast<uint16_t>(b) ^ (b < 0 ? 0x7fffu : 0u);
        return Elem<Tin>::load(u);
    }
};

// Reduction across the wave.  amax / amin reduce the order-preserving keys
// with integer max / min -- a lane holding NaN (no elements, or only NaNs)
// takes the key that loses -- and decode the winner; sums add floats.
template <int OP>
__device__ __forceinline__ float lane_reduce(float v) {
    if constexpr (kMinMax<OP>) {
        using K = KeyOps<OP>;
        const int32_t k = v != v ? K::id32() : key32(__float_as_uint(v));
        const float r = wave_allreduce(__int_as_float(k), [](float a, float b) {
            return __int_as_float(K::pick(__float_as_int(a), __float_as_int(b)));
        });
        const int32_t kr = __float_as_int(r);
        return kr == K::id32() ? Combine<OP>::identity() : K::value32(kr);
    } else {
        return wave_reduce<OP>(v);
    }
}

// Final value of a reduction: the mean divides the float32 sum by the
// number of reduced elements.
template <int OP>
__device__ __forceinline__ float finish(float v, int64_t count, bool final_pass) {
    if constexpr (OP == TP_AMD_REDUCE_MEAN) {
        if (final_pass) return v / static_cast<float>(count);
    }
    return v;
}

// A packet of one repeated 32-bit word (the padding of partial batches).
__device__ __forceinline__ uint4 splat(uint32_t w) { return make_uint4(w, w, w, w); }

// One thread's share of packets [pb, pe) of a row segment: packets
// pb + tid, pb + tid + THREADS, ...  Loads go out in batches of U (4 by default), the
// batch's out-of-range slots padded with a value that leaves the result
// unchanged, so every batch's loads are in flight together.  Float combine
// in element order.
// NT: non-temporal loads (the default for rows streamed once); false keeps
// the default policy, under which a tensor the previous kernel left in the
// 256 MB Infinity Cache is read from there.
template <typename Tin, int OP, int THREADS, int U = 4, bool NT = true>
__device__ __forceinline__ float row_exact(const typename Elem<Tin>::storage* p, int64_t pb,
                                           int64_t pe, int tid) {
    constexpr int N = Packet<Tin>::N;
    // Zeros add nothing; NaN is skipped by amax / amin.
    constexpr uint32_t kPad = kMinMax<OP> ? (N == 4 ? 0x7fc00000u : (std::is_same_v<Tin, bf16_t>
                                                                          ? 0x7fc07fc0u
                                                                          : 0x7e007e00u))
                                          : 0u;
    float acc = Combine<OP>::identity();
    for (int64_t q0 = pb + tid; q0 < pe; q0 += static_cast<int64_t>(U) * THREADS) {
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t q = q0 + static_cast<int64_t>(u) * THREADS;
            raw[u] = q < pe ? (NT ? load_raw_nt(p + q * N) : *reinterpret_cast<const uint4*>(p + q * N))
                            : splat(kPad);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v[N];
            unpack<Tin>(raw[u], v);
#pragma unroll
            for (int j = 0; j < N; ++j) acc = Combine<OP>::apply(acc, v[j]);
        }
    }
    return acc;
}

// The same share for amax / amin on integer keys (NaN when a NaN wins or the
// share is empty).  The padding is the NaN pattern whose key loses to every
// value.
template <typename Tin, int OP, int THREADS, int U = 4, bool NT = true>
__device__ __forceinline__ float row_keys(const typename Elem<Tin>::storage* p, int64_t pb,
                                          int64_t pe, int tid) {
    constexpr int N = Packet<Tin>::N;
    using K = KeyOps<OP>;
    constexpr bool kWide = sizeof(typename Elem<Tin>::storage) == 4;
    constexpr uint32_t kPad = K::kMax ? 0xffffffffu : (kWide ? 0x7fffffffu : 0x7fff7fffu);
    int32_t k32 = K::id32();
    short2_t k16 = {K::id16(), K::id16()};
    for (int64_t q0 = pb + tid; q0 < pe; q0 += static_cast<int64_t>(U) * THREADS) {
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t q = q0 + static_cast<int64_t>(u) * THREADS;
            raw[u] = q < pe ? (NT ? load_raw_nt(p + q * N) : *reinterpret_cast<const uint4*>(p + q * N))
                            : splat(kPad);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (kWide) k32 = K::pick(k32, key32(w[i]));
                else k16 = K::pick(k16, key16x2(w[i]));
            }
        }
    }
    if constexpr (kWide) return K::value32(k32);
    else return K::template value16<Tin>(k16);
}

// Row segments.  Segment s covers row s / nseg, elements
// [(s % nseg) * chunk, min(r, ... + chunk)).  WAVES wavefronts share one
// segment (1: each wave of the block takes its own segment).
template <typename Tin, typename Tout, int OP, int WAVES, bool VEC>
__global__ __launch_bounds__(kBlock) void reduce_rows_kernel(
    const typename Elem<Tin>::storage* x, typename Elem<Tout>::storage* out, int64_t nsegs,
    int64_t r, int64_t chunk, int64_t nseg, bool final_pass, int64_t count) {
    constexpr int N = VEC ? Packet<Tin>::N : 1;
    constexpr int kSegsPerBlock = (kBlock / kWave) / WAVES;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t seg = static_cast<int64_t>(blockIdx.x) * kSegsPerBlock + wave / WAVES;
    const int tid = (wave % WAVES) * kWave + lane;  // thread index within the segment
    constexpr int kThreads = WAVES * kWave;
    float acc = Combine<OP>::identity();
    if (seg < nsegs) {
        const int64_t row = seg / nseg, part = seg - row * nseg;
        const int64_t begin = part * chunk;
        const int64_t end = begin + chunk < r ? begin + chunk : r;
        const typename Elem<Tin>::storage* p = x + row * r;
        if constexpr (VEC) {
            // begin and end are multiples of N (chunk and r are).
            const int64_t pb = begin / N, pe = end / N;
            if constexpr (kMinMax<OP>) {
                acc = row_keys<Tin, OP, kThreads>(p, pb, pe, tid);
                if (acc != acc) acc = row_exact<Tin, OP, kThreads>(p, pb, pe, tid);
            } else {
                acc = row_exact<Tin, OP, kThreads>(p, pb, pe, tid);
            }
        } else {
            for (int64_t j = begin + tid; j < end; j += kThreads) {
                acc = Combine<OP>::apply(acc, Elem<Tin>::load(p[j]));
            }
        }
    }
    acc = lane_reduce<OP>(acc);
    if constexpr (WAVES > 1) {
        __shared__ float partial[kBlock / kWave];
        if (lane == 0) partial[wave] = acc;
        __syncthreads();
        if (wave == 0) {
            acc = lane < WAVES ? partial[lane] : Combine<OP>::identity();
            acc = lane_reduce<OP>(acc);
        }
        if (threadIdx.x == 0 && seg < nsegs) {
            out[seg] = Elem<Tout>::store(finish<OP>(acc, count, final_pass));
        }
    } else {
        if (lane == 0 && seg < nsegs) out[seg] = Elem<Tout>::store(finish<OP>(acc, count, final_pass));
    }
}

// The value of `v` over a block of BLOCK threads (combined over its waves
// in wave order), in thread 0.
template <int OP, int BLOCK = kBlock>
__device__ __forceinline__ float block_reduce(float v) {
    __shared__ float waves[BLOCK / kWave];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    v = lane_reduce<OP>(v);
    if (lane == 0) waves[wave] = v;
    __syncthreads();
    if (wave == 0) {
        v = lane < BLOCK / kWave ? waves[lane] : Combine<OP>::identity();
        v = lane_reduce<OP>(v);
    }
    return v;
}

// Arrival counters of the one-launch folds.  Agent-scope atomics on one
// 128-byte line serialize (measured: 2048 arrivals on one counter add about
// 20 us to a 15 us kernel, 64 arrivals on each of 32 counters on separate
// lines add nothing measurable, the same 32 counters packed on one line add
// 11 us), so every counter has a line of its own.
constexpr int kCounterStride = 32;  // uint32 slots per 128-byte line

// Few long rows (a whole-tensor sum, a loss over all logits): each row is
// split into nseg segments, one block of fused_threads() a segment, and the
// partials are folded in the same launch.  Block s reduces segment s (row s / nseg,
// elements [(s % nseg) * chunk, +chunk)), stores its float32 partial with an
// agent-coherent store, waits for the store to complete, and counts its
// arrival on its group's counter (kFoldGroup consecutive segments of the
// row, so that no counter sees more than kFoldGroup arrivals).  When the row
// has several groups, each group's last arrival then counts the group on the
// row's counter.  The row's last arrival reads all nseg partials back with
// agent-coherent loads and folds them in a fixed order (thread t takes
// partials t, t + blockDim, ... in turn, then the block combines its lanes and
// waves in order), so the bits do not depend on which block came last, and
// writes the result.  Each counter is reset by its last arrival for the next
// launch (device globals start zeroed when the code object loads).
//
// Ordering: the fold relies on gfx950's memory system, not on a C++ release
// / acquire pair.  An agent-scope store is issued with sc1 set and written
// through to the device-coherent level (past the non-coherent per-XCD L2),
// and s_waitcnt vmcnt(0) returns only once that write is acknowledged; the
// counter's atomic add is issued after it, and the agent-scope loads of the
// last block (sc1 set) read the coherent level.  An agent-scope release
// would instead write back this XCD's whole L2 in every block.  Other
// targets are refused at compile time rather than trusted to behave alike.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the one-launch reduction folds rely on gfx950's write-through ordering"
#endif
constexpr int kFoldGroup = 64;
constexpr int64_t kMaxFoldGroups = 8192;
constexpr int64_t kMaxFoldRows = 4096;
__device__ unsigned int group_counters[kMaxFoldGroups * kCounterStride];
__device__ unsigned int row_counters[kMaxFoldRows * kCounterStride];

// Threads of a fused-fold block, and such blocks a CU (segments_per_cu):
// 1024 threads a CU either way.  Measured on whole 4096^2 tensors, averages of
// 20 calls back to back: float32 sum 10.5 us as two 512-thread blocks a CU,
// against 10.8 (two of 256), 11.9 (one of 512 or of 1024), 11.3 (four of
// 256); bf16 sum 5.7 us as one 1024-thread block, 5.7 (two of 512), 5.9 (one
// of 512), 6.1 (two of 256), 6.7 (two of 1024); bf16 amax 6.0-6.1 us as one
// 1024-thread block against 6.5 (two of 256).
template <typename Tin>
constexpr int fused_threads() {
    return sizeof(typename Elem<Tin>::storage) == 4 ? 512 : 1024;
}
constexpr int64_t segments_per_cu(int64_t packet) { return packet == 4 ? 2 : 1; }

template <typename Tin, int OP, bool VEC, int BLOCK = fused_threads<Tin>()>
__global__ __launch_bounds__(BLOCK) void reduce_rows_fused_kernel(
    const typename Elem<Tin>::storage* x, typename Elem<Tin>::storage* out, float* partial,
    int64_t r, int64_t chunk, int64_t nseg, int64_t ngroups) {
    constexpr int N = VEC ? Packet<Tin>::N : 1;
    const int64_t seg = blockIdx.x;
    const int64_t row = seg / nseg, part = seg - row * nseg;
    const int64_t begin = part * chunk;
    const int64_t end = begin + chunk < r ? begin + chunk : r;
    const typename Elem<Tin>::storage* p = x + row * r;
    const int tid = threadIdx.x;
    float acc = Combine<OP>::identity();
    if constexpr (VEC) {
        // 16-bit tensors load with the default policy, float32 ones
        // non-temporally.  Measured on whole 4096^2 tensors called back to
        // back: bf16 sum 5.86 us against 8.32 us non-temporal (the 32 MiB
        // are served from the Infinity Cache), float32 11.0 us against
        // 12.6 us with the default policy.
        constexpr bool kNt = sizeof(typename Elem<Tin>::storage) == 4;
        const int64_t pb = begin / N, pe = end / N;
        if constexpr (kMinMax<OP>) {
            acc = row_keys<Tin, OP, BLOCK, 8, kNt>(p, pb, pe, tid);
            if (acc != acc) acc = row_exact<Tin, OP, BLOCK, 8, kNt>(p, pb, pe, tid);
        } else {
            acc = row_exact<Tin, OP, BLOCK, 8, kNt>(p, pb, pe, tid);
        }
    } else {
        for (int64_t j = begin + tid; j < end; j += BLOCK) {
            acc = Combine<OP>::apply(acc, Elem<Tin>::load(p[j]));
        }
    }
    acc = block_reduce<OP, BLOCK>(acc);
    // The block's group of segments, and that group's slot among the row's.
    const int64_t group = part / kFoldGroup;
    const int64_t first = group * kFoldGroup;
    const int64_t gsize = nseg - first < kFoldGroup ? nseg - first : kFoldGroup;
    const int64_t gslot = row * ngroups + group;
    __shared__ bool last;
    if (tid == 0) {
        __hip_atomic_store(&partial[seg], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        bool done = __hip_atomic_fetch_add(&group_counters[gslot * kCounterStride], 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) == gsize - 1;
        if (done && ngroups > 1) {
            // The group's last arrival: its partials are all stored; count the
            // group on the row's counter.
            __hip_atomic_store(&group_counters[gslot * kCounterStride], 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            done = __hip_atomic_fetch_add(&row_counters[row * kCounterStride], 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == ngroups - 1;
            if (done) {
                __hip_atomic_store(&row_counters[row * kCounterStride], 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        } else if (done) {
            __hip_atomic_store(&group_counters[gslot * kCounterStride], 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        last = done;
    }
    __syncthreads();
    if (!last) return;
    // Every segment of the row has stored its partial: fold them in order,
    // thread t taking partials t, t + 256, ...
    const float* q = partial + row * nseg;
    float v = Combine<OP>::identity();
    for (int64_t k = tid; k < nseg; k += BLOCK) {
        v = Combine<OP>::apply(v, __hip_atomic_load(q + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    v = block_reduce<OP, BLOCK>(v);
    if (tid == 0) out[row] = Elem<Tin>::store(finish<OP>(v, r, true));
}

// amax / amin of one thread's N columns over rows row0, row0 + G, ... < end
// on integer keys (a column comes out NaN when a NaN wins or it has no rows).
template <typename Tin, int OP, int G, bool NT>
__device__ __forceinline__ void cols_keys(float (&acc)[Packet<Tin>::N],
                                          const typename Elem<Tin>::storage* p, int64_t row0,
                                          int64_t end, int64_t inner) {
    constexpr int U = 8;
    using K = KeyOps<OP>;
    constexpr bool kWide = sizeof(typename Elem<Tin>::storage) == 4;
    int32_t k32[4];
    short2_t k16[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        k32[i] = K::id32();
        k16[i] = short2_t{K::id16(), K::id16()};
    }
    auto take = [&](const uint4& raw) {
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (kWide) k32[i] = K::pick(k32[i], key32(w[i]));
            else k16[i] = K::pick(k16[i], key16x2(w[i]));
        }
    };
    int64_t row = row0;
    for (; row + (U - 1) * G < end; row += U * G) {
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const auto* q = p + (row + u * G) * inner;
            raw[u] = NT ? load_raw_nt(q) : *reinterpret_cast<const uint4*>(q);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) take(raw[u]);
    }
    for (; row < end; row += G) take(*reinterpret_cast<const uint4*>(p + row * inner));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (kWide) {
            acc[i] = K::value32(k32[i]);
        } else {
            acc[2 * i] = K::template value16<Tin>(short2_t{k16[i].x, k16[i].x});
            acc[2 * i + 1] = K::template value16<Tin>(short2_t{k16[i].y, k16[i].y});
        }
    }
}

// Column reductions.  A block covers the columns of col_lanes lanes (16
// lanes of 16-byte packets of a 16-bit type, 64 lanes of float32 packets or
// of single elements) over the rows [ch * chunk, +chunk) of every outer index
// o = z, z + gridDim.z, ...; its kBlock / col_lanes row groups stride down
// those rows, and the groups are combined in a fixed order.  With one chunk
// the block writes the result; otherwise it writes float32 partials
// out[(o * nchunk + ch) * inner + col].
//
// FUSE folds the second pass in: the partials are written and read back
// with agent-coherent accesses; every block counts its arrival in
// col_counters (one 128-byte line per column range o * gridDim.x +
// blockIdx.x) once its partial stores have
// completed, and the last of the nchunk blocks of a column range reads the
// nchunk partials back in chunk order, writes the result, and resets the
// counter to zero for the next launch.  The counters start at zero (device
// globals are zeroed when the code object loads).
template <typename Tin, bool VEC>
constexpr int col_lanes() {
    // Measured on X1 and X2 of config 3: 16-bit packets run best as 16 lanes
    // (128 columns) per row, float32 packets and single elements as 64.
    return VEC && sizeof(typename Elem<Tin>::storage) == 2 ? 16 : 64;
}

constexpr int64_t kMaxColCounters = 8192;
__device__ unsigned int col_counters[kMaxColCounters * kCounterStride];

template <typename Tin, typename Tout, int OP, bool VEC, bool FUSE>
__global__ __launch_bounds__(kBlock) void reduce_cols_kernel(
    const typename Elem<Tin>::storage* x, typename Elem<Tout>::storage* out,
    typename Elem<Tin>::storage* result, int64_t outer, int64_t r, int64_t inner, int64_t chunk,
    int64_t nchunk, bool final_pass, int64_t count) {
    constexpr int N = VEC ? Packet<Tin>::N : 1;
    constexpr int LANES = col_lanes<Tin, VEC>();
    // Non-temporal loads measured faster with 64 lanes a row, plain ones
    // with 16.
    constexpr bool NT = LANES == 64;
    constexpr int G = kBlock / LANES;  // row groups
    constexpr int COLS = LANES * N;    // columns per block
    __shared__ float partial[G][COLS + 1];
    __shared__ bool last;
    const int lane = threadIdx.x % LANES, rg = threadIdx.x / LANES;
    const int64_t col = (static_cast<int64_t>(blockIdx.x) * LANES + lane) * N;
    const int64_t ch = blockIdx.y;
    const int64_t begin = ch * chunk;
    const int64_t end = begin + chunk < r ? begin + chunk : r;
    for (int64_t o = blockIdx.z; o < outer; o += gridDim.z) {
        float acc[N];
#pragma unroll
        for (int j = 0; j < N; ++j) acc[j] = Combine<OP>::identity();
        bool exact = !(kMinMax<OP> && VEC);
        if constexpr (kMinMax<OP> && VEC) {
            if (col < inner) {
                cols_keys<Tin, OP, G, NT>(acc, x + o * r * inner + col, begin + rg, end, inner);
#pragma unroll
                for (int j = 0; j < N; ++j) exact = exact || acc[j] != acc[j];
                if (exact) {
#pragma unroll
                    for (int j = 0; j < N; ++j) acc[j] = Combine<OP>::identity();
                }
            }
        }
        if (exact && col < inner) {
            const typename Elem<Tin>::storage* p = x + o * r * inner + col;
            int64_t row = begin + rg;
            constexpr int U = 8;
            for (; row + (U - 1) * G < end; row += U * G) {
                if constexpr (VEC) {
                    Packet<Tin> v[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const auto* q = p + (row + u * G) * inner;
                        v[u] = NT ? load_packet_nt<Tin>(q) : load_packet<Tin>(q);
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u)
#pragma unroll
                        for (int j = 0; j < N; ++j)
                            acc[j] = Combine<OP>::apply(acc[j], Elem<Tin>::load(v[u].v[j]));
                } else {
                    typename Elem<Tin>::storage v[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) v[u] = p[(row + u * G) * inner];
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        acc[0] = Combine<OP>::apply(acc[0], Elem<Tin>::load(v[u]));
                }
            }
            for (; row < end; row += G) {
                if constexpr (VEC) {
                    const Packet<Tin> v = load_packet<Tin>(p + row * inner);
#pragma unroll
                    for (int j = 0; j < N; ++j)
                        acc[j] = Combine<OP>::apply(acc[j], Elem<Tin>::load(v.v[j]));
                } else {
                    acc[0] = Combine<OP>::apply(acc[0], Elem<Tin>::load(p[row * inner]));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < N; ++j) partial[rg][lane * N + j] = acc[j];
        __syncthreads();
        // The row groups are combined in a fixed order.
        for (int e = threadIdx.x; e < COLS; e += kBlock) {
            float v = partial[0][e];
#pragma unroll
            for (int g = 1; g < G; ++g) v = Combine<OP>::apply(v, partial[g][e]);
            const int64_t c = static_cast<int64_t>(blockIdx.x) * COLS + e;
            if (c < inner) {
                auto* dst = out + (o * nchunk + ch) * inner + c;
                const auto val = Elem<Tout>::store(finish<OP>(v, count, final_pass));
                if constexpr (FUSE) {
                    // Agent-coherent store: written through past this XCD's L2.
                    __hip_atomic_store(dst, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    *dst = val;
                }
            }
        }
        if constexpr (FUSE) {
            static_assert(std::is_same<Tout, float>::value, "partials are float32");
            // Every thread's partial stores have completed (device-visible,
            // being agent-coherent) before the block counts its arrival.  A
            // device-scope fence would write back the whole L2 per block.
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            const int64_t slot = (o * gridDim.x + blockIdx.x) * kCounterStride;
            if (threadIdx.x == 0) {
                last = __hip_atomic_fetch_add(&col_counters[slot], 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT) == nchunk - 1;
            }
            __syncthreads();
            if (last) {
                for (int e = threadIdx.x; e < COLS; e += kBlock) {
                    const int64_t c = static_cast<int64_t>(blockIdx.x) * COLS + e;
                    if (c < inner) {
                        float* q = out + o * nchunk * inner + c;
                        auto at = [&](int64_t k) {
                            return __hip_atomic_load(q + k * inner, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        };
                        // Eight loads in flight at a time, folded in chunk order.
                        float v = at(0);
                        int64_t k = 1;
                        for (; k + 8 <= nchunk; k += 8) {
                            float t[8];
#pragma unroll
                            for (int u = 0; u < 8; ++u) t[u] = at(k + u);
#pragma unroll
                            for (int u = 0; u < 8; ++u) v = Combine<OP>::apply(v, t[u]);
                        }
                        for (; k < nchunk; ++k) v = Combine<OP>::apply(v, at(k));
                        result[o * inner + c] = Elem<Tin>::store(finish<OP>(v, count, true));
                    }
                }
                if (threadIdx.x == 0) {
                    __hip_atomic_store(&col_counters[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        __syncthreads();
    }
}

// Device memory for the float32 partials of a split reduction: a caller's
// buffer of `floats` elements (the allocation-free entry point), or, when
// `ptr` is null, a workspace from the caching allocator.
struct Scratch {
    float* ptr = nullptr;
    int64_t floats = 0;
};

class Partials {
public:
    Partials(const Scratch& scratch, int64_t floats, int device) {
        if (scratch.ptr != nullptr) {
            TP_AMD_CHECK(floats <= scratch.floats, "reduction needs ", floats * 4,
                         " bytes of partials, more than the ", scratch.floats * 4,
                         "-byte static scratch; use tp_amd_launch_reduce");
            ptr_ = scratch.ptr;
        } else {
            ws_ = Workspace(static_cast<size_t>(floats) * sizeof(float), device);
            ptr_ = static_cast<float*>(ws_.get());
        }
    }
    float* get() const { return ptr_; }

private:
    Workspace ws_;
    float* ptr_ = nullptr;
};

// How a reduction of [outer, r, inner] is split, decided on the host from
// the shape, the packet width and the CU count alone, so that the launch
// and the partials-size query (tp_amd_reduce_partial_bytes) agree.
//   inner == 1 (rows): rows short or many enough run one segment per row;
//     otherwise each row is cut into nseg segments of `chunk` elements
//     (about two blocks per CU, at least 4096 elements each) whose float32
//     partials the last block of the row folds.
//   inner > 1 (columns): bx column ranges of cols_per_block columns times z
//     outer indices; with fewer of those than CUs the rows are cut into
//     nchunk chunks whose partials the last block of a column range folds.
struct SplitPlan {
    int64_t nseg = 1, chunk = 0, ngroups = 0;  // rows
    int64_t bx = 0, z = 0, nchunk = 1;         // columns (chunk: rows a chunk)
    int64_t partial_floats = 0;
};

SplitPlan plan_split(int64_t outer, int64_t r, int64_t inner, int64_t cus, int64_t packet, bool vec,
                     int64_t cols_per_block) {
    SplitPlan sp;
    if (inner == 1) {
        // About segments_per_cu(packet) blocks a CU (above).
        if (outer < cus * 16 && r >= 8192) {
            int64_t nseg = (cus * segments_per_cu(packet) + outer - 1) / outer;
            const int64_t max_seg = r / 4096;  // >= 2 here
            if (nseg > max_seg) nseg = max_seg;
            int64_t chunk = (r + nseg - 1) / nseg;
            if (vec) chunk = (chunk + packet - 1) / packet * packet;
            nseg = (r + chunk - 1) / chunk;
            if (nseg > 1) {
                sp.nseg = nseg;
                sp.chunk = chunk;
                sp.ngroups = (nseg + kFoldGroup - 1) / kFoldGroup;
                sp.partial_floats = outer * nseg;
            }
        }
        return sp;
    }
    sp.bx = (inner + cols_per_block - 1) / cols_per_block;
    sp.z = outer < 65535 ? outer : 65535;
    const int64_t base_blocks = sp.bx * sp.z;
    // About one block per CU, each with eight 16-byte loads per thread in
    // flight: nchunk = round(CUs / column ranges).  Measured on config 3's
    // dim-0 reductions against the earlier two blocks per CU: X2 [4096,
    // 32000] bf16 1 chunk 40.8 us against 3 chunks 43.6 us, fp32 2 chunks
    // 79 us against 5 chunks 85 us; X1 [32768, 4096] bf16 8 chunks 41.1 us
    // against 16 chunks 43.2 us, fp32 16 or 32 chunks alike.  Fewer chunks
    // write fewer partials, and the blocks fill the CUs in one even round.
    int64_t nchunk = 1;
    if (base_blocks < cus && r >= 64) {
        nchunk = (cus + base_blocks / 2) / base_blocks;
        const int64_t max_chunks = r / 32;  // keep >= 32 rows per chunk
        if (nchunk > max_chunks) nchunk = max_chunks > 1 ? max_chunks : 1;
        if (nchunk > 65535) nchunk = 65535;
    }
    sp.chunk = (r + nchunk - 1) / nchunk;
    sp.nchunk = (r + sp.chunk - 1) / sp.chunk;
    if (sp.nchunk > 1) sp.partial_floats = outer * sp.nchunk * inner;
    return sp;
}

template <typename T, int OP>
void reduce_typed(int device, int64_t outer, int64_t r, int64_t inner, const void* xv,
                  void* outv, const Scratch& scratch) {
    using S = typename Elem<T>::storage;
    const S* x = static_cast<const S*>(xv);
    S* out = static_cast<S*>(outv);
    hipStream_t st = stream(device);
    const int64_t cus = cu_count(device);
    constexpr int N = Packet<T>::N;
    if (inner == 1) {
        const bool vec = r % N == 0 && aligned16(x);
        const SplitPlan sp = plan_split(outer, r, 1, cus, N, vec, 0);
        if (sp.nseg > 1) {
            TP_AMD_CHECK(outer <= kMaxFoldRows && outer * sp.ngroups <= kMaxFoldGroups,
                         "row reduction: ", outer, " rows of ", sp.nseg, " segments exceed the arrival counters");
            const int64_t nsegs = outer * sp.nseg;
            Partials partial(scratch, sp.partial_floats, device);
            if (vec) {
                reduce_rows_fused_kernel<T, OP, true><<<static_cast<unsigned>(nsegs), fused_threads<T>(), 0, st>>>(
                    x, out, partial.get(), r, sp.chunk, sp.nseg, sp.ngroups);
            } else {
                reduce_rows_fused_kernel<T, OP, false><<<static_cast<unsigned>(nsegs), fused_threads<T>(), 0, st>>>(
                    x, out, partial.get(), r, sp.chunk, sp.nseg, sp.ngroups);
            }
            TP_AMD_HIP_CHECK(hipGetLastError());
            return;
        }
        // One segment per row.  Four waves share a row of 4096 elements or
        // more; amax / amin of 16-bit storage (integer keys) run best one
        // wave a row up to 16 KB (measured on 4096-element bf16 rows: 40 us
        // against 45-49 us).
        const bool key16 = kMinMax<OP> && sizeof(S) == 2;
        const bool long_rows = key16 ? r * 2 >= 16384 : r >= 4096;
        auto launch_rows = [&](auto waves_tag, auto vec_tag) {
            constexpr int W = decltype(waves_tag)::value;
            constexpr bool V = decltype(vec_tag)::value;
            constexpr int per_block = (kBlock / kWave) / W;
            const int64_t blocks = (outer + per_block - 1) / per_block;
            reduce_rows_kernel<T, T, OP, W, V><<<blocks, kBlock, 0, st>>>(x, out, outer, r, r, 1, true, r);
        };
        using One = std::integral_constant<int, 1>;
        using Four = std::integral_constant<int, 4>;
        using Yes = std::true_type;
        using No = std::false_type;
        if (long_rows) {
            vec ? launch_rows(Four{}, Yes{}) : launch_rows(Four{}, No{});
        } else {
            vec ? launch_rows(One{}, Yes{}) : launch_rows(One{}, No{});
        }
        TP_AMD_HIP_CHECK(hipGetLastError());
        return;
    }
    // Column reductions.
    const bool vec = inner % N == 0 && aligned16(x);
    const int64_t cols_per_block = vec ? col_lanes<T, true>() * N : col_lanes<T, false>();
    const SplitPlan sp = plan_split(outer, r, inner, cus, N, vec, cols_per_block);
    const int64_t bx = sp.bx, nchunk = sp.nchunk, chunk = sp.chunk;
    const dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>(nchunk), static_cast<unsigned>(sp.z));
    if (nchunk == 1) {
        if (vec) {
            reduce_cols_kernel<T, T, OP, true, false>
                <<<grid, kBlock, 0, st>>>(x, out, nullptr, outer, r, inner, chunk, 1, true, r);
        } else {
            reduce_cols_kernel<T, T, OP, false, false>
                <<<grid, kBlock, 0, st>>>(x, out, nullptr, outer, r, inner, chunk, 1, true, r);
        }
        TP_AMD_HIP_CHECK(hipGetLastError());
        return;
    }
    // Rows are split only when bx * outer < cus, so one arrival counter
    // per column range always fits.
    TP_AMD_CHECK(outer * bx <= kMaxColCounters, "column reduction: ", outer * bx,
                 " column ranges exceed the arrival counters");
    Partials partials(scratch, sp.partial_floats, device);
    float* partial = partials.get();
    // One launch: the last block of each column range folds the partials.
    if (vec) {
        reduce_cols_kernel<T, float, OP, true, true>
            <<<grid, kBlock, 0, st>>>(x, partial, out, outer, r, inner, chunk, nchunk, false, r);
    } else {
        reduce_cols_kernel<T, float, OP, false, true>
            <<<grid, kBlock, 0, st>>>(x, partial, out, outer, r, inner, chunk, nchunk, false, r);
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template <typename T>
void reduce_dispatch_op(int device, int op, int64_t outer, int64_t r, int64_t inner,
                        const void* x, void* out, const Scratch& scratch) {
    switch (op) {
        case TP_AMD_REDUCE_SUM:
            reduce_typed<T, TP_AMD_REDUCE_SUM>(device, outer, r, inner, x, out, scratch);
            break;
        case TP_AMD_REDUCE_MEAN:
            reduce_typed<T, TP_AMD_REDUCE_MEAN>(device, outer, r, inner, x, out, scratch);
            break;
        case TP_AMD_REDUCE_AMAX:
            reduce_typed<T, TP_AMD_REDUCE_AMAX>(device, outer, r, inner, x, out, scratch);
            break;
        case TP_AMD_REDUCE_AMIN:
            reduce_typed<T, TP_AMD_REDUCE_AMIN>(device, outer, r, inner, x, out, scratch);
            break;
        default: TP_AMD_CHECK(false, "unknown reduce op ", op);
    }
}

// Allocation-free partials: a static device array, one per GPU, holding the
// split reductions' float32 partials (at most kScratchFloats).  Host code
// never passes `reduce_scratch` itself to a kernel: its device address on
// each GPU comes from hipGetSymbolAddress, taken once per device with that
// device current.
constexpr int64_t kScratchFloats = int64_t{1} << 18;  // 1 MiB
__device__ __attribute__((aligned(256))) float reduce_scratch[kScratchFloats];

Scratch static_scratch(int device) {
    static std::mutex mutex;
    static float* ptrs[kMaxDevices] = {};
    TP_AMD_CHECK(device >= 0 && device < kMaxDevices, "device ", device, " out of range");
    std::lock_guard<std::mutex> lock(mutex);
    if (ptrs[device] == nullptr) {
        void* p = nullptr;
        TP_AMD_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(reduce_scratch)));
        ptrs[device] = static_cast<float*>(p);
    }
    return Scratch{ptrs[device], kScratchFloats};
}

int launch_reduce(int device, int op, int dtype, int64_t outer, int64_t r, int64_t inner,
                  const void* x, void* out, bool no_alloc) {
    return guarded([&] {
        TP_AMD_CHECK(outer >= 0 && r >= 0 && inner >= 0, "negative reduce extent");
        if (outer == 0 || inner == 0) return;
        TP_AMD_CHECK(r > 0, "reduce over an empty axis: the caller fills the result");
        const OnDevice scope(device);
        const int index = scope.index();
        const Scratch scratch = no_alloc ? static_scratch(index) : Scratch{};
        switch (dtype) {
            case TP_AMD_FLOAT32: reduce_dispatch_op<float>(index, op, outer, r, inner, x, out, scratch); break;
            case TP_AMD_BFLOAT16: reduce_dispatch_op<bf16_t>(index, op, outer, r, inner, x, out, scratch); break;
            case TP_AMD_FLOAT16: reduce_dispatch_op<f16_t>(index, op, outer, r, inner, x, out, scratch); break;
            default:
                TP_AMD_CHECK(false, "reductions take float32, float16 or bfloat16, got ",
                             dtype_name(dtype));
        }
    });
}

}  // namespace

}  // namespace tp_amd

using namespace tp_amd;

extern "C" {

int tp_amd_launch_reduce(int device, int op, int dtype, int64_t outer, int64_t r,
                         int64_t inner, const void* x, void* out) {
    return launch_reduce(device, op, dtype, outer, r, inner, x, out, false);
}

int tp_amd_launch_reduce_noalloc(int device, int op, int dtype, int64_t outer, int64_t r,
                                 int64_t inner, const void* x, void* out) {
    return launch_reduce(device, op, dtype, outer, r, inner, x, out, true);
}

size_t tp_amd_reduce_noalloc_scratch_bytes(void) {
    return static_cast<size_t>(kScratchFloats) * sizeof(float);
}

int64_t tp_amd_reduce_partial_bytes(int compute_units, int dtype, int64_t outer, int64_t r, int64_t inner) {
    int64_t esize = 0;
    switch (dtype) {
        case TP_AMD_FLOAT32: esize = 4; break;
        case TP_AMD_BFLOAT16:
        case TP_AMD_FLOAT16: esize = 2; break;
        default: return -1;
    }
    if (compute_units <= 0 || outer < 0 || r < 0 || inner < 0) return -1;
    if (outer == 0 || inner == 0 || r == 0) return 0;
    const int64_t packet = 16 / esize;
    const bool vec = (inner == 1 ? r : inner) % packet == 0;
    // col_lanes: 16 lanes of 16-bit packets, 64 lanes of float32 packets or single elements
    const int64_t cols_per_block = vec ? (esize == 2 ? 16 : 64) * packet : 64;
    return plan_split(outer, r, inner, compute_units, packet, vec, cols_per_block).partial_floats *
           static_cast<int64_t>(sizeof(float));
}

}  // extern "C"
