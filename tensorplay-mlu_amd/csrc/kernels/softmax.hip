// Fused softmax / log_softmax forward and backward for gfx950 (the
// reference's cnnlSoftmaxForward / cnnlSoftmaxBackward,
// tensorplay_mlu/csrc/ReduceKernels.cpp:171-199).
//
// Rows along the last axis (inner == 1) are held in registers: each row is
// read from HBM once and written once.  A configuration (WAVES, EPT) gives a
// row WAVES wavefronts and each thread EPT elements (EPT / N 16-byte
// packets), so rows up to 64 * WAVES * EPT elements stay on chip; up to 4
// waves per row, a 256-thread block holds 4 / WAVES rows, so several blocks
// share a CU.  The row max and the exponential sum combine across lanes with
// shuffles and across waves in LDS.  Longer rows (a multiple of the packet,
// 16-byte aligned) take a block-per-row kernel that keeps a running (max,
// sum) per thread over the row, then re-reads it -- from L2, which holds the
// CU's current row -- to write the result.  Anything else takes a scalar
// block-per-row kernel.  Softmax over a leading axis (inner > 1) walks the
// reduced axis with the contiguous inner axis across threads.
//
// The per-element arithmetic is kept short because for 16-bit storage it,
// not HBM, would set the pace: exponentials are 2^(d log2 e) on v_exp_f32
// with d = x - max formed first, the softmax quotient is one reciprocal per
// row, and results are packed with the hardware round-to-nearest-even
// conversions.

#include <cmath>
#include <type_traits>

#include "device_common.h"
#include "../allocator.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kBlock = 256;
constexpr float kLog2e = 1.44269504088896340736f;

// e^d on v_exp_f32 (the softmax arguments d = x - max are <= 0, where its
// error stays within a few float32 ulps), as (2^(a/2))^2 with a = d log2 e:
// the instruction returns 0 for results below 2^-126, where the halves are
// still normal and their product underflows gradually, so an entry 88-103
// below its row's maximum keeps its subnormal value (bfloat16 has them).
__device__ __forceinline__ float exp_fast(float d) {
    const float h = __builtin_amdgcn_exp2f(d * (0.5f * kLog2e));
    return h * h;
}

__device__ __forceinline__ float wave_max(float v) {
    return wave_allreduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_sum(float v) {
    return wave_allreduce(v, [](float a, float b) { return a + b; });
}

// Layout of a (WAVES, EPT) configuration: WAVES <= 4 packs 4 / WAVES rows
// into a 256-thread block; more waves make one row per block.
template <int WAVES>
constexpr int block_threads() {
    return WAVES >= 4 ? WAVES * kWave : kBlock;
}
template <int WAVES>
constexpr int rows_per_block() {
    return WAVES >= 4 ? 1 : 4 / WAVES;
}

// Reduce ``v`` over the WAVES waves of this thread's row.  ``scratch`` holds
// one float per wave of the block.  Every wave of the block must call it.
template <int WAVES, bool MAX>
__device__ __forceinline__ float row_reduce(float v, float* scratch) {
    v = MAX ? wave_max(v) : wave_sum(v);
    if constexpr (WAVES > 1) {
        const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
        const int first = (wave / WAVES) * WAVES;
        __syncthreads();  // scratch may still be read from the previous use
        if (lane == 0) scratch[wave] = v;
        __syncthreads();
        const float t = lane < WAVES ? scratch[first + lane] : (MAX ? -INFINITY : 0.0f);
        v = MAX ? wave_max(t) : wave_sum(t);
    }
    return v;
}

template <typename T, int WAVES, int EPT>
__global__ __launch_bounds__(block_threads<WAVES>()) void softmax_rows_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t rows, int64_t D,
    bool log) {
    constexpr int N = Packet<T>::N;
    constexpr int VPT = EPT / N;
    static_assert(VPT * N == EPT, "EPT must be a whole number of packets");
    constexpr int kThreads = WAVES * kWave;
    __shared__ float scratch[block_threads<WAVES>() / kWave];
    const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block<WAVES>() +
                        threadIdx.x / kThreads;
    const int tid = threadIdx.x % kThreads;
    const bool active = row < rows;  // uniform per wave
    const int64_t npk = D / N;
    const typename Elem<T>::storage* xr = x + (active ? row : 0) * D;
    float v[VPT][N];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (active && q < npk) {
            unpack<T>(load_raw_nt(xr + q * N), v[k]);
#pragma unroll
            for (int j = 0; j < N; ++j) m = fmaxf(m, v[k][j]);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) v[k][j] = -INFINITY;
        }
    }
    m = row_reduce<WAVES, true>(m, scratch);
    // A row of -inf (or an inactive one) would give inf - inf; exp(-inf - 0)
    // keeps it at 0 instead.
    const float shift = m == -INFINITY ? 0.0f : m;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
        for (int j = 0; j < N; ++j) {
            v[k][j] -= shift;
            const float e = exp_fast(v[k][j]);
            s += e;
            if (!log) v[k][j] = e;
        }
    s = row_reduce<WAVES, false>(s, scratch);
    if (!active) return;
    const float lse = logf(s);
    const float inv = 1.0f / s;
    typename Elem<T>::storage* yr = y + row * D;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (q < npk) {
            float o[N];
#pragma unroll
            for (int j = 0; j < N; ++j) o[j] = log ? v[k][j] - lse : v[k][j] * inv;
            store_raw_nt(yr + q * N, pack<T>(o));
        }
    }
}

// Rows that need a whole 16-wave block: one such block fills a CU, so a
// block per row would leave the CU idle while each row's loads are in
// flight.  Instead a grid of one block per CU walks the rows, and the loads
// of its next row are issued before the current row is reduced and written
// (two register sets, alternating).  Rows are addressed through buffer
// resources (a row and the whole grid under 4 GiB of offsets per row): no
// branch surrounds a load or store, so the compiler waits for a prefetched
// row without also waiting for the stores issued after it.
template <typename T, int VPT>
struct RowBuffer {
    uint4 raw[VPT];
};

// Row `row` (zeros past the last row or the row's end).
template <typename T, int VPT>
__device__ __forceinline__ void fetch_row(RowBuffer<T, VPT>& b, const typename Elem<T>::storage* x,
                                          int64_t row, int64_t rows, int64_t D, int tid) {
    const bool ok = row < rows;
    const Rsrc r = buffer_over(x + (ok ? row : 0) * D,
                               ok ? static_cast<uint32_t>(D * sizeof(typename Elem<T>::storage)) : 0u);
#pragma unroll
    for (int k = 0; k < VPT; ++k) b.raw[k] = buffer_load16(r, static_cast<uint32_t>(tid + k * 16 * kWave) * 16u);
}

__device__ __forceinline__ uint32_t& word(uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// float32 rows work in place in the packet registers (a second float copy
// of the row would not fit beside the prefetched next row).
template <int VPT>
__device__ __forceinline__ void finish_row_f32(RowBuffer<float, VPT>& b, float* yr, int64_t npk,
                                               int tid, bool log, float* scratch) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const bool in = tid + k * 16 * kWave < npk;
#pragma unroll
        for (int j = 0; j < 4; ++j) m = fmaxf(m, in ? __uint_as_float(word(b.raw[k], j)) : -INFINITY);
    }
    m = row_reduce<16, true>(m, scratch);
    const float shift = m == -INFINITY ? 0.0f : m;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const bool in = tid + k * 16 * kWave < npk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float d = __uint_as_float(word(b.raw[k], j)) - shift;
            const float e = exp_fast(d);
            s += in ? e : 0.0f;
            word(b.raw[k], j) = __float_as_uint(log ? d : e);
        }
    }
    s = row_reduce<16, false>(s, scratch);
    const float lse = logf(s);
    const float inv = 1.0f / s;
    const Rsrc out = buffer_over(yr, static_cast<uint32_t>(npk * 16));
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        uint4 o = b.raw[k];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = __uint_as_float(word(o, j));
            word(o, j) = __float_as_uint(log ? v - lse : v * inv);
        }
        buffer_store16(out, static_cast<uint32_t>(tid + k * 16 * kWave) * 16u, o);
    }
}

template <typename T, int VPT>
__device__ __forceinline__ void finish_row(RowBuffer<T, VPT>& b,
                                           typename Elem<T>::storage* yr, int64_t npk, int tid,
                                           bool log, float* scratch) {
    if constexpr (sizeof(typename Elem<T>::storage) == 4) {
        finish_row_f32<VPT>(b, yr, npk, tid, log, scratch);
        return;
    }
    constexpr int N = Packet<T>::N;
    float v[VPT][N];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const bool in = tid + k * 16 * kWave < npk;
        unpack<T>(b.raw[k], v[k]);
#pragma unroll
        for (int j = 0; j < N; ++j) {
            v[k][j] = in ? v[k][j] : -INFINITY;
            m = fmaxf(m, v[k][j]);
        }
    }
    m = row_reduce<16, true>(m, scratch);
    const float shift = m == -INFINITY ? 0.0f : m;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
        for (int j = 0; j < N; ++j) {
            v[k][j] -= shift;
            const float e = exp_fast(v[k][j]);
            s += e;
            if (!log) v[k][j] = e;
        }
    s = row_reduce<16, false>(s, scratch);
    const float lse = logf(s);
    const float inv = 1.0f / s;
    const Rsrc out = buffer_over(yr, static_cast<uint32_t>(npk * 16));
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        float o[N];
#pragma unroll
        for (int j = 0; j < N; ++j) o[j] = log ? v[k][j] - lse : v[k][j] * inv;
        buffer_store16(out, static_cast<uint32_t>(tid + k * 16 * kWave) * 16u, pack<T>(o));
    }
}

template <typename T, int VPT>
__global__ __launch_bounds__(16 * kWave) void softmax_rows_stream_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t rows, int64_t D,
    bool log) {
    constexpr int N = Packet<T>::N;
    __shared__ float scratch[16];
    const int tid = threadIdx.x;
    const int64_t npk = D / N;
    const int64_t step = gridDim.x;
    RowBuffer<T, VPT> a, b;
    int64_t row = blockIdx.x;
    fetch_row<T, VPT>(a, x, row, rows, D, tid);
    drain();
    // Uniform per block: every thread walks the same rows.
    for (; row < rows; row += 2 * step) {
        fetch_row<T, VPT>(b, x, row + step, rows, D, tid);
        finish_row<T, VPT>(a, y + row * D, npk, tid, log, scratch);
        if (row + step >= rows) break;
        fetch_row<T, VPT>(a, x, row + 2 * step, rows, D, tid);
        finish_row<T, VPT>(b, y + (row + step) * D, npk, tid, log, scratch);
    }
}

// The backward keeps the two rows as raw packets (16-bit storage takes half
// the registers of unpacked floats) and converts them on use.
template <typename T, int WAVES, int EPT>
__global__ __launch_bounds__(block_threads<WAVES>()) void softmax_backward_rows_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy,
    typename Elem<T>::storage* dx, int64_t rows, int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
    constexpr int VPT = EPT / N;
    static_assert(VPT * N == EPT, "EPT must be a whole number of packets");
    constexpr int kThreads = WAVES * kWave;
    __shared__ float scratch[block_threads<WAVES>() / kWave];
    const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block<WAVES>() +
                        threadIdx.x / kThreads;
    const int tid = threadIdx.x % kThreads;
    const bool active = row < rows;
    const int64_t npk = D / N;
    const int64_t base = (active ? row : 0) * D;
    uint4 ry[VPT], rg[VPT];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (active && q < npk) {
            ry[k] = load_raw_nt(y + base + q * N);
            rg[k] = load_raw_nt(dy + base + q * N);
        } else {
            ry[k] = rg[k] = make_uint4(0, 0, 0, 0);  // zeros add nothing to the sum
        }
    }
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        float a[N], g[N];
        unpack<T>(ry[k], a);
        unpack<T>(rg[k], g);
#pragma unroll
        for (int j = 0; j < N; ++j) s += log ? g[j] : g[j] * a[j];
    }
    s = row_reduce<WAVES, false>(s, scratch);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (q < npk) {
            float a[N], g[N], o[N];
            unpack<T>(ry[k], a);
            unpack<T>(rg[k], g);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                o[j] = log ? g[j] - exp_fast(a[j]) * s : a[j] * (g[j] - s);
            }
            store_raw_nt(dx + base + q * N, pack<T>(o));
        }
    }
}

// The backward of rows that need a whole 16-wave block, the forward's
// stream scheme for two inputs: one block per CU walks the rows with the
// next row's y and dy loaded before this row's reduction (two register sets
// of raw packets), all through buffer resources.  Packets past the row's
// end load as zeros and add nothing to the row sum.
template <typename T, int VPT>
struct GradRows {
    uint4 y[VPT], g[VPT];
};

template <typename T, int VPT>
__global__ __launch_bounds__(16 * kWave) void softmax_backward_stream_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy,
    typename Elem<T>::storage* dx, int64_t rows, int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
    __shared__ float scratch[16];
    const int tid = threadIdx.x;
    const uint32_t row_bytes = static_cast<uint32_t>(D * sizeof(typename Elem<T>::storage));
    const int64_t step = gridDim.x;
    auto fetch = [&](GradRows<T, VPT>& b, int64_t row) {
        const bool ok = row < rows;
        const int64_t at = (ok ? row : 0) * D;
        const Rsrc ry = buffer_over(y + at, ok ? row_bytes : 0u);
        const Rsrc rg = buffer_over(dy + at, ok ? row_bytes : 0u);
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const uint32_t off = static_cast<uint32_t>(tid + k * 16 * kWave) * 16u;
            b.y[k] = buffer_load16(ry, off);
            b.g[k] = buffer_load16(rg, off);
        }
    };
    auto finish = [&](const GradRows<T, VPT>& b, int64_t row) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            float a[N], g[N];
            unpack<T>(b.y[k], a);
            unpack<T>(b.g[k], g);
#pragma unroll
            for (int j = 0; j < N; ++j) s += log ? g[j] : g[j] * a[j];
        }
        s = row_reduce<16, false>(s, scratch);
        const Rsrc out = buffer_over(dx + row * D, row_bytes);
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            float a[N], g[N], o[N];
            unpack<T>(b.y[k], a);
            unpack<T>(b.g[k], g);
#pragma unroll
            for (int j = 0; j < N; ++j) o[j] = log ? g[j] - exp_fast(a[j]) * s : a[j] * (g[j] - s);
            buffer_store16(out, static_cast<uint32_t>(tid + k * 16 * kWave) * 16u, pack<T>(o));
        }
    };
    GradRows<T, VPT> a, b;
    int64_t row = blockIdx.x;
    fetch(a, row);
    drain();
    for (; row < rows; row += 2 * step) {
        fetch(b, row + step);
        finish(a, row);
        if (row + step >= rows) break;
        fetch(a, row + 2 * step);
        finish(b, row + step);
    }
}

// (max, sum) pairs: the sum is relative to the max.
__device__ __forceinline__ void online_merge(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;  // both empty
    s = s * exp_fast(m - mn) + s2 * exp_fast(m2 - mn);
    m = mn;
}

__device__ __forceinline__ void block_merge(float& m, float& s) {
    __shared__ float sm[kBlock / kWave], ss[kBlock / kWave];
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float m2 = wave_shfl_xor(m, o), s2 = wave_shfl_xor(s, o);
        online_merge(m, s, m2, s2);
    }
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) {
        sm[wave] = m;
        ss[wave] = s;
    }
    __syncthreads();
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int w = 1; w < kBlock / kWave; ++w) online_merge(m, s, sm[w], ss[w]);
}

// Long rows (D a multiple of the packet, 16-byte aligned): a 256-thread
// block per row.  Pass 1 keeps a running (max, sum) per thread, UNROLL
// packets in flight; pass 2 re-reads the row (an L2 hit: the CU's current
// row is the most recent data it touched) and writes the result.
template <typename T, int UNROLL>
__global__ __launch_bounds__(kBlock) void softmax_rows_long_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
    const int64_t npk = D / N;
    const typename Elem<T>::storage* xr = x + static_cast<int64_t>(blockIdx.x) * D;
    float m = -INFINITY, s = 0.0f;
    for (int64_t q0 = threadIdx.x; q0 < npk; q0 += static_cast<int64_t>(kBlock) * UNROLL) {
        uint4 raw[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t q = q0 + static_cast<int64_t>(u) * kBlock;
            raw[u] = q < npk ? *reinterpret_cast<const uint4*>(xr + q * N)
                             : make_uint4(0xff800000u, 0xff800000u, 0xff800000u, 0xff800000u);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t q = q0 + static_cast<int64_t>(u) * kBlock;
            if (q >= npk) continue;
            float v[N];
            unpack<T>(raw[u], v);
            float pm = v[0];
#pragma unroll
            for (int j = 1; j < N; ++j) pm = fmaxf(pm, v[j]);
            const float mn = fmaxf(m, pm);
            if (mn == -INFINITY) continue;
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < N; ++j) t += exp_fast(v[j] - mn);
            s = s * exp_fast(m - mn) + t;
            m = mn;
        }
    }
    block_merge(m, s);
    const float shift = m == -INFINITY ? 0.0f : m;
    const float lse = logf(s);
    const float inv = 1.0f / s;
    typename Elem<T>::storage* yr = y + static_cast<int64_t>(blockIdx.x) * D;
    for (int64_t q = threadIdx.x; q < npk; q += kBlock) {
        float v[N], o[N];
        unpack<T>(*reinterpret_cast<const uint4*>(xr + q * N), v);
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const float d = v[j] - shift;
            o[j] = log ? d - lse : exp_fast(d) * inv;
        }
        store_raw_nt(yr + q * N, pack<T>(o));
    }
}

template <typename T, int UNROLL>
__global__ __launch_bounds__(kBlock) void softmax_backward_rows_long_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy,
    typename Elem<T>::storage* dx, int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
    __shared__ float scratch[kBlock / kWave];
    const int64_t npk = D / N;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * D;
    float s = 0.0f;
    for (int64_t q0 = threadIdx.x; q0 < npk; q0 += static_cast<int64_t>(kBlock) * UNROLL) {
        uint4 ra[UNROLL], rg[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t q = q0 + static_cast<int64_t>(u) * kBlock;
            const bool in = q < npk;
            ra[u] = in ? *reinterpret_cast<const uint4*>(y + base + q * N) : make_uint4(0, 0, 0, 0);
            rg[u] = in ? *reinterpret_cast<const uint4*>(dy + base + q * N) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            float a[N], g[N];
            unpack<T>(ra[u], a);
            unpack<T>(rg[u], g);
#pragma unroll
            for (int j = 0; j < N; ++j) s += log ? g[j] : g[j] * a[j];
        }
    }
    s = row_reduce<kBlock / kWave, false>(s, scratch);
    for (int64_t q = threadIdx.x; q < npk; q += kBlock) {
        float a[N], g[N], o[N];
        unpack<T>(*reinterpret_cast<const uint4*>(y + base + q * N), a);
        unpack<T>(*reinterpret_cast<const uint4*>(dy + base + q * N), g);
#pragma unroll
        for (int j = 0; j < N; ++j) o[j] = log ? g[j] - exp_fast(a[j]) * s : a[j] * (g[j] - s);
        store_raw_nt(dx + base + q * N, pack<T>(o));
    }
}

// Any row length or alignment: block per row, running (max, sum) in one
// read, results in a second.
template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_rows_generic_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t D, bool log) {
    const int64_t row = blockIdx.x;
    const typename Elem<T>::storage* xr = x + row * D;
    float m = -INFINITY, s = 0.0f;
    for (int64_t j = threadIdx.x; j < D; j += kBlock) {
        const float v = Elem<T>::load(xr[j]);
        if (v == -INFINITY) continue;  // contributes exp(-inf) = 0
        if (v > m) {
            s = s * exp_fast(m - v) + 1.0f;
            m = v;
        } else {
            s += exp_fast(v - m);
        }
    }
    block_merge(m, s);
    const float shift = m == -INFINITY ? 0.0f : m;
    const float lse = logf(s);
    const float inv = 1.0f / s;
    typename Elem<T>::storage* yr = y + row * D;
    for (int64_t j = threadIdx.x; j < D; j += kBlock) {
        const float d = Elem<T>::load(xr[j]) - shift;
        yr[j] = Elem<T>::store(log ? d - lse : exp_fast(d) * inv);
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_backward_rows_generic_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy,
    typename Elem<T>::storage* dx, int64_t D, bool log) {
    __shared__ float scratch[kBlock / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * D;
    float s = 0.0f;
    for (int64_t j = threadIdx.x; j < D; j += kBlock) {
        const float g = Elem<T>::load(dy[base + j]);
        s += log ? g : g * Elem<T>::load(y[base + j]);
    }
    s = row_reduce<kBlock / kWave, false>(s, scratch);
    for (int64_t j = threadIdx.x; j < D; j += kBlock) {
        const float a = Elem<T>::load(y[base + j]), g = Elem<T>::load(dy[base + j]);
        dx[base + j] = Elem<T>::store(log ? g - exp_fast(a) * s : a * (g - s));
    }
}

// ---- softmax over a dimension that is not the last ---------------------------
//
// [outer, D, inner] with inner > 1: a block takes 64 consecutive columns of
// one outer index (one a lane, so a wave reads 64 neighbours of a row) and
// one slice of D; its four waves take the slice's rows in turn, eight rows
// loaded together a lane (rows past the slice are clamped and masked, so
// the loads carry no branch).  Per column, the forward keeps a running
// (max, sum of exp) and the backward a running sum; the waves' partials
// fold through LDS in wave order.  With enough column tiles to fill the GPU
// there is one slice and one launch (MODE kColFused); otherwise a first
// launch writes each slice's partials (kColStats) and a second folds them in
// slice order and writes the output (kColWrite).  The earlier kernel gave
// each column to one thread, which walked D alone: 2.4 ms for a dim-0
// softmax of [4096, 4096].
constexpr int kColWaves = 4;
constexpr int kColWidth = kWave;  // columns of a block
constexpr int kColBatch = 8;      // rows loaded together a lane
constexpr int kColFused = 0, kColStats = 1, kColWrite = 2;

struct ColBlock {
    int64_t o, c0, d0, d1, sl;
};

// Block b: column tile b % tiles, slice (b / tiles) % slices, outer index
// b / (tiles * slices).
__device__ __forceinline__ ColBlock col_block(int64_t tiles, int64_t slices, int64_t D, int64_t dslice) {
    ColBlock cb;
    int64_t b = blockIdx.x;
    cb.c0 = (b % tiles) * kColWidth;
    b /= tiles;
    cb.sl = b % slices;
    cb.o = b / slices;
    cb.d0 = cb.sl * dslice;
    cb.d1 = cb.d0 + dslice < D ? cb.d0 + dslice : D;
    return cb;
}

// The larger of a and b, NaN if either is (fmaxf returns the other operand
// for a NaN, which would let a column whose only numbers are NaN and -inf
// look empty and be skipped).
__device__ __forceinline__ float max_keep_nan(float a, float b) { return (a > b || a != a) ? a : b; }

// (m, s) <- (m, s) merged with (m2, s2), each s a sum of exp(v - m).  A NaN
// maximum makes the merged sum NaN, so the column's outputs become NaN.
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
    const float mn = max_keep_nan(m, m2);
    if (mn == -INFINITY) return;
    s = (m == -INFINITY ? 0.0f : s * exp_fast(m - mn)) + (m2 == -INFINITY ? 0.0f : s2 * exp_fast(m2 - mn));
    m = mn;
}

template <typename T, int MODE>
__global__ __launch_bounds__(kColWaves * kWave) void softmax_cols_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, float* pm, float* ps, int64_t outer,
    int64_t D, int64_t inner, int64_t tiles, int64_t slices, int64_t dslice, bool log) {
    __shared__ float sm[kColWaves][kColWidth], ss[kColWaves][kColWidth];
    const ColBlock cb = col_block(tiles, slices, D, dslice);
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    const int64_t c = cb.c0 + lane;
    const bool live = c < inner;
    const int64_t base = cb.o * D * inner + (live ? c : inner - 1);
    const typename Elem<T>::storage* col = x + base;
    float m = -INFINITY, s = 0.0f;
    if constexpr (MODE != kColWrite) {
        for (int64_t d = cb.d0 + w; d < cb.d1; d += kColWaves * kColBatch) {
            float v[kColBatch];
#pragma unroll
            for (int j = 0; j < kColBatch; ++j) {
                const int64_t dj = d + j * kColWaves;
                v[j] = Elem<T>::load(col[(dj < cb.d1 ? dj : cb.d1 - 1) * inner]);
            }
            float bm = -INFINITY;
#pragma unroll
            for (int j = 0; j < kColBatch; ++j) {
                if (d + j * kColWaves >= cb.d1) v[j] = -INFINITY;
                bm = max_keep_nan(bm, v[j]);
            }
            if (bm == -INFINITY) continue;  // only -inf and masked rows: nothing to add
            float bs = 0.0f;
#pragma unroll
            for (int j = 0; j < kColBatch; ++j) bs += exp_fast(v[j] - bm);
            lse_merge(m, s, bm, bs);
        }
        sm[w][lane] = m;
        ss[w][lane] = s;
        __syncthreads();
        m = sm[0][lane];
        s = ss[0][lane];
#pragma unroll
        for (int k = 1; k < kColWaves; ++k) lse_merge(m, s, sm[k][lane], ss[k][lane]);
        if constexpr (MODE == kColStats) {
            if (w == 0 && live) {
                const int64_t at = (cb.sl * outer + cb.o) * inner + c;
                pm[at] = m;
                ps[at] = s;
            }
            return;
        }
    } else {
        const int64_t cc = live ? c : inner - 1;
        for (int64_t k = 0; k < slices; ++k) {
            const int64_t at = (k * outer + cb.o) * inner + cc;
            lse_merge(m, s, pm[at], ps[at]);
        }
    }
    // A column of -inf (or an empty one) would give inf - inf; exp(-inf - 0)
    // keeps it at 0 instead.
    const float shift = m == -INFINITY ? 0.0f : m;
    const float lse = logf(s);
    const float inv = 1.0f / s;
    typename Elem<T>::storage* out = y + base;
    for (int64_t d = cb.d0 + w; d < cb.d1; d += kColWaves * kColBatch) {
        float v[kColBatch];
#pragma unroll
        for (int j = 0; j < kColBatch; ++j) {
            const int64_t dj = d + j * kColWaves;
            v[j] = Elem<T>::load(col[(dj < cb.d1 ? dj : cb.d1 - 1) * inner]) - shift;
        }
#pragma unroll
        for (int j = 0; j < kColBatch; ++j) {
            const int64_t dj = d + j * kColWaves;
            if (live && dj < cb.d1) out[dj * inner] = Elem<T>::store(log ? v[j] - lse : exp_fast(v[j]) * inv);
        }
    }
}

// The backward: per column s = sum over D of dy (log) or dy * y, then
// dx = dy - exp(y) s (log) or y (dy - s).
template <typename T, int MODE>
__global__ __launch_bounds__(kColWaves * kWave) void softmax_backward_cols_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy, typename Elem<T>::storage* dx,
    float* ps, int64_t outer, int64_t D, int64_t inner, int64_t tiles, int64_t slices, int64_t dslice, bool log) {
    __shared__ float ss[kColWaves][kColWidth];
    const ColBlock cb = col_block(tiles, slices, D, dslice);
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    const int64_t c = cb.c0 + lane;
    const bool live = c < inner;
    const int64_t base = cb.o * D * inner + (live ? c : inner - 1);
    const typename Elem<T>::storage* ycol = y + base;
    const typename Elem<T>::storage* gcol = dy + base;
    float s = 0.0f;
    if constexpr (MODE != kColWrite) {
        for (int64_t d = cb.d0 + w; d < cb.d1; d += kColWaves * kColBatch) {
            float a[kColBatch], g[kColBatch];
#pragma unroll
            for (int j = 0; j < kColBatch; ++j) {
                const int64_t dj = d + j * kColWaves;
                const int64_t at = (dj < cb.d1 ? dj : cb.d1 - 1) * inner;
                a[j] = Elem<T>::load(ycol[at]);
                g[j] = Elem<T>::load(gcol[at]);
            }
#pragma unroll
            for (int j = 0; j < kColBatch; ++j) {
                if (d + j * kColWaves < cb.d1) s += log ? g[j] : g[j] * a[j];
            }
        }
        ss[w][lane] = s;
        __syncthreads();
        s = ss[0][lane];
#pragma unroll
        for (int k = 1; k < kColWaves; ++k) s += ss[k][lane];
        if constexpr (MODE == kColStats) {
            if (w == 0 && live) ps[(cb.sl * outer + cb.o) * inner + c] = s;
            return;
        }
    } else {
        const int64_t cc = live ? c : inner - 1;
        for (int64_t k = 0; k < slices; ++k) s += ps[(k * outer + cb.o) * inner + cc];
    }
    typename Elem<T>::storage* out = dx + base;
    for (int64_t d = cb.d0 + w; d < cb.d1; d += kColWaves * kColBatch) {
        float a[kColBatch], g[kColBatch];
#pragma unroll
        for (int j = 0; j < kColBatch; ++j) {
            const int64_t dj = d + j * kColWaves;
            const int64_t at = (dj < cb.d1 ? dj : cb.d1 - 1) * inner;
            a[j] = Elem<T>::load(ycol[at]);
            g[j] = Elem<T>::load(gcol[at]);
        }
#pragma unroll
        for (int j = 0; j < kColBatch; ++j) {
            const int64_t dj = d + j * kColWaves;
            if (live && dj < cb.d1) {
                out[dj * inner] = Elem<T>::store(log ? g[j] - exp_fast(a[j]) * s : a[j] * (g[j] - s));
            }
        }
    }
}

// Tiles, slices and rows a slice for the column kernels: enough blocks for
// two a CU, slices of at least 64 rows.
struct ColPlan {
    int64_t tiles, slices, dslice, blocks;
};

ColPlan col_plan(int64_t outer, int64_t D, int64_t inner, int device) {
    ColPlan p;
    p.tiles = (inner + kColWidth - 1) / kColWidth;
    const int64_t base = outer * p.tiles;
    const int64_t want = 2 * static_cast<int64_t>(cu_count(device));
    int64_t slices = (want + base - 1) / base;
    const int64_t most = (D + 63) / 64;
    if (slices > most) slices = most;
    if (slices < 1) slices = 1;
    p.dslice = (D + slices - 1) / slices;
    p.slices = (D + p.dslice - 1) / p.dslice;
    p.blocks = base * p.slices;
    return p;
}

// ---- configuration choice ---------------------------------------------------

// A register-resident layout; waves == 0 means the long-row kernel.
struct RowConfig {
    int waves, ept;
};

template <typename T, int W, int E>
void launch_forward_rows(int device, const void* x, void* y, int64_t rows, int64_t D, bool log) {
    using S = typename Elem<T>::storage;
    const int64_t blocks = (rows + rows_per_block<W>() - 1) / rows_per_block<W>();
    softmax_rows_kernel<T, W, E><<<blocks, block_threads<W>(), 0, stream(device)>>>(
        static_cast<const S*>(x), static_cast<S*>(y), rows, D, log);
}

template <typename T, int W, int E>
void launch_backward_rows(int device, const void* y, const void* dy, void* dx, int64_t rows,
                          int64_t D, bool log) {
    using S = typename Elem<T>::storage;
    const int64_t blocks = (rows + rows_per_block<W>() - 1) / rows_per_block<W>();
    softmax_backward_rows_kernel<T, W, E><<<blocks, block_threads<W>(), 0, stream(device)>>>(
        static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), rows, D, log);
}

// The layouts compiled, as (waves per row, packets per thread): the
// measured best on MI355X puts about two 16-byte packets in each thread and
// grows the number of waves with the row, up to 16 (a 1024-thread block);
// longer rows then take more packets per thread, up to 32 float32 values.
#define TP_AMD_SOFTMAX_CONFIGS(X) \
    X(1, 1) X(1, 2) X(2, 2) X(4, 2) X(8, 2) X(16, 2) X(16, 4) X(16, 8)

template <typename T>
bool launch_forward_config(RowConfig c, int device, const void* x, void* y, int64_t rows,
                           int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
#define TP_AMD_FWD(W, V)                                                             \
    if constexpr (V * N <= 32) {                                                     \
        if (c.waves == W && c.ept == V * N) {                                        \
            launch_forward_rows<T, W, V * N>(device, x, y, rows, D, log);            \
            return true;                                                             \
        }                                                                            \
    }
    TP_AMD_SOFTMAX_CONFIGS(TP_AMD_FWD)
#undef TP_AMD_FWD
    return false;
}

template <typename T>
bool launch_backward_config(RowConfig c, int device, const void* y, const void* dy, void* dx,
                            int64_t rows, int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
#define TP_AMD_BWD(W, V)                                                             \
    if constexpr (V * N <= 32) {                                                     \
        if (c.waves == W && c.ept == V * N) {                                        \
            launch_backward_rows<T, W, V * N>(device, y, dy, dx, rows, D, log);      \
            return true;                                                             \
        }                                                                            \
    }
    TP_AMD_SOFTMAX_CONFIGS(TP_AMD_BWD)
#undef TP_AMD_BWD
    return false;
}

// The compiled layout for a row of D elements (waves == 0: none holds it).
template <typename T>
RowConfig choose_config(int64_t D) {
    constexpr int N = Packet<T>::N;
    constexpr int kPairs[][2] = {{1, 1}, {1, 2}, {2, 2}, {4, 2}, {8, 2}, {16, 2}, {16, 4}, {16, 8}};
    const int64_t npk = (D + N - 1) / N;
    for (const auto& c : kPairs) {
        if (c[1] * N > 32) break;
        if (static_cast<int64_t>(c[0]) * kWave * c[1] >= npk) return RowConfig{c[0], c[1] * N};
    }
    return RowConfig{0, 0};
}

template <typename T>
void softmax_typed(int device, bool log, int64_t outer, int64_t D, int64_t inner, const void* x,
                   void* y) {
    using S = typename Elem<T>::storage;
    constexpr int N = Packet<T>::N;
    hipStream_t st = stream(device);
    if (inner == 1) {
        const bool vec = D % N == 0 && aligned16(x) && aligned16(y);
        const RowConfig c = choose_config<T>(D);
        if (vec && c.waves == 16) {
            // Rows that need a whole block: one block per CU walks them.
            const int64_t grid = outer < cu_count(device) ? outer : cu_count(device);
            const int vpt = c.ept / N;
            if (vpt <= 2) {
                softmax_rows_stream_kernel<T, 2><<<grid, 16 * kWave, 0, st>>>(
                    static_cast<const S*>(x), static_cast<S*>(y), outer, D, log);
            } else if (vpt <= 4) {
                softmax_rows_stream_kernel<T, 4><<<grid, 16 * kWave, 0, st>>>(
                    static_cast<const S*>(x), static_cast<S*>(y), outer, D, log);
            } else if constexpr (N == 4) {
                softmax_rows_stream_kernel<T, 8><<<grid, 16 * kWave, 0, st>>>(
                    static_cast<const S*>(x), static_cast<S*>(y), outer, D, log);
            }
        } else if (vec && c.waves > 0) {
            launch_forward_config<T>(c, device, x, y, outer, D, log);
        } else if (vec) {
            softmax_rows_long_kernel<T, 4><<<outer, kBlock, 0, st>>>(
                static_cast<const S*>(x), static_cast<S*>(y), D, log);
        } else {
            softmax_rows_generic_kernel<T><<<outer, kBlock, 0, st>>>(
                static_cast<const S*>(x), static_cast<S*>(y), D, log);
        }
    } else {
        const ColPlan cp = col_plan(outer, D, inner, device);
        TP_AMD_CHECK(cp.blocks < (int64_t{1} << 31), "softmax: ", cp.blocks, " blocks exceed the grid");
        const unsigned blocks = static_cast<unsigned>(cp.blocks);
        if (cp.slices == 1) {
            softmax_cols_kernel<T, kColFused><<<blocks, kColWaves * kWave, 0, st>>>(
                static_cast<const S*>(x), static_cast<S*>(y), nullptr, nullptr, outer, D, inner, cp.tiles, 1, cp.dslice,
                log);
        } else {
            const size_t parts = static_cast<size_t>(cp.slices * outer * inner);
            Workspace ws(2 * parts * sizeof(float), device);
            float* pm = static_cast<float*>(ws.get());
            float* ps = pm + parts;
            softmax_cols_kernel<T, kColStats><<<blocks, kColWaves * kWave, 0, st>>>(
                static_cast<const S*>(x), nullptr, pm, ps, outer, D, inner, cp.tiles, cp.slices, cp.dslice, log);
            softmax_cols_kernel<T, kColWrite><<<blocks, kColWaves * kWave, 0, st>>>(
                static_cast<const S*>(x), static_cast<S*>(y), pm, ps, outer, D, inner, cp.tiles, cp.slices, cp.dslice,
                log);
        }
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template <typename T>
void softmax_backward_typed(int device, bool log, int64_t outer, int64_t D, int64_t inner,
                            const void* y, const void* dy, void* dx) {
    using S = typename Elem<T>::storage;
    constexpr int N = Packet<T>::N;
    hipStream_t st = stream(device);
    if (inner == 1) {
        const bool vec = D % N == 0 && aligned16(y) && aligned16(dy) && aligned16(dx);
        const RowConfig c = choose_config<T>(D);
        if (vec && c.waves == 16 && c.ept / N <= 4) {
            // Rows that need a whole block: one block per CU walks them.
            const int64_t grid = outer < cu_count(device) ? outer : cu_count(device);
            if (c.ept / N <= 2) {
                softmax_backward_stream_kernel<T, 2><<<grid, 16 * kWave, 0, st>>>(
                    static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), outer, D, log);
            } else {
                softmax_backward_stream_kernel<T, 4><<<grid, 16 * kWave, 0, st>>>(
                    static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), outer, D, log);
            }
        } else if (vec && c.waves > 0) {
            launch_backward_config<T>(c, device, y, dy, dx, outer, D, log);
        } else if (vec) {
            softmax_backward_rows_long_kernel<T, 2><<<outer, kBlock, 0, st>>>(
                static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), D, log);
        } else {
            softmax_backward_rows_generic_kernel<T><<<outer, kBlock, 0, st>>>(
                static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), D, log);
        }
    } else {
        const ColPlan cp = col_plan(outer, D, inner, device);
        TP_AMD_CHECK(cp.blocks < (int64_t{1} << 31), "softmax backward: ", cp.blocks, " blocks exceed the grid");
        const unsigned blocks = static_cast<unsigned>(cp.blocks);
        if (cp.slices == 1) {
            softmax_backward_cols_kernel<T, kColFused><<<blocks, kColWaves * kWave, 0, st>>>(
                static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), nullptr, outer, D, inner,
                cp.tiles, 1, cp.dslice, log);
        } else {
            Workspace ws(static_cast<size_t>(cp.slices * outer * inner) * sizeof(float), device);
            float* ps = static_cast<float*>(ws.get());
            softmax_backward_cols_kernel<T, kColStats><<<blocks, kColWaves * kWave, 0, st>>>(
                static_cast<const S*>(y), static_cast<const S*>(dy), nullptr, ps, outer, D, inner, cp.tiles,
                cp.slices, cp.dslice, log);
            softmax_backward_cols_kernel<T, kColWrite><<<blocks, kColWaves * kWave, 0, st>>>(
                static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), ps, outer, D, inner,
                cp.tiles, cp.slices, cp.dslice, log);
        }
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace

}  // namespace tp_amd

using namespace tp_amd;

extern "C" {

int tp_amd_launch_softmax(int device, int log, int dtype, int64_t outer, int64_t dim,
                          int64_t inner, const void* x, void* y) {
    return guarded([&] {
        TP_AMD_CHECK(outer >= 0 && dim >= 0 && inner >= 0, "negative softmax extent");
        if (outer == 0 || dim == 0 || inner == 0) return;
        TP_AMD_CHECK(outer <= 0x7fffffff, "softmax: too many rows");
        const OnDevice scope(device);
        const int index = scope.index();
        switch (dtype) {
            case TP_AMD_FLOAT32: softmax_typed<float>(index, log != 0, outer, dim, inner, x, y); break;
            case TP_AMD_BFLOAT16: softmax_typed<bf16_t>(index, log != 0, outer, dim, inner, x, y); break;
            case TP_AMD_FLOAT16: softmax_typed<f16_t>(index, log != 0, outer, dim, inner, x, y); break;
            default:
                TP_AMD_CHECK(false, "softmax takes float32, float16 or bfloat16, got ",
                             dtype_name(dtype));
        }
    });
}

int tp_amd_launch_softmax_backward(int device, int log, int dtype, int64_t outer, int64_t dim,
                                   int64_t inner, const void* y, const void* dy, void* dx) {
    return guarded([&] {
        TP_AMD_CHECK(outer >= 0 && dim >= 0 && inner >= 0, "negative softmax extent");
        if (outer == 0 || dim == 0 || inner == 0) return;
        TP_AMD_CHECK(outer <= 0x7fffffff, "softmax: too many rows");
        const OnDevice scope(device);
        const int index = scope.index();
        switch (dtype) {
            case TP_AMD_FLOAT32:
                softmax_backward_typed<float>(index, log != 0, outer, dim, inner, y, dy, dx);
                break;
            case TP_AMD_BFLOAT16:
                softmax_backward_typed<bf16_t>(index, log != 0, outer, dim, inner, y, dy, dx);
                break;
            case TP_AMD_FLOAT16:
                softmax_backward_typed<f16_t>(index, log != 0, outer, dim, inner, y, dy, dx);
                break;
            default:
                TP_AMD_CHECK(false, "softmax takes float32, float16 or bfloat16, got ",
                             dtype_name(dtype));
        }
    });
}

}  // extern "C"
