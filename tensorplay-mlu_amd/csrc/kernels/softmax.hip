// Fused softmax / log_softmax forward and backward for gfx950 (the
// reference's cnnlSoftmaxForward / cnnlSoftmaxBackward,
// tensorplay_mlu/csrc/ReduceKernels.cpp:171-199).
//
// Rows along the last axis (inner == 1) are held in registers: each row is
// read from HBM once and written once.  WAVES wavefronts share a row and
// each thread keeps VPT 16-byte packets of it, so rows up to
// 64 * WAVES * VPT * N elements (65536 fp32 forward, 32768 fp32 backward)
// stay on chip; the row max and the exponential sum combine across lanes
// with shuffles and across waves in LDS.  Rows too long for that, or whose
// length is not a multiple of the packet, take a block-per-row kernel that
// keeps a running (max, sum) pair and reads the row twice.  Softmax over a
// leading axis (inner > 1) walks the reduced axis with the contiguous inner
// axis across threads.

#include <cmath>

#include "device_common.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) v = fmaxf(v, wave_shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) v += wave_shfl_xor(v, m);
    return v;
}

// Reduce ``v`` over the WAVES waves that share a row (WAVES > 1: the whole
// block is one row).  ``scratch`` holds one float per wave.
template <int WAVES, bool MAX>
__device__ __forceinline__ float row_reduce(float v, float* scratch) {
    v = MAX ? wave_max(v) : wave_sum(v);
    if constexpr (WAVES > 1) {
        const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
        __syncthreads();  // scratch may still be read from the previous use
        if (lane == 0) scratch[wave] = v;
        __syncthreads();
        float t = lane < WAVES ? scratch[lane] : (MAX ? -INFINITY : 0.0f);
        v = MAX ? wave_max(t) : wave_sum(t);
    }
    return v;
}

// Block size for a config: one wave per row packs 4 rows into 256 threads.
template <int WAVES>
constexpr int block_threads() {
    return WAVES == 1 ? kBlock : WAVES * kWave;
}

template <typename T, int WAVES, int VPT>
__global__ __launch_bounds__(block_threads<WAVES>()) void softmax_rows_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t rows, int64_t D,
    bool log) {
    constexpr int N = Packet<T>::N;
    constexpr int kRowsPerBlock = WAVES == 1 ? kBlock / kWave : 1;
    constexpr int kThreads = WAVES * kWave;
    __shared__ float scratch[WAVES > 1 ? WAVES : 1];
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock +
                        (WAVES == 1 ? threadIdx.x / kWave : 0);
    const int tid = WAVES == 1 ? threadIdx.x % kWave : threadIdx.x;
    const bool active = row < rows;  // uniform per wave
    const int64_t npk = D / N;
    const typename Elem<T>::storage* xr = x + (active ? row : 0) * D;
    float v[VPT][N];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (active && q < npk) {
            const Packet<T> p = load_packet_nt<T>(xr + q * N);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                v[k][j] = Elem<T>::load(p.v[j]);
                m = fmaxf(m, v[k][j]);
            }
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
            v[k][j] = log ? v[k][j] - shift : expf(v[k][j] - shift);
            s += log ? expf(v[k][j]) : v[k][j];
        }
    s = row_reduce<WAVES, false>(s, scratch);
    const float lse = logf(s);
    if (!active) return;
    typename Elem<T>::storage* yr = y + row * D;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (q < npk) {
            Packet<T> p;
#pragma unroll
            for (int j = 0; j < N; ++j) p.v[j] = Elem<T>::store(log ? v[k][j] - lse : v[k][j] / s);
            store_packet_nt<T>(yr + q * N, p);
        }
    }
}

template <typename T, int WAVES, int VPT>
__global__ __launch_bounds__(block_threads<WAVES>()) void softmax_backward_rows_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy,
    typename Elem<T>::storage* dx, int64_t rows, int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
    constexpr int kRowsPerBlock = WAVES == 1 ? kBlock / kWave : 1;
    constexpr int kThreads = WAVES * kWave;
    __shared__ float scratch[WAVES > 1 ? WAVES : 1];
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock +
                        (WAVES == 1 ? threadIdx.x / kWave : 0);
    const int tid = WAVES == 1 ? threadIdx.x % kWave : threadIdx.x;
    const bool active = row < rows;
    const int64_t npk = D / N;
    const int64_t base = (active ? row : 0) * D;
    float a[VPT][N], g[VPT][N];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (active && q < npk) {
            const Packet<T> py = load_packet_nt<T>(y + base + q * N);
            const Packet<T> pg = load_packet_nt<T>(dy + base + q * N);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                a[k][j] = Elem<T>::load(py.v[j]);
                g[k][j] = Elem<T>::load(pg.v[j]);
                s += log ? g[k][j] : g[k][j] * a[k][j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) a[k][j] = g[k][j] = 0.0f;
        }
    }
    s = row_reduce<WAVES, false>(s, scratch);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (q < npk) {
            Packet<T> p;
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float r = log ? g[k][j] - expf(a[k][j]) * s : a[k][j] * (g[k][j] - s);
                p.v[j] = Elem<T>::store(r);
            }
            store_packet_nt<T>(dx + base + q * N, p);
        }
    }
}

// Any row length: block per row, running (max, sum) in one read, results in
// a second.  Used for rows not a multiple of the packet or beyond the
// register-resident configs.
__device__ __forceinline__ void online_merge(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;  // both empty
    s = s * expf(m - mn) + s2 * expf(m2 - mn);
    m = mn;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_rows_generic_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t D, bool log) {
    __shared__ float sm[kBlock / kWave], ss[kBlock / kWave];
    const int64_t row = blockIdx.x;
    const typename Elem<T>::storage* xr = x + row * D;
    float m = -INFINITY, s = 0.0f;
    for (int64_t j = threadIdx.x; j < D; j += kBlock) {
        const float v = Elem<T>::load(xr[j]);
        if (v == -INFINITY) continue;  // contributes exp(-inf) = 0
        if (v > m) {
            s = s * expf(m - v) + 1.0f;
            m = v;
        } else {
            s += expf(v - m);
        }
    }
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
    for (int w = 1; w < kBlock / kWave; ++w) online_merge(m, s, sm[w], ss[w]);
    const float shift = m == -INFINITY ? 0.0f : m;
    const float lse = logf(s);
    typename Elem<T>::storage* yr = y + row * D;
    for (int64_t j = threadIdx.x; j < D; j += kBlock) {
        const float v = Elem<T>::load(xr[j]) - shift;
        yr[j] = Elem<T>::store(log ? v - lse : expf(v) / s);
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
        dx[base + j] = Elem<T>::store(log ? g - expf(a) * s : a * (g - s));
    }
}

// inner > 1: thread per (outer, inner) position, walking D with stride inner.
template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_strided_kernel(
    const typename Elem<T>::storage* x, typename Elem<T>::storage* y, int64_t outer, int64_t D,
    int64_t inner, bool log) {
    const int64_t total = outer * inner;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; t < total;
         t += stride) {
        const int64_t o = t / inner, i = t - o * inner;
        const int64_t base = o * D * inner + i;
        float m = -INFINITY, s = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
            const float v = Elem<T>::load(x[base + d * inner]);
            if (v == -INFINITY) continue;  // contributes exp(-inf) = 0
            if (v > m) {
                s = s * expf(m - v) + 1.0f;
                m = v;
            } else {
                s += expf(v - m);
            }
        }
        const float shift = m == -INFINITY ? 0.0f : m;
        const float lse = logf(s);
        for (int64_t d = 0; d < D; ++d) {
            const float v = Elem<T>::load(x[base + d * inner]) - shift;
            y[base + d * inner] = Elem<T>::store(log ? v - lse : expf(v) / s);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_backward_strided_kernel(
    const typename Elem<T>::storage* y, const typename Elem<T>::storage* dy,
    typename Elem<T>::storage* dx, int64_t outer, int64_t D, int64_t inner, bool log) {
    const int64_t total = outer * inner;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; t < total;
         t += stride) {
        const int64_t o = t / inner, i = t - o * inner;
        const int64_t base = o * D * inner + i;
        float s = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
            const float g = Elem<T>::load(dy[base + d * inner]);
            s += log ? g : g * Elem<T>::load(y[base + d * inner]);
        }
        for (int64_t d = 0; d < D; ++d) {
            const float a = Elem<T>::load(y[base + d * inner]);
            const float g = Elem<T>::load(dy[base + d * inner]);
            dx[base + d * inner] = Elem<T>::store(log ? g - expf(a) * s : a * (g - s));
        }
    }
}

// Register-resident configurations (WAVES, VPT), smallest capacity first.
struct RowConfig {
    int waves, vpt;
};
constexpr RowConfig kForwardConfigs[] = {{1, 1}, {1, 2}, {1, 4},  {1, 8},  {1, 16},
                                         {4, 8}, {4, 16}, {16, 8}, {16, 16}};
constexpr RowConfig kBackwardConfigs[] = {{1, 1}, {1, 2}, {1, 4}, {1, 8},
                                          {4, 4}, {4, 8}, {16, 4}, {16, 8}};

template <typename T, int W, int V>
void launch_forward_rows(int device, const void* x, void* y, int64_t rows, int64_t D, bool log) {
    using S = typename Elem<T>::storage;
    constexpr int rows_per_block = W == 1 ? kBlock / kWave : 1;
    const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
    softmax_rows_kernel<T, W, V><<<blocks, block_threads<W>(), 0, stream(device)>>>(
        static_cast<const S*>(x), static_cast<S*>(y), rows, D, log);
}

template <typename T, int W, int V>
void launch_backward_rows(int device, const void* y, const void* dy, void* dx, int64_t rows,
                          int64_t D, bool log) {
    using S = typename Elem<T>::storage;
    constexpr int rows_per_block = W == 1 ? kBlock / kWave : 1;
    const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
    softmax_backward_rows_kernel<T, W, V><<<blocks, block_threads<W>(), 0, stream(device)>>>(
        static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), rows, D, log);
}

template <typename T>
bool forward_rows_resident(int device, const void* x, void* y, int64_t rows, int64_t D,
                           bool log) {
    constexpr int N = Packet<T>::N;
    for (const RowConfig& c : kForwardConfigs) {
        if (static_cast<int64_t>(c.waves) * kWave * c.vpt * N < D) continue;
#define TP_AMD_FWD(W, V)                                                            \
    if (c.waves == W && c.vpt == V) {                                               \
        launch_forward_rows<T, W, V>(device, x, y, rows, D, log);                   \
        return true;                                                                \
    }
        TP_AMD_FWD(1, 1) TP_AMD_FWD(1, 2) TP_AMD_FWD(1, 4) TP_AMD_FWD(1, 8) TP_AMD_FWD(1, 16)
        TP_AMD_FWD(4, 8) TP_AMD_FWD(4, 16) TP_AMD_FWD(16, 8) TP_AMD_FWD(16, 16)
#undef TP_AMD_FWD
    }
    return false;
}

template <typename T>
bool backward_rows_resident(int device, const void* y, const void* dy, void* dx, int64_t rows,
                            int64_t D, bool log) {
    constexpr int N = Packet<T>::N;
    for (const RowConfig& c : kBackwardConfigs) {
        if (static_cast<int64_t>(c.waves) * kWave * c.vpt * N < D) continue;
#define TP_AMD_BWD(W, V)                                                            \
    if (c.waves == W && c.vpt == V) {                                               \
        launch_backward_rows<T, W, V>(device, y, dy, dx, rows, D, log);             \
        return true;                                                                \
    }
        TP_AMD_BWD(1, 1) TP_AMD_BWD(1, 2) TP_AMD_BWD(1, 4) TP_AMD_BWD(1, 8)
        TP_AMD_BWD(4, 4) TP_AMD_BWD(4, 8) TP_AMD_BWD(16, 4) TP_AMD_BWD(16, 8)
#undef TP_AMD_BWD
    }
    return false;
}

int64_t strided_grid(int64_t total, int device) {
    const int64_t want = (total + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(cu_count(device)) * 32;
    return want < cap ? (want > 0 ? want : 1) : cap;
}

template <typename T>
void softmax_typed(int device, bool log, int64_t outer, int64_t D, int64_t inner, const void* x,
                   void* y) {
    using S = typename Elem<T>::storage;
    constexpr int N = Packet<T>::N;
    hipStream_t st = stream(device);
    if (inner == 1) {
        const bool vec = D % N == 0 && aligned16(x) && aligned16(y);
        if (!(vec && forward_rows_resident<T>(device, x, y, outer, D, log))) {
            softmax_rows_generic_kernel<T><<<outer, kBlock, 0, st>>>(
                static_cast<const S*>(x), static_cast<S*>(y), D, log);
        }
    } else {
        softmax_strided_kernel<T><<<strided_grid(outer * inner, device), kBlock, 0, st>>>(
            static_cast<const S*>(x), static_cast<S*>(y), outer, D, inner, log);
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
        if (!(vec && backward_rows_resident<T>(device, y, dy, dx, outer, D, log))) {
            softmax_backward_rows_generic_kernel<T><<<outer, kBlock, 0, st>>>(
                static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), D, log);
        }
    } else {
        softmax_backward_strided_kernel<T><<<strided_grid(outer * inner, device), kBlock, 0, st>>>(
            static_cast<const S*>(y), static_cast<const S*>(dy), static_cast<S*>(dx), outer, D,
            inner, log);
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
        const int index = resolve_device(device);
        DeviceGuard guard(index);
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
        const int index = resolve_device(device);
        DeviceGuard guard(index);
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
