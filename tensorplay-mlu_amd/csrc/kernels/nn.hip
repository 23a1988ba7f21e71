// Neural-network layers for gfx950: layer norm forward and backward, dropout
// on a Philox4x32-10 stream, embedding lookup and its dense gradient, and the
// negative log-likelihood loss forward and backward (the reference's CNNL
// calls in tensorplay_mlu/csrc/NNKernels.cpp:57-395).
//
// Layer norm keeps a row in registers: WAVES wavefronts per row, VPT 16-byte
// packets per thread, so a row is read once and written once.  Statistics
// are float32 whatever the storage (the reference's stats_dtype, :52-54).
// The backward walks rows with a grid of a few blocks per CU; each thread
// keeps its columns' running dW and dB, and the blocks' float32 partials are
// folded by a column reduction afterwards.
//
// Indices that fall outside their table (an embedding index, an NLL target
// that is not ignore_index) are never dereferenced: the lookup writes NaN
// for that row and the loss counts NaN for that sample, so the result shows
// the error instead of the kernel reading out of bounds.

#include <cmath>
#include <type_traits>

#include "device_common.h"
#include "../allocator.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kBlock = 256;

template <typename T>
using S_ = typename Elem<T>::storage;

struct Plus {
    __device__ float operator()(float a, float b) const { return a + b; }
};

// The float32 value as computed.  Without it the compiler folds a final
// multiply into the 16-bit conversion as fma(a, b, +0), which rounds once
// instead of through float32 and turns a -0 product into +0.
__device__ __forceinline__ float opaque(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// ---- layer norm -------------------------------------------------------------

template <int WAVES>
constexpr int ln_threads() {
    return WAVES * kWave < kBlock ? kBlock : WAVES * kWave;
}

// Sum over the WAVES waves of one row (rows of a block are independent).
template <int WAVES>
__device__ __forceinline__ float row_sum(float v, float* scratch) {
    v = wave_allreduce(v, Plus{});
    if constexpr (WAVES > 1) {
        const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
        const int first = (wave / WAVES) * WAVES;
        __syncthreads();  // the previous use of scratch is done
        if (lane == 0) scratch[wave] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) t += scratch[first + w];
        v = t;
    }
    return v;
}

template <typename T, int VPT>
__device__ __forceinline__ void load_params(const S_<T>* p, float (&out)[VPT][Packet<T>::N],
                                            int tid, int threads, int64_t npk, float fallback) {
    constexpr int N = Packet<T>::N;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * threads;
        if (p != nullptr && q < npk) {
            unpack<T>(*reinterpret_cast<const uint4*>(p + q * N), out[k]);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) out[k][j] = fallback;
        }
    }
}

// y = (x - mean) rstd w + b over rows of D (a multiple of the packet).
template <typename T, int WAVES, int VPT>
__global__ __launch_bounds__(ln_threads<WAVES>()) void layer_norm_rows_kernel(
    const S_<T>* x, const S_<T>* w, const S_<T>* b, S_<T>* y, float* mean_out, float* rstd_out,
    int64_t rows, int64_t D, float eps) {
    constexpr int N = Packet<T>::N;
    constexpr int kThreads = WAVES * kWave;
    constexpr int kRows = ln_threads<WAVES>() / kThreads;
    __shared__ float scratch[ln_threads<WAVES>() / kWave];
    const int tid = threadIdx.x % kThreads;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRows + threadIdx.x / kThreads;
    const bool active = row < rows;
    const int64_t npk = D / N;
    float v[VPT][N];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (active && q < npk) {
            unpack<T>(load_raw_nt(x + row * D + q * N), v[k]);
#pragma unroll
            for (int j = 0; j < N; ++j) s += v[k][j];
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) v[k][j] = 0.0f;
        }
    }
    const float inv_d = 1.0f / static_cast<float>(D);
    const float mean = row_sum<WAVES>(s, scratch) * inv_d;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (active && q < npk) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float d = v[k][j] - mean;
                ss += d * d;
            }
        }
    }
    const float var = row_sum<WAVES>(ss, scratch) * inv_d;
    const float rstd = 1.0f / sqrtf(var + eps);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
        if (q < npk) {
            float wv[N], bv[N], o[N];
            if (w != nullptr) unpack<T>(*reinterpret_cast<const uint4*>(w + q * N), wv);
            if (b != nullptr) unpack<T>(*reinterpret_cast<const uint4*>(b + q * N), bv);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float t = (v[k][j] - mean) * rstd;
                o[j] = fmaf(t, w != nullptr ? wv[j] : 1.0f, b != nullptr ? bv[j] : 0.0f);
            }
            store_raw_nt(y + row * D + q * N, pack<T>(o));
        }
    }
    if (tid == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// Any D and alignment: a block per row, reading the row twice (once for the
// statistics, once for the output; the second read hits L2).
template <typename T>
__global__ __launch_bounds__(kBlock) void layer_norm_generic_kernel(
    const S_<T>* x, const S_<T>* w, const S_<T>* b, S_<T>* y, float* mean_out, float* rstd_out,
    int64_t D, float eps) {
    __shared__ float scratch[kBlock / kWave];
    const int64_t row = blockIdx.x;
    const S_<T>* xr = x + row * D;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < D; i += kBlock) s += Elem<T>::load(xr[i]);
    const float inv_d = 1.0f / static_cast<float>(D);
    const float mean = row_sum<kBlock / kWave>(s, scratch) * inv_d;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < D; i += kBlock) {
        const float d = Elem<T>::load(xr[i]) - mean;
        ss += d * d;
    }
    const float rstd = 1.0f / sqrtf(row_sum<kBlock / kWave>(ss, scratch) * inv_d + eps);
    for (int64_t i = threadIdx.x; i < D; i += kBlock) {
        const float t = (Elem<T>::load(xr[i]) - mean) * rstd;
        const float wv = w != nullptr ? Elem<T>::load(w[i]) : 1.0f;
        const float bv = b != nullptr ? Elem<T>::load(b[i]) : 0.0f;
        y[row * D + i] = Elem<T>::store(fmaf(t, wv, bv));
    }
    if (threadIdx.x == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// Backward over rows of D (a multiple of the packet).  Block b takes rows
// b, b + gridDim.x, ...; per row
//   xhat = (x - mean) rstd,  g = dy w,
//   dx = rstd (g - mean(g) - xhat mean(g xhat)),
// and each thread adds dy xhat and dy into its columns' running sums, written
// at the end as the block's float32 partial rows of dW and dB.
template <typename T, int WAVES, int VPT>
__global__ __launch_bounds__(WAVES * kWave) void layer_norm_backward_rows_kernel(
    const S_<T>* dy, const S_<T>* x, const float* mean, const float* rstd, const S_<T>* w,
    S_<T>* dx, float* dw_part, float* db_part, int64_t rows, int64_t D) {
    constexpr int N = Packet<T>::N;
    constexpr int kThreads = WAVES * kWave;
    __shared__ float scratch[WAVES];
    const int tid = threadIdx.x;
    const int64_t npk = D / N;
    float wv[VPT][N], pw[VPT][N], pb[VPT][N];
    load_params<T, VPT>(w, wv, tid, kThreads, npk, 1.0f);
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
        for (int j = 0; j < N; ++j) pw[k][j] = pb[k][j] = 0.0f;
    const float inv_d = 1.0f / static_cast<float>(D);
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const float mu = mean[row], rs = rstd[row];
        float xh[VPT][N], g[VPT][N];
        float a = 0.0f, c = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
            if (q < npk) {
                float xv[N], dv[N];
                unpack<T>(load_raw_nt(x + row * D + q * N), xv);
                unpack<T>(load_raw_nt(dy + row * D + q * N), dv);
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    xh[k][j] = (xv[j] - mu) * rs;
                    g[k][j] = dv[j] * wv[k][j];
                    a += g[k][j];
                    c += g[k][j] * xh[k][j];
                    pw[k][j] = fmaf(dv[j], xh[k][j], pw[k][j]);
                    pb[k][j] += dv[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < N; ++j) xh[k][j] = g[k][j] = 0.0f;
            }
        }
        a = row_sum<WAVES>(a, scratch) * inv_d;
        c = row_sum<WAVES>(c, scratch) * inv_d;
        if (dx != nullptr) {
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
                const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
                if (q < npk) {
                    float o[N];
#pragma unroll
                    for (int j = 0; j < N; ++j) o[j] = rs * (g[k][j] - a - xh[k][j] * c);
                    store_raw_nt(dx + row * D + q * N, pack<T>(o));
                }
            }
        }
    }
    if (dw_part != nullptr) {
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
            if (q < npk) {
                float* pwr = dw_part + static_cast<int64_t>(blockIdx.x) * D + q * N;
                float* pbr = db_part + static_cast<int64_t>(blockIdx.x) * D + q * N;
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    pwr[j] = pw[k][j];
                    pbr[j] = pb[k][j];
                }
            }
        }
    }
}

// Any D: a block per row for dx, reading x and dy twice.
template <typename T>
__global__ __launch_bounds__(kBlock) void layer_norm_backward_generic_kernel(
    const S_<T>* dy, const S_<T>* x, const float* mean, const float* rstd, const S_<T>* w,
    S_<T>* dx, int64_t D) {
    __shared__ float scratch[kBlock / kWave];
    const int64_t row = blockIdx.x;
    const float mu = mean[row], rs = rstd[row];
    float a = 0.0f, c = 0.0f;
    for (int64_t i = threadIdx.x; i < D; i += kBlock) {
        const float xh = (Elem<T>::load(x[row * D + i]) - mu) * rs;
        const float g = Elem<T>::load(dy[row * D + i]) * (w != nullptr ? Elem<T>::load(w[i]) : 1.0f);
        a += g;
        c += g * xh;
    }
    const float inv_d = 1.0f / static_cast<float>(D);
    a = row_sum<kBlock / kWave>(a, scratch) * inv_d;
    c = row_sum<kBlock / kWave>(c, scratch) * inv_d;
    for (int64_t i = threadIdx.x; i < D; i += kBlock) {
        const float xh = (Elem<T>::load(x[row * D + i]) - mu) * rs;
        const float g = Elem<T>::load(dy[row * D + i]) * (w != nullptr ? Elem<T>::load(w[i]) : 1.0f);
        dx[row * D + i] = Elem<T>::store(rs * (g - a - xh * c));
    }
}

// dW and dB for any D: column j of the block's column range summed over all
// rows (a thread per column, rows strided over the block's row groups).
template <typename T>
__global__ __launch_bounds__(kBlock) void layer_norm_param_grad_generic_kernel(
    const S_<T>* dy, const S_<T>* x, const float* mean, const float* rstd, float* dw, float* db,
    int64_t rows, int64_t D) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= D) return;
    float sw = 0.0f, sb = 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const float g = Elem<T>::load(dy[r * D + j]);
        sw = fmaf(g, (Elem<T>::load(x[r * D + j]) - mean[r]) * rstd[r], sw);
        sb += g;
    }
    dw[j] = sw;
    db[j] = sb;
}

// Sum over `parts` float32 rows of D columns, in row order, rounded to T.
template <typename T>
__global__ __launch_bounds__(kBlock) void fold_rows_kernel(const float* part, int64_t parts, int64_t D,
                                                           S_<T>* out) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= D) return;
    float s = 0.0f;
    for (int64_t p = 0; p < parts; ++p) s += part[p * D + j];
    out[j] = Elem<T>::store(s);
}

struct RowShape {
    int waves = 0;  // 0: no register layout holds the row
    int vpt = 0;
};

// Smallest (waves, packets per thread) holding npk packets, up to 16 waves
// of max_vpt packets (one wave takes 1, 2, ... max_vpt; more waves take
// max_vpt).
RowShape row_shape(int64_t npk, int max_vpt) {
    for (int waves : {1, 2, 4, 8, 16}) {
        for (int vpt : {1, 2, 4}) {
            if (vpt > max_vpt || (waves > 1 && vpt < max_vpt)) continue;
            if (static_cast<int64_t>(waves) * kWave * vpt >= npk) return RowShape{waves, vpt};
        }
    }
    return RowShape{};
}

// The forward holds up to 4 packets a thread; the backward, which keeps five
// float arrays per thread, 4 of float32 and 2 of a 16-bit type.
#define TP_AMD_LN_SHAPES(X) \
    X(1, 1) X(1, 2) X(1, 4) X(2, 2) X(2, 4) X(4, 2) X(4, 4) X(8, 2) X(8, 4) X(16, 2) X(16, 4)
template <typename T>
constexpr int bwd_max_vpt() {
    return Packet<T>::N == 4 ? 4 : 2;
}

template <typename T>
void layer_norm_typed(int device, int64_t rows, int64_t D, const void* xv, const void* wv,
                      const void* bv, void* yv, float* mean, float* rstd, float eps) {
    using S = S_<T>;
    constexpr int N = Packet<T>::N;
    const S* x = static_cast<const S*>(xv);
    const S* w = static_cast<const S*>(wv);
    const S* b = static_cast<const S*>(bv);
    S* y = static_cast<S*>(yv);
    hipStream_t st = stream(device);
    const bool vec = D % N == 0 && aligned16(x) && aligned16(y) && (w == nullptr || aligned16(w)) &&
                     (b == nullptr || aligned16(b));
    const RowShape rs = vec ? row_shape(D / N, 4) : RowShape{};
#define TP_AMD_LN_FWD(W, V)                                                                      \
    if constexpr (W == 1 || V == 4) {                                                            \
        if (rs.waves == W && rs.vpt == V) {                                                      \
            constexpr int kRows = ln_threads<W>() / (W * kWave);                                 \
            const int64_t blocks = (rows + kRows - 1) / kRows;                                   \
            layer_norm_rows_kernel<T, W, V><<<blocks, ln_threads<W>(), 0, st>>>(                 \
                x, w, b, y, mean, rstd, rows, D, eps);                                           \
            TP_AMD_HIP_CHECK(hipGetLastError());                                                 \
            return;                                                                              \
        }                                                                                        \
    }
    TP_AMD_LN_SHAPES(TP_AMD_LN_FWD)
#undef TP_AMD_LN_FWD
    layer_norm_generic_kernel<T><<<rows, kBlock, 0, st>>>(x, w, b, y, mean, rstd, D, eps);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template <typename T>
void layer_norm_backward_typed(int device, int64_t rows, int64_t D, const void* dyv, const void* xv,
                               const float* mean, const float* rstd, const void* wv, void* dxv,
                               void* dwv, void* dbv) {
    using S = S_<T>;
    constexpr int N = Packet<T>::N;
    const S* dy = static_cast<const S*>(dyv);
    const S* x = static_cast<const S*>(xv);
    const S* w = static_cast<const S*>(wv);
    S* dx = static_cast<S*>(dxv);
    hipStream_t st = stream(device);
    const bool params = dwv != nullptr || dbv != nullptr;
    const bool vec = D % N == 0 && aligned16(x) && aligned16(dy) && (dx == nullptr || aligned16(dx)) &&
                     (w == nullptr || aligned16(w));
    const RowShape shape = vec ? row_shape(D / N, bwd_max_vpt<T>()) : RowShape{};
    if (shape.waves > 0) {
        // A few blocks per CU walk the rows; each leaves one partial row of
        // dW and of dB.
        const int64_t per_cu = shape.waves >= 4 ? 2 : 8;
        int64_t grid = static_cast<int64_t>(cu_count(device)) * per_cu;
        if (grid > rows) grid = rows;
        Workspace ws(params ? static_cast<size_t>(2 * grid * D) * sizeof(float) : 0, device);
        float* dw_part = params ? static_cast<float*>(ws.get()) : nullptr;
        float* db_part = params ? dw_part + grid * D : nullptr;
#define TP_AMD_LN_BWD(W, V)                                                                    \
    if constexpr (V <= bwd_max_vpt<T>() && (W == 1 || V == bwd_max_vpt<T>())) {                \
        if (shape.waves == W && shape.vpt == V) {                                              \
            layer_norm_backward_rows_kernel<T, W, V><<<grid, W * kWave, 0, st>>>(              \
                dy, x, mean, rstd, w, dx, dw_part, db_part, rows, D);                          \
        }                                                                                      \
    }
        TP_AMD_LN_SHAPES(TP_AMD_LN_BWD)
#undef TP_AMD_LN_BWD
        TP_AMD_HIP_CHECK(hipGetLastError());
        if (params) {
            const int64_t blocks = (D + kBlock - 1) / kBlock;
            Workspace tmp;
            if (dwv == nullptr || dbv == nullptr) tmp = Workspace(static_cast<size_t>(D) * sizeof(S), device);
            fold_rows_kernel<T><<<blocks, kBlock, 0, st>>>(dw_part, grid, D,
                                                           static_cast<S*>(dwv ? dwv : tmp.get()));
            fold_rows_kernel<T><<<blocks, kBlock, 0, st>>>(db_part, grid, D,
                                                           static_cast<S*>(dbv ? dbv : tmp.get()));
            TP_AMD_HIP_CHECK(hipGetLastError());
        }
        return;
    }
    if (dx != nullptr) {
        layer_norm_backward_generic_kernel<T><<<rows, kBlock, 0, st>>>(dy, x, mean, rstd, w, dx, D);
        TP_AMD_HIP_CHECK(hipGetLastError());
    }
    if (params) {
        Workspace ws(static_cast<size_t>(2 * D) * sizeof(float), device);
        float* dwf = static_cast<float*>(ws.get());
        float* dbf = dwf + D;
        const int64_t blocks = (D + kBlock - 1) / kBlock;
        layer_norm_param_grad_generic_kernel<T><<<blocks, kBlock, 0, st>>>(dy, x, mean, rstd, dwf, dbf,
                                                                           rows, D);
        Workspace tmp;
        if (dwv == nullptr || dbv == nullptr) tmp = Workspace(static_cast<size_t>(D) * sizeof(S), device);
        fold_rows_kernel<T><<<blocks, kBlock, 0, st>>>(dwf, 1, D, static_cast<S*>(dwv ? dwv : tmp.get()));
        fold_rows_kernel<T><<<blocks, kBlock, 0, st>>>(dbf, 1, D, static_cast<S*>(dbv ? dbv : tmp.get()));
        TP_AMD_HIP_CHECK(hipGetLastError());
    }
}

// ---- dropout: Philox4x32-10 -------------------------------------------------
//
// The counter-based generator of Salmon, Moraes, Dror and Shaw, "Parallel
// random numbers: as easy as 1, 2, 3" (SC 2011): ten rounds of two 32 x 32
// -> 64-bit multiplies on a 4-word counter under a 2-word key bumped by the
// Weyl constants after each round.  Element e of a tensor takes word e % 4
// of the block for counter (e / 4, 0, offset_lo, offset_hi) under the key
// (seed_lo, seed_hi); its uniform is (word >> 8) * 2^-24 in [0, 1), and it is
// kept when the uniform is >= p, decided exactly as word >> 8 >= ceil(p 2^24).

struct Philox {
    uint32_t c[4];
};

__device__ __forceinline__ Philox philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                uint32_t k0, uint32_t k1) {
    constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = static_cast<uint64_t>(M0) * c0;
        const uint64_t p1 = static_cast<uint64_t>(M1) * c2;
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
        k0 += W0;
        k1 += W1;
    }
    return Philox{{c0, c1, c2, c3}};
}

// Four elements per thread (one Philox block): out = keep ? x * scale : 0,
// mask = keep.
template <typename T>
__global__ __launch_bounds__(kBlock) void dropout_kernel(const S_<T>* x, S_<T>* out, uint8_t* mask,
                                                         int64_t n, uint32_t threshold, float scale,
                                                         uint32_t k0, uint32_t k1, uint32_t off0,
                                                         uint32_t off1) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;  // Philox block
    const int64_t e0 = g * 4;
    if (e0 >= n) return;
    const Philox r = philox4x32_10(static_cast<uint32_t>(g), static_cast<uint32_t>(g >> 32), off0, off1,
                                   k0, k1);
    const bool full = e0 + 4 <= n;
    uint8_t m[4];
    float xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        m[j] = (r.c[j] >> 8) >= threshold ? 1 : 0;
        xv[j] = (full || e0 + j < n) ? Elem<T>::load(x[e0 + j]) : 0.0f;
    }
    if (full) {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[e0 + j] = Elem<T>::store(m[j] ? opaque(xv[j] * scale) : 0.0f);
        uint32_t packed = m[0] | (m[1] << 8) | (m[2] << 16) | (static_cast<uint32_t>(m[3]) << 24);
        if ((reinterpret_cast<uintptr_t>(mask + e0) & 3u) == 0) {
            *reinterpret_cast<uint32_t*>(mask + e0) = packed;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) mask[e0 + j] = m[j];
        }
    } else {
        for (int j = 0; j < 4 && e0 + j < n; ++j) {
            out[e0 + j] = Elem<T>::store(m[j] ? opaque(xv[j] * scale) : 0.0f);
            mask[e0 + j] = m[j];
        }
    }
}

// out = grad * mask * scale (mask bytes 0 / 1).
template <typename T>
__global__ __launch_bounds__(kBlock) void dropout_backward_kernel(const S_<T>* grad, const uint8_t* mask,
                                                                  S_<T>* out, int64_t n, float scale) {
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = i0 + j;
        if (i < n) {
            const float m = mask[i] != 0 ? 1.0f : 0.0f;
            out[i] = Elem<T>::store(opaque(Elem<T>::load(grad[i]) * m * scale));
        }
    }
}

// ---- embedding ---------------------------------------------------------------

template <typename I>
__device__ __forceinline__ int64_t index_at(const void* idx, int64_t i) {
    return static_cast<int64_t>(static_cast<const I*>(idx)[i]);
}

// out[i, :] = weight[idx[i], :]; a wave per index.  An index outside
// [0, V) writes a NaN row.
template <typename T, typename I, bool VEC>
__global__ __launch_bounds__(kBlock) void embedding_kernel(const S_<T>* weight, const void* idx,
                                                           S_<T>* out, int64_t n, int64_t V,
                                                           int64_t D) {
    constexpr int N = VEC ? Packet<T>::N : 1;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (i >= n) return;
    const int64_t r = index_at<I>(idx, i);
    const bool ok = r >= 0 && r < V;
    const int64_t units = D / N;
    for (int64_t q = lane; q < units; q += kWave) {
        if constexpr (VEC) {
            uint4 v;
            if (ok) {
                v = *reinterpret_cast<const uint4*>(weight + r * D + q * N);
            } else {
                float nan[N];
#pragma unroll
                for (int j = 0; j < N; ++j) nan[j] = __builtin_nanf("");
                v = pack<T>(nan);
            }
            store_raw_nt(out + i * D + q * N, v);
        } else {
            out[i * D + q] = ok ? weight[r * D + q] : Elem<T>::store(__builtin_nanf(""));
        }
    }
}

// counts[idx[i]] += 1 for valid, non-padding indices.
template <typename I>
__global__ __launch_bounds__(kBlock) void embedding_count_kernel(const void* idx, int64_t n, int64_t V,
                                                                 int64_t padding_idx, int* counts) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const int64_t r = index_at<I>(idx, i);
    if (r >= 0 && r < V && r != padding_idx) atomicAdd(&counts[r], 1);
}

// acc[idx[i], :] += dy[i, :] (divided by the index's count with
// scale_grad_by_freq); a wave per index, float32 atomics.
template <typename T, typename I>
__global__ __launch_bounds__(kBlock) void embedding_backward_kernel(const S_<T>* dy, const void* idx,
                                                                    int64_t n, int64_t V, int64_t D,
                                                                    int64_t padding_idx,
                                                                    const int* counts, float* acc) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (i >= n) return;
    const int64_t r = index_at<I>(idx, i);
    if (r < 0 || r >= V || r == padding_idx) return;
    const float scale = counts != nullptr ? 1.0f / static_cast<float>(counts[r]) : 1.0f;
    for (int64_t q = lane; q < D; q += kWave) {
        atomicAdd(&acc[r * D + q], Elem<T>::load(dy[i * D + q]) * scale);
    }
}

// A float32 buffer to T (or a plain copy for float32), n elements.
template <typename T>
__global__ __launch_bounds__(kBlock) void store_from_float_kernel(const float* src, S_<T>* dst, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i < n) dst[i] = Elem<T>::store(src[i]);
}

__global__ __launch_bounds__(kBlock) void zero_words_kernel(uint32_t* p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// ---- negative log-likelihood -------------------------------------------------

// Per sample: loss_i = -w[t_i] x[i, t_i] and its weight w[t_i] (0 and 0 for
// ignore_index, NaN for a target outside [0, C)).  reduction 0 writes
// y[i]; otherwise each block writes its (sum loss, sum weight) to part.
template <typename T, typename I>
__global__ __launch_bounds__(kBlock) void nll_kernel(const S_<T>* x, const void* target, const S_<T>* w,
                                                     int64_t n, int64_t C, int64_t ignore_index,
                                                     int reduction, S_<T>* y, float* part) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    float loss = 0.0f, wt = 0.0f;
    if (i < n) {
        const int64_t t = index_at<I>(target, i);
        if (t != ignore_index) {
            if (t >= 0 && t < C) {
                wt = w != nullptr ? Elem<T>::load(w[t]) : 1.0f;
                loss = -wt * Elem<T>::load(x[i * C + t]);
            } else {
                loss = wt = __builtin_nanf("");
            }
        }
        if (reduction == 0) y[i] = Elem<T>::store(loss);
    }
    if (reduction == 0) return;
    __shared__ float s_loss[kBlock / kWave], s_wt[kBlock / kWave];
    loss = wave_allreduce(loss, Plus{});
    wt = wave_allreduce(wt, Plus{});
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) {
        s_loss[wave] = loss;
        s_wt[wave] = wt;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = 0.0f, b = 0.0f;
        for (int k = 0; k < kBlock / kWave; ++k) {
            a += s_loss[k];
            b += s_wt[k];
        }
        part[2 * blockIdx.x] = a;
        part[2 * blockIdx.x + 1] = b;
    }
}

// The block partials summed in order: y = sum loss (/ sum weight for the
// mean), total = sum weight.
template <typename T>
__global__ void nll_finish_kernel(const float* part, int64_t blocks, int reduction, S_<T>* y,
                                  S_<T>* total) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float a = 0.0f, b = 0.0f;
    for (int64_t k = 0; k < blocks; ++k) {
        a += part[2 * k];
        b += part[2 * k + 1];
    }
    y[0] = Elem<T>::store(reduction == 1 ? a / b : a);
    total[0] = Elem<T>::store(b);
}

// dx[i, c] = (c == t_i) ? -w[t_i] g_i : 0, with g_i = grad[i] (reduction
// none), grad[0] / total (mean) or grad[0] (sum); a NaN row for a target
// outside [0, C) that is not ignore_index.
template <typename T, typename I>
__global__ __launch_bounds__(kBlock) void nll_backward_kernel(const S_<T>* grad, const void* target,
                                                              const S_<T>* w, const S_<T>* total,
                                                              int64_t n, int64_t C, int64_t ignore_index,
                                                              int reduction, S_<T>* dx) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (e >= n * C) return;
    const int64_t i = e / C, c = e - i * C;
    const int64_t t = index_at<I>(target, i);
    float v = 0.0f;
    if (t != ignore_index) {
        if (t < 0 || t >= C) {
            v = __builtin_nanf("");
        } else if (c == t) {
            const float g = reduction == 0 ? Elem<T>::load(grad[i])
                            : reduction == 1 ? Elem<T>::load(grad[0]) / Elem<T>::load(total[0])
                                             : Elem<T>::load(grad[0]);
            v = -(w != nullptr ? Elem<T>::load(w[t]) : 1.0f) * g;
        }
    }
    dx[e] = Elem<T>::store(opaque(v));
}

template <typename T, typename F>
void dispatch_index(int index_dtype, F&& f) {
    if (index_dtype == TP_AMD_INT64) {
        f(int64_t{});
    } else if (index_dtype == TP_AMD_INT32) {
        f(int32_t{});
    } else {
        TP_AMD_CHECK(false, "indices must be int32 or int64, got ", dtype_name(index_dtype));
    }
}

int64_t blocks_for(int64_t n, int64_t per_block) { return (n + per_block - 1) / per_block; }

}  // namespace

}  // namespace tp_amd

using namespace tp_amd;

#define TP_AMD_DISPATCH_NN(dtype, T, ...)                                                  \
    switch (dtype) {                                                                       \
        case TP_AMD_FLOAT32: { using T = float; __VA_ARGS__; break; }                      \
        case TP_AMD_BFLOAT16: { using T = bf16_t; __VA_ARGS__; break; }                    \
        case TP_AMD_FLOAT16: { using T = f16_t; __VA_ARGS__; break; }                      \
        default: TP_AMD_CHECK(false, "takes float32, float16 or bfloat16, got ",          \
                              dtype_name(dtype));                                          \
    }

extern "C" {

int tp_amd_launch_layer_norm(int device, int dtype, int64_t rows, int64_t dim, const void* x,
                             const void* weight, const void* bias, double eps, void* y, float* mean,
                             float* rstd) {
    return guarded([&] {
        TP_AMD_CHECK(rows >= 0 && dim > 0, "layer_norm: bad extent");
        if (rows == 0) return;
        TP_AMD_CHECK(rows <= 0x7fffffff, "layer_norm: too many rows");
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        TP_AMD_DISPATCH_NN(dtype, T, layer_norm_typed<T>(index, rows, dim, x, weight, bias, y, mean, rstd,
                                                         static_cast<float>(eps)));
    });
}

int tp_amd_launch_layer_norm_backward(int device, int dtype, int64_t rows, int64_t dim,
                                      const void* grad_out, const void* x, const float* mean,
                                      const float* rstd, const void* weight, void* dx, void* dweight,
                                      void* dbias) {
    return guarded([&] {
        TP_AMD_CHECK(rows >= 0 && dim > 0, "layer_norm_backward: bad extent");
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        if (rows == 0) {
            // No rows: the parameter gradients are zero.
            TP_AMD_DISPATCH_NN(dtype, T, {
                Workspace z(static_cast<size_t>(dim) * sizeof(float), index);
                zero_words_kernel<<<blocks_for(dim, kBlock), kBlock, 0, stream(index)>>>(
                    static_cast<uint32_t*>(z.get()), dim);
                for (void* p : {dweight, dbias}) {
                    if (p != nullptr) {
                        store_from_float_kernel<T><<<blocks_for(dim, kBlock), kBlock, 0, stream(index)>>>(
                            static_cast<const float*>(z.get()), static_cast<S_<T>*>(p), dim);
                    }
                }
            });
            TP_AMD_HIP_CHECK(hipGetLastError());
            return;
        }
        TP_AMD_CHECK(rows <= 0x7fffffff, "layer_norm_backward: too many rows");
        TP_AMD_DISPATCH_NN(dtype, T, layer_norm_backward_typed<T>(index, rows, dim, grad_out, x, mean, rstd,
                                                                  weight, dx, dweight, dbias));
    });
}

int tp_amd_launch_dropout(int device, int dtype, int64_t n, const void* x, double p, uint64_t seed,
                          uint64_t offset, void* out, uint8_t* mask) {
    return guarded([&] {
        TP_AMD_CHECK(n >= 0 && p >= 0.0 && p < 1.0, "dropout: need 0 <= p < 1");
        if (n == 0) return;
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        const float scale = static_cast<float>(1.0 / (1.0 - p));
        // p 2^24 is exact in double; a 24-bit uniform u 2^-24 is >= p exactly
        // when u >= ceil(p 2^24) (at most 2^24, which keeps nothing).
        const uint32_t threshold = static_cast<uint32_t>(std::ceil(std::ldexp(p, 24)));
        const int64_t blocks = blocks_for((n + 3) / 4, kBlock);
        TP_AMD_DISPATCH_NN(dtype, T, {
            dropout_kernel<T><<<blocks, kBlock, 0, stream(index)>>>(
                static_cast<const S_<T>*>(x), static_cast<S_<T>*>(out), mask, n, threshold, scale,
                static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32),
                static_cast<uint32_t>(offset), static_cast<uint32_t>(offset >> 32));
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_dropout_backward(int device, int dtype, int64_t n, const void* grad,
                                   const uint8_t* mask, double scale, void* out) {
    return guarded([&] {
        TP_AMD_CHECK(n >= 0, "dropout_backward: negative extent");
        if (n == 0) return;
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        const int64_t blocks = blocks_for((n + 3) / 4, kBlock);
        TP_AMD_DISPATCH_NN(dtype, T, {
            dropout_backward_kernel<T><<<blocks, kBlock, 0, stream(index)>>>(
                static_cast<const S_<T>*>(grad), mask, static_cast<S_<T>*>(out), n,
                static_cast<float>(scale));
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_embedding(int device, int dtype, int64_t num_weights, int64_t dim, const void* weight,
                            int index_dtype, int64_t n, const void* indices, void* out) {
    return guarded([&] {
        TP_AMD_CHECK(num_weights >= 0 && dim >= 0 && n >= 0, "embedding: negative extent");
        if (n == 0 || dim == 0) return;
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        const int64_t blocks = blocks_for(n, kBlock / kWave);
        TP_AMD_DISPATCH_NN(dtype, T, {
            const bool vec = dim % Packet<T>::N == 0 && aligned16(weight) && aligned16(out);
            dispatch_index<T>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                if (vec) {
                    embedding_kernel<T, I, true><<<blocks, kBlock, 0, stream(index)>>>(
                        static_cast<const S_<T>*>(weight), indices, static_cast<S_<T>*>(out), n,
                        num_weights, dim);
                } else {
                    embedding_kernel<T, I, false><<<blocks, kBlock, 0, stream(index)>>>(
                        static_cast<const S_<T>*>(weight), indices, static_cast<S_<T>*>(out), n,
                        num_weights, dim);
                }
            });
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_embedding_backward(int device, int dtype, int64_t n, int64_t dim, const void* grad,
                                     int index_dtype, const void* indices, int64_t num_weights,
                                     int64_t padding_idx, int scale_grad_by_freq, void* out) {
    return guarded([&] {
        TP_AMD_CHECK(num_weights >= 0 && dim >= 0 && n >= 0, "embedding_backward: negative extent");
        if (num_weights == 0 || dim == 0) return;
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        hipStream_t st = stream(index);
        const int64_t total = num_weights * dim;
        TP_AMD_DISPATCH_NN(dtype, T, {
            // float32 accumulates in place; 16-bit types in a float32 buffer.
            const bool in_place = std::is_same<T, float>::value;
            Workspace acc_ws(in_place ? 0 : static_cast<size_t>(total) * sizeof(float), index);
            float* acc = in_place ? static_cast<float*>(out) : static_cast<float*>(acc_ws.get());
            zero_words_kernel<<<blocks_for(total, kBlock), kBlock, 0, st>>>(reinterpret_cast<uint32_t*>(acc),
                                                                             total);
            Workspace count_ws(scale_grad_by_freq ? static_cast<size_t>(num_weights) * sizeof(int) : 0, index);
            int* counts = scale_grad_by_freq ? static_cast<int*>(count_ws.get()) : nullptr;
            if (n > 0) {
                dispatch_index<T>(index_dtype, [&](auto tag) {
                    using I = decltype(tag);
                    if (counts != nullptr) {
                        zero_words_kernel<<<blocks_for(num_weights, kBlock), kBlock, 0, st>>>(
                            reinterpret_cast<uint32_t*>(counts), num_weights);
                        embedding_count_kernel<I><<<blocks_for(n, kBlock), kBlock, 0, st>>>(
                            indices, n, num_weights, padding_idx, counts);
                    }
                    embedding_backward_kernel<T, I><<<blocks_for(n, kBlock / kWave), kBlock, 0, st>>>(
                        static_cast<const S_<T>*>(grad), indices, n, num_weights, dim, padding_idx, counts,
                        acc);
                });
            }
            if (!in_place) {
                store_from_float_kernel<T><<<blocks_for(total, kBlock), kBlock, 0, st>>>(
                    acc, static_cast<S_<T>*>(out), total);
            }
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_nll_loss(int device, int dtype, int64_t n, int64_t classes, const void* x,
                           int index_dtype, const void* target, const void* weight, int reduction,
                           int64_t ignore_index, void* y, void* total_weight) {
    return guarded([&] {
        TP_AMD_CHECK(n > 0 && classes > 0, "nll_loss: empty input");
        TP_AMD_CHECK(reduction >= 0 && reduction <= 2, "nll_loss: reduction must be 0, 1 or 2");
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        hipStream_t st = stream(index);
        const int64_t blocks = blocks_for(n, kBlock);
        TP_AMD_DISPATCH_NN(dtype, T, {
            Workspace part(reduction == 0 ? 0 : static_cast<size_t>(2 * blocks) * sizeof(float), index);
            dispatch_index<T>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                nll_kernel<T, I><<<blocks, kBlock, 0, st>>>(
                    static_cast<const S_<T>*>(x), target, static_cast<const S_<T>*>(weight), n, classes,
                    ignore_index, reduction, static_cast<S_<T>*>(y), static_cast<float*>(part.get()));
            });
            if (reduction != 0) {
                nll_finish_kernel<T><<<1, kWave, 0, st>>>(static_cast<const float*>(part.get()), blocks,
                                                          reduction, static_cast<S_<T>*>(y),
                                                          static_cast<S_<T>*>(total_weight));
            }
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_nll_loss_backward(int device, int dtype, int64_t n, int64_t classes, const void* grad,
                                    int index_dtype, const void* target, const void* weight,
                                    int reduction, int64_t ignore_index, const void* total_weight,
                                    void* dx) {
    return guarded([&] {
        TP_AMD_CHECK(n > 0 && classes > 0, "nll_loss_backward: empty input");
        TP_AMD_CHECK(reduction >= 0 && reduction <= 2, "nll_loss_backward: reduction must be 0, 1 or 2");
        const int index = resolve_device(device);
        DeviceGuard guard(index);
        const int64_t blocks = blocks_for(n * classes, kBlock);
        TP_AMD_DISPATCH_NN(dtype, T, {
            dispatch_index<T>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                nll_backward_kernel<T, I><<<blocks, kBlock, 0, stream(index)>>>(
                    static_cast<const S_<T>*>(grad), target, static_cast<const S_<T>*>(weight),
                    static_cast<const S_<T>*>(total_weight), n, classes, ignore_index, reduction,
                    static_cast<S_<T>*>(dx));
            });
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

}  // extern "C"
