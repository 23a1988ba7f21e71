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

// Two sums at once, each added in the same order as `row_sum` (so the same
// bits), with one pair of barriers; scratch holds 2 floats a wave.
template <int WAVES>
__device__ __forceinline__ void row_sum2(float& a, float& c, float* scratch) {
    a = wave_allreduce(a, Plus{});
    c = wave_allreduce(c, Plus{});
    if constexpr (WAVES > 1) {
        const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
        const int first = (wave / WAVES) * WAVES;
        __syncthreads();  // the previous use of scratch is done
        if (lane == 0) {
            scratch[2 * wave] = a;
            scratch[2 * wave + 1] = c;
        }
        __syncthreads();
        float ta = 0.0f, tc = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            ta += scratch[2 * (first + w)];
            tc += scratch[2 * (first + w) + 1];
        }
        a = ta;
        c = tc;
    }
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

// y = (x - mean) rstd w + b over rows of D (a multiple of the packet; a row
// and the statistics arrays under 4 GiB).  A block holds kRows rows at a time
// (WAVES waves each) and walks rows with stride gridDim.x kRows, two rows a
// step in two register sets: the next row's packets are loaded before this
// row's reductions, so the loads stay in flight across the barriers.  w and b
// stay in registers as packets.  Rows load with the default cache policy
// ([8192, 4096] bf16: 22.5 us, 25.9 us with non-temporal loads).
template <typename T, int WAVES, int VPT>
__global__ __launch_bounds__(ln_threads<WAVES>()) void layer_norm_rows_kernel(
    const S_<T>* x, const S_<T>* w, const S_<T>* b, S_<T>* y, float* mean_out, float* rstd_out,
    int64_t rows, int64_t D, float eps) {
    constexpr int N = Packet<T>::N;
    constexpr int kThreads = WAVES * kWave;
    constexpr int kRows = ln_threads<WAVES>() / kThreads;
    __shared__ float scratch[ln_threads<WAVES>() / kWave];
    const int tid = threadIdx.x % kThreads;
    const int group = threadIdx.x / kThreads;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kRows;
    const uint32_t row_bytes = static_cast<uint32_t>(D * sizeof(S_<T>));
    const int64_t npk = D / N;
    const float inv_d = 1.0f / static_cast<float>(D);
    const Rsrc stats_m = buffer_over(mean_out, static_cast<uint32_t>(rows * sizeof(float)));
    const Rsrc stats_r = buffer_over(rstd_out, static_cast<uint32_t>(rows * sizeof(float)));
    uint4 wr[VPT], br[VPT];
    {
        const Rsrc rw = buffer_over(w, w != nullptr ? row_bytes : 0);
        const Rsrc rb = buffer_over(b, b != nullptr ? row_bytes : 0);
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const uint32_t off = static_cast<uint32_t>(tid + k * kThreads) * 16u;
            wr[k] = buffer_load16_cached(rw, off);
            br[k] = buffer_load16_cached(rb, off);
        }
    }
    auto fetch = [&](uint4 (&buf)[VPT], int64_t row) {
        const Rsrc r = buffer_over(x + (row < rows ? row : 0) * D, row < rows ? row_bytes : 0);
#pragma unroll
        for (int k = 0; k < VPT; ++k) buf[k] = buffer_load16_cached(r, static_cast<uint32_t>(tid + k * kThreads) * 16u);
    };
    auto process = [&](const uint4 (&buf)[VPT], int64_t row) {
        float v[VPT][N];
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            unpack<T>(buf[k], v[k]);  // zeros past the row's end
#pragma unroll
            for (int j = 0; j < N; ++j) s += v[k][j];
        }
        const float mean = row_sum<WAVES>(s, scratch) * inv_d;
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const bool in = tid + k * kThreads < npk;
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float d = in ? v[k][j] - mean : 0.0f;
                ss += d * d;
            }
        }
        const float var = row_sum<WAVES>(ss, scratch) * inv_d;
        const float rstd = 1.0f / sqrtf(var + eps);
        const bool active = row < rows;
        const Rsrc ry = buffer_over(y + (active ? row : 0) * D, active ? row_bytes : 0);
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            float wv[N], bv[N], o[N];
            unpack<T>(wr[k], wv);
            unpack<T>(br[k], bv);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const float t = (v[k][j] - mean) * rstd;
                o[j] = fmaf(t, w != nullptr ? wv[j] : 1.0f, b != nullptr ? bv[j] : 0.0f);
            }
            buffer_store16(ry, static_cast<uint32_t>(tid + k * kThreads) * 16u, pack<T>(o));
        }
        const uint32_t stat_off = tid == 0 && active ? static_cast<uint32_t>(row) * 4u : kOutOfRange;
        buffer_store_f32(stats_m, stat_off, mean);
        buffer_store_f32(stats_r, stat_off, rstd);
    };
    uint4 a[VPT], bq[VPT];
    const int64_t first = static_cast<int64_t>(blockIdx.x) * kRows;
    fetch(a, uniform(first + group));
    drain();
    for (int64_t base = first; base < rows; base += 2 * stride) {
        fetch(bq, uniform(base + stride + group));
        process(a, uniform(base + group));
        if (base + stride >= rows) break;
        fetch(a, uniform(base + 2 * stride + group));
        process(bq, uniform(base + stride + group));
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

// Backward over rows of D (a multiple of the packet; a row and the
// statistics under 4 GiB).  A block is GROUPS row groups of WAVES waves; group
// g of block b takes rows (b GROUPS + g) + i gridDim.x GROUPS.  Per row
//   xhat = (x - mean) rstd,  g = dy w,
//   dx = rstd (g - mean(g) - xhat mean(g xhat)),
// and each thread adds dy xhat and dy into its columns' running sums.  Rows
// go two a step in two register sets of raw packets: the next row's x and dy
// (and statistics) are loaded before this row's reductions, so the loads
// stay in flight across the barriers; xhat and g are recomputed from the
// packets for dx.  At the end the groups' running sums are added in order
// through LDS (D floats of dynamic shared memory) into the block's float32
// partial rows of dW and dB.

// The blocks' partial rows of dW and dB are stored in chunks of kFoldChunk
// columns (128 bytes), a chunk of every block together: chunk c of block b's
// row at (c * blocks + b) * kFoldChunk, so the fold reads each chunk's rows
// as one contiguous run.  The last chunk is padded to kFoldChunk columns.
constexpr int kFoldChunk = 32;

template <typename T, int VPT>
struct BwdRow {
    uint4 x[VPT], d[VPT];
    float mu, rs;
};

template <typename T, int WAVES, int VPT, int GROUPS>
__global__ __launch_bounds__(GROUPS * WAVES * kWave) void layer_norm_backward_rows_kernel(
    const S_<T>* dy, const S_<T>* x, const float* mean, const float* rstd, const S_<T>* w,
    S_<T>* dx, float* dw_part, float* db_part, int64_t rows, int64_t D) {
    constexpr int N = Packet<T>::N;
    constexpr int kThreads = WAVES * kWave;
    extern __shared__ float fold[];
    __shared__ float scratch[2 * GROUPS * WAVES];
    const int tid = threadIdx.x % kThreads;
    const int group = threadIdx.x / kThreads;
    const int64_t npk = D / N;
    const uint32_t row_bytes = static_cast<uint32_t>(D * sizeof(S_<T>));
    const Rsrc rmean = buffer_over(mean, static_cast<uint32_t>(rows * sizeof(float)));
    const Rsrc rrstd = buffer_over(rstd, static_cast<uint32_t>(rows * sizeof(float)));
    uint4 wr[VPT];
    {
        const Rsrc rw = buffer_over(w, w != nullptr ? row_bytes : 0);
#pragma unroll
        for (int k = 0; k < VPT; ++k) wr[k] = buffer_load16_cached(rw, static_cast<uint32_t>(tid + k * kThreads) * 16u);
    }
    float pw[VPT][N], pb[VPT][N];
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
        for (int j = 0; j < N; ++j) pw[k][j] = pb[k][j] = 0.0f;
    const float inv_d = 1.0f / static_cast<float>(D);
    // Row `row`'s packets and statistics (zeros past the last row).
    auto fetch = [&](BwdRow<T, VPT>& buf, int64_t row) {
        const bool ok = row < rows;
        const int64_t at = (ok ? row : 0) * D;
        const Rsrc rx = buffer_over(x + at, ok ? row_bytes : 0);
        const Rsrc rd = buffer_over(dy + at, ok ? row_bytes : 0);
        const uint32_t soff = ok ? static_cast<uint32_t>(row) * 4u : kOutOfRange;
        buf.mu = buffer_load_f32(rmean, soff);
        buf.rs = buffer_load_f32(rrstd, soff);
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const uint32_t off = static_cast<uint32_t>(tid + k * kThreads) * 16u;
            buf.x[k] = buffer_load16_cached(rx, off);
            buf.d[k] = buffer_load16_cached(rd, off);
        }
    };
    // xhat and g of packet k (zeros past the row's end).
    auto terms = [&](const BwdRow<T, VPT>& buf, int k, float (&xh)[N], float (&g)[N], float (&dv)[N]) {
        const bool in = tid + k * kThreads < npk;
        float xv[N], wv[N];
        unpack<T>(buf.x[k], xv);
        unpack<T>(buf.d[k], dv);
        unpack<T>(wr[k], wv);
#pragma unroll
        for (int j = 0; j < N; ++j) {
            xh[j] = in ? (xv[j] - buf.mu) * buf.rs : 0.0f;
            g[j] = dv[j] * (w != nullptr ? wv[j] : 1.0f);
        }
    };
    auto process = [&](const BwdRow<T, VPT>& buf, int64_t row) {
        float a = 0.0f, c = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            float xh[N], g[N], dv[N];
            terms(buf, k, xh, g, dv);
#pragma unroll
            for (int j = 0; j < N; ++j) {
                a += g[j];
                c += g[j] * xh[j];
                pw[k][j] = fmaf(dv[j], xh[j], pw[k][j]);
                pb[k][j] += dv[j];
            }
        }
        row_sum2<WAVES>(a, c, scratch);
        a *= inv_d;
        c *= inv_d;
        const bool write = dx != nullptr && row < rows;
        const Rsrc rdx = buffer_over(dx + (write ? row * D : 0), write ? row_bytes : 0);
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            float xh[N], g[N], dv[N], o[N];
            terms(buf, k, xh, g, dv);
#pragma unroll
            for (int j = 0; j < N; ++j) o[j] = buf.rs * (g[j] - a - xh[j] * c);
            buffer_store16(rdx, static_cast<uint32_t>(tid + k * kThreads) * 16u, pack<T>(o));
        }
    };
    const int64_t first = static_cast<int64_t>(blockIdx.x) * GROUPS;
    const int64_t step = static_cast<int64_t>(gridDim.x) * GROUPS;
    BwdRow<T, VPT> ra, rb;
    fetch(ra, uniform(first + group));
    drain();
    for (int64_t base = first; base < rows; base += 2 * step) {
        fetch(rb, uniform(base + step + group));
        process(ra, uniform(base + group));
        if (base + step >= rows) break;
        fetch(ra, uniform(base + 2 * step + group));
        process(rb, uniform(base + step + group));
    }
    if (dw_part == nullptr) return;
    // Groups 1 .. GROUPS-1 add into `fold` in turn, group 0 adds last and
    // writes the block's partial row; dW then dB.
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        float (&mine)[VPT][N] = which == 0 ? pw : pb;
        float* out = (which == 0 ? dw_part : db_part) + static_cast<int64_t>(blockIdx.x) * kFoldChunk;
        for (int src = GROUPS - 1; src >= 0; --src) {
            if constexpr (GROUPS > 1) __syncthreads();
            if (group == src) {
#pragma unroll
                for (int k = 0; k < VPT; ++k) {
                    const int64_t q = tid + static_cast<int64_t>(k) * kThreads;
                    if (q < npk) {
                        // A packet's N columns lie in one chunk.
                        float* at = out + (q * N / kFoldChunk) * gridDim.x * kFoldChunk + q * N % kFoldChunk;
#pragma unroll
                        for (int j = 0; j < N; ++j) {
                            float v = mine[k][j];
                            if (src < GROUPS - 1) v += fold[q * N + j];
                            if (src > 0) {
                                fold[q * N + j] = v;
                            } else if constexpr (sizeof(S_<T>) == 2) {
                                // 16-bit rows: non-temporal partials, bf16
                                // [8192, 4096] 35.9-36.2 against 36.5-36.8
                                // us (float32 rows: no gain)
                                __builtin_nontemporal_store(v, &at[j]);
                            } else {
                                at[j] = v;
                            }
                        }
                    }
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

// dW and dB partials for any D: a block takes 64 columns (one a lane) and
// one slice of the rows, its four waves the slice's rows in turn, eight rows
// loaded together a lane (rows past the slice clamped and masked); the
// waves' sums fold through LDS in wave order into the slice's partial row,
// stored in the chunked layout fold_rows_kernel reads (`parts` = slices).
// The earlier pass gave each column to one thread walking every row: 733 us
// of the 2048 x 12288 fp32 backward.
constexpr int kParamWaves = 4;
constexpr int kParamBatch = 8;

template <typename T>
__global__ __launch_bounds__(kParamWaves * kWave) void layer_norm_param_grad_generic_kernel(
    const S_<T>* dy, const S_<T>* x, const float* mean, const float* rstd, float* dw_part, float* db_part,
    int64_t rows, int64_t D, int64_t tiles, int64_t slices, int64_t rslice) {
    __shared__ float sw_s[kParamWaves][kWave], sb_s[kParamWaves][kWave];
    const int64_t tile = blockIdx.x % tiles, sl = blockIdx.x / tiles;
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    const int64_t j = tile * kWave + lane;
    const bool live = j < D;
    const int64_t jj = live ? j : D - 1;
    const int64_t r0 = sl * rslice, r1 = r0 + rslice < rows ? r0 + rslice : rows;
    float sw = 0.0f, sb = 0.0f;
    for (int64_t r = r0 + w; r < r1; r += kParamWaves * kParamBatch) {
        float g[kParamBatch], xv[kParamBatch], mu[kParamBatch], rs[kParamBatch];
#pragma unroll
        for (int k = 0; k < kParamBatch; ++k) {
            const int64_t rk = r + k * kParamWaves;
            const int64_t rr = rk < r1 ? rk : r1 - 1;
            g[k] = Elem<T>::load(dy[rr * D + jj]);
            xv[k] = Elem<T>::load(x[rr * D + jj]);
            mu[k] = mean[rr];
            rs[k] = rstd[rr];
        }
#pragma unroll
        for (int k = 0; k < kParamBatch; ++k) {
            if (r + k * kParamWaves < r1) {
                sw = fmaf(g[k], (xv[k] - mu[k]) * rs[k], sw);
                sb += g[k];
            }
        }
    }
    sw_s[w][lane] = sw;
    sb_s[w][lane] = sb;
    __syncthreads();
    if (w == 0 && live) {
        for (int k = 1; k < kParamWaves; ++k) {
            sw += sw_s[k][lane];
            sb += sb_s[k][lane];
        }
        const int64_t at = ((j / kFoldChunk) * slices + sl) * kFoldChunk + j % kFoldChunk;
        dw_part[at] = sw;
        db_part[at] = sb;
    }
}

// Sum over `parts` float32 rows of D columns, stored in chunks of
// kFoldChunk columns (above), rounded to T: blockIdx.y picks the matrix
// (0: part0 into out0, 1: part1 into out1; a null output is skipped).  The
// fold reads a few MB just written and is bound by latency, so a block is
// two waves on one chunk (a thread takes four columns, one 16-byte load a
// row, in kFoldGroups row groups) and each thread has kFoldBatch loads in
// flight: group g adds rows g, g + kFoldGroups, ... kFoldBatch at a time
// into as many running sums, which are then added pairwise, and the groups
// in a pairwise tree, so the result does not depend on timing.  Measured
// against 1024-thread blocks over 64 columns of the plain [parts][D] layout
// (whose per-row bounds branch left one load in flight at a time): 4.6
// against 4.8 us for 2 x 256 rows of 4096, the whole backward 1-2 us faster.
constexpr int kFoldQuads = kFoldChunk / 4;
constexpr int kFoldGroups = 16;
constexpr int kFoldThreads = kFoldQuads * kFoldGroups;
constexpr int kFoldBatch = 16;

// Floats of a [parts][D] partial in the chunked layout.
inline int64_t fold_floats(int64_t parts, int64_t D) {
    return parts * ((D + kFoldChunk - 1) / kFoldChunk) * kFoldChunk;
}

template <typename T>
__global__ __launch_bounds__(kFoldThreads) void fold_rows_kernel(const float* part0, const float* part1,
                                                                 int64_t parts, int64_t D, S_<T>* out0,
                                                                 S_<T>* out1) {
    __shared__ float4 sums[kFoldGroups][kFoldQuads];
    S_<T>* out = blockIdx.y == 0 ? out0 : out1;
    if (out == nullptr) return;
    const int quad = threadIdx.x % kFoldQuads, grp = threadIdx.x / kFoldQuads;
    const int64_t j0 = (static_cast<int64_t>(blockIdx.x) * kFoldQuads + quad) * 4;
    // This block's chunk: `parts` rows of kFoldQuads 16-byte quads.  Quads
    // past D in the last chunk hold padding, read and never stored.
    const float4* part = reinterpret_cast<const float4*>(blockIdx.y == 0 ? part0 : part1) +
                         static_cast<int64_t>(blockIdx.x) * parts * kFoldQuads + quad;
    float acc[kFoldBatch][4];
#pragma unroll
    for (int l = 0; l < kFoldBatch; ++l) acc[l][0] = acc[l][1] = acc[l][2] = acc[l][3] = 0.0f;
    int64_t p = grp;
    for (; p + (kFoldBatch - 1) * kFoldGroups < parts; p += kFoldBatch * kFoldGroups) {
        float4 v[kFoldBatch];
#pragma unroll
        for (int l = 0; l < kFoldBatch; ++l) v[l] = part[(p + l * kFoldGroups) * kFoldQuads];
        // Keep the loads together: left alone, the scheduler issues two and
        // waits for them before the next two.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int l = 0; l < kFoldBatch; ++l) {
            acc[l][0] += v[l].x;
            acc[l][1] += v[l].y;
            acc[l][2] += v[l].z;
            acc[l][3] += v[l].w;
        }
    }
    for (; p < parts; p += kFoldGroups) {
        const float4 v = part[p * kFoldQuads];
        acc[0][0] += v.x;
        acc[0][1] += v.y;
        acc[0][2] += v.z;
        acc[0][3] += v.w;
    }
#pragma unroll
    for (int h = kFoldBatch / 2; h >= 1; h /= 2) {
#pragma unroll
        for (int l = 0; l < h; ++l) {
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[l][k] += acc[l + h][k];
        }
    }
    sums[grp][quad] = make_float4(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
    // pairwise tree over the groups
#pragma unroll
    for (int h = kFoldGroups / 2; h >= 1; h /= 2) {
        __syncthreads();
        if (grp < h) {
            const float4 u = sums[grp + h][quad];
            float4& t = sums[grp][quad];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
    }
    __syncthreads();
    if (grp == 0) {
        const float4 t = sums[0][quad];
        const float r[4] = {t.x, t.y, t.z, t.w};
        for (int k = 0; k < 4; ++k) {
            if (j0 + k < D) out[j0 + k] = Elem<T>::store(r[k]);
        }
    }
}

inline dim3 fold_grid(int64_t D) {
    return dim3(static_cast<uint32_t>((D + 4 * kFoldQuads - 1) / (4 * kFoldQuads)), 2);
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

// The backward's shape: 8 elements a thread (fp32 2 packets, 16-bit 1) on
// the fewest waves, up to 16, that hold the row.
constexpr int bwd_vpt(int elems) { return 8 / elems; }

RowShape backward_row_shape(int64_t npk, int elems) {
    const int vpt = bwd_vpt(elems);
    for (int waves : {1, 2, 4, 8, 16}) {
        if (static_cast<int64_t>(waves) * kWave * vpt >= npk) return RowShape{waves, vpt};
    }
    return RowShape{};
}

// The forward holds up to 4 packets a thread.
#define TP_AMD_LN_SHAPES(X) \
    X(1, 1) X(1, 2) X(1, 4) X(2, 2) X(2, 4) X(4, 2) X(4, 4) X(8, 2) X(8, 4) X(16, 2) X(16, 4)
// Waves a row in the backward; a block holds 16 waves in 16 / W row groups.
#define TP_AMD_LN_BWD_SHAPES(X) X(1) X(2) X(4) X(8) X(16)

// Blocks of `kernel` the GPU holds at once (its occupancy per CU times the
// CUs), at most `work`.
template <typename K>
int64_t resident_grid(K kernel, int threads, int device, int64_t work, size_t lds = 0) {
    int per_cu = 0;
    TP_AMD_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds));
    const int64_t grid = static_cast<int64_t>(cu_count(device)) * (per_cu > 0 ? per_cu : 1);
    return grid < work ? grid : work;
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
    // The row kernels address rows and the statistics with 32-bit byte offsets.
    const bool vec = D % N == 0 && rows < (int64_t{1} << 30) && aligned16(x) && aligned16(y) &&
                     (w == nullptr || aligned16(w)) && (b == nullptr || aligned16(b));
    const RowShape rs = vec ? row_shape(D / N, 4) : RowShape{};
#define TP_AMD_LN_FWD(W, V)                                                                      \
    if constexpr (W == 1 || V == 4) {                                                            \
        if (rs.waves == W && rs.vpt == V) {                                                      \
            constexpr int kRows = ln_threads<W>() / (W * kWave);                                 \
            const int64_t blocks = resident_grid(layer_norm_rows_kernel<T, W, V>, ln_threads<W>(), \
                                                 device, (rows + kRows - 1) / kRows);            \
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
    // The row kernels address rows and the statistics with 32-bit byte offsets.
    const bool vec = D % N == 0 && rows < (int64_t{1} << 30) && aligned16(x) && aligned16(dy) &&
                     (dx == nullptr || aligned16(dx)) && (w == nullptr || aligned16(w));
    const RowShape shape = vec ? backward_row_shape(D / N, N) : RowShape{};
    if (shape.waves > 0) {
        // As many blocks as the GPU holds at once walk the rows; each leaves
        // one partial row of dW and of dB.
        int64_t grid = 0;
        Workspace ws;
        float *dw_part = nullptr, *db_part = nullptr;
        auto launch = [&](auto kernel, int groups, int threads) {
            const size_t lds = groups > 1 ? static_cast<size_t>(D) * sizeof(float) : 0;
            grid = resident_grid(kernel, threads, device, (rows + groups - 1) / groups, lds);
            if (params) {
                ws = Workspace(static_cast<size_t>(2 * fold_floats(grid, D)) * sizeof(float), device);
                dw_part = static_cast<float*>(ws.get());
                db_part = dw_part + fold_floats(grid, D);
            }
            kernel<<<grid, threads, lds, st>>>(dy, x, mean, rstd, w, dx, dw_part, db_part, rows, D);
        };
        constexpr int V = bwd_vpt(N);
#define TP_AMD_LN_BWD(W)                                                                             \
    if (shape.waves == W) launch(layer_norm_backward_rows_kernel<T, W, V, 16 / W>, 16 / W, 16 * kWave);
        TP_AMD_LN_BWD_SHAPES(TP_AMD_LN_BWD)
#undef TP_AMD_LN_BWD
        TP_AMD_HIP_CHECK(hipGetLastError());
        if (params) {
            fold_rows_kernel<T><<<fold_grid(D), kFoldThreads, 0, st>>>(dw_part, db_part, grid, D, static_cast<S*>(dwv),
                                                              static_cast<S*>(dbv));
            TP_AMD_HIP_CHECK(hipGetLastError());
        }
        return;
    }
    if (dx != nullptr) {
        layer_norm_backward_generic_kernel<T><<<rows, kBlock, 0, st>>>(dy, x, mean, rstd, w, dx, D);
        TP_AMD_HIP_CHECK(hipGetLastError());
    }
    if (params) {
        // Enough row slices for two blocks a CU, each at least 64 rows.
        const int64_t tiles = (D + kWave - 1) / kWave;
        const int64_t want = 2 * static_cast<int64_t>(cu_count(device));
        int64_t slices = std::min<int64_t>((want + tiles - 1) / tiles, (rows + 63) / 64);
        if (slices < 1) slices = 1;
        const int64_t rslice = (rows + slices - 1) / slices;
        slices = (rows + rslice - 1) / rslice;
        Workspace ws(static_cast<size_t>(2 * fold_floats(slices, D)) * sizeof(float), device);
        float* dwf = static_cast<float*>(ws.get());
        float* dbf = dwf + fold_floats(slices, D);
        layer_norm_param_grad_generic_kernel<T><<<static_cast<unsigned>(tiles * slices), kParamWaves * kWave, 0, st>>>(
            dy, x, mean, rstd, dwf, dbf, rows, D, tiles, slices, rslice);
        fold_rows_kernel<T><<<fold_grid(D), kFoldThreads, 0, st>>>(dwf, dbf, slices, D, static_cast<S*>(dwv),
                                                          static_cast<S*>(dbv));
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

// The keep bits of Philox blocks b0 .. b0 + NB - 1, four elements each.
template <int NB>
__device__ __forceinline__ void keep_bits(int64_t b0, uint32_t threshold, uint32_t k0, uint32_t k1,
                                          uint32_t off0, uint32_t off1, uint8_t (&m)[4 * NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint64_t blk = static_cast<uint64_t>(b0 + b);
        const Philox r = philox4x32_10(static_cast<uint32_t>(blk), static_cast<uint32_t>(blk >> 32), off0,
                                       off1, k0, k1);
#pragma unroll
        for (int j = 0; j < 4; ++j) m[4 * b + j] = (r.c[j] >> 8) >= threshold ? 1 : 0;
    }
}

// N mask bytes (4 or 8) as one store; the address is a multiple of N.
template <int N>
__device__ __forceinline__ void store_mask(uint8_t* p, const uint8_t (&m)[N]) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) lo |= static_cast<uint32_t>(m[j]) << (8 * j);
    if constexpr (N == 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) hi |= static_cast<uint32_t>(m[4 + j]) << (8 * j);
        *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
    } else {
        *reinterpret_cast<uint32_t*>(p) = lo;
    }
}

template <int N>
__device__ __forceinline__ void load_mask(const uint8_t* p, float (&m)[N]) {
    uint32_t w[N / 4];
    if constexpr (N == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        w[0] = v.x;
        w[1] = v.y;
    } else {
        w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
#pragma unroll
    for (int j = 0; j < N; ++j) m[j] = ((w[j / 4] >> (8 * (j % 4))) & 0xffu) != 0 ? 1.0f : 0.0f;
}

// One 16-byte packet per thread (4 float32 or 8 16-bit elements, one or two
// Philox blocks): out = keep ? x * scale : 0, mask = keep.  `vec` says x and
// out are 16-byte aligned; elements past the last whole packet, or all of
// them without `vec`, go one at a time.
template <typename T>
__global__ __launch_bounds__(kBlock) void dropout_kernel(const S_<T>* x, S_<T>* out, uint8_t* mask,
                                                         int64_t n, uint32_t threshold, float scale,
                                                         uint32_t k0, uint32_t k1, uint32_t off0,
                                                         uint32_t off1, bool vec) {
    constexpr int N = Packet<T>::N;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t e0 = t * N;
    if (e0 >= n) return;
    uint8_t m[N];
    keep_bits<N / 4>(t * (N / 4), threshold, k0, k1, off0, off1, m);
    if (vec && e0 + N <= n) {
        float xv[N], o[N];
        unpack<T>(*reinterpret_cast<const uint4*>(x + e0), xv);
#pragma unroll
        for (int j = 0; j < N; ++j) o[j] = m[j] ? opaque(xv[j] * scale) : 0.0f;
        store_raw_nt(out + e0, pack<T>(o));
        store_mask<N>(mask + e0, m);
    } else {
        for (int j = 0; j < N && e0 + j < n; ++j) {
            out[e0 + j] = Elem<T>::store(m[j] ? opaque(Elem<T>::load(x[e0 + j]) * scale) : 0.0f);
            mask[e0 + j] = m[j];
        }
    }
}

// out = grad * mask * scale (mask bytes 0 / 1), one packet per thread.
template <typename T>
__global__ __launch_bounds__(kBlock) void dropout_backward_kernel(const S_<T>* grad, const uint8_t* mask,
                                                                  S_<T>* out, int64_t n, float scale,
                                                                  bool vec) {
    constexpr int N = Packet<T>::N;
    const int64_t e0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * N;
    if (e0 >= n) return;
    if (vec && e0 + N <= n) {
        float g[N], m[N], o[N];
        unpack<T>(load_raw_nt(grad + e0), g);
        load_mask<N>(mask + e0, m);
#pragma unroll
        for (int j = 0; j < N; ++j) o[j] = opaque(g[j] * m[j] * scale);
        store_raw_nt(out + e0, pack<T>(o));
    } else {
        for (int j = 0; j < N && e0 + j < n; ++j) {
            const float m = mask[e0 + j] != 0 ? 1.0f : 0.0f;
            out[e0 + j] = Elem<T>::store(opaque(Elem<T>::load(grad[e0 + j]) * m * scale));
        }
    }
}

// ---- embedding ---------------------------------------------------------------

template <typename I>
__device__ __forceinline__ int64_t index_at(const void* idx, int64_t i) {
    return static_cast<int64_t>(static_cast<const I*>(idx)[i]);
}

// Index i through a resource over the index array: 0 past its end, with no
// branch, so a thread's loads of a batch go out together.
template <typename I>
__device__ __forceinline__ int64_t index_load(Rsrc r, int64_t i) {
    const uint32_t off = static_cast<uint32_t>(i) * static_cast<uint32_t>(sizeof(I));
    if constexpr (sizeof(I) == 8) {
        typedef unsigned int U32x2 __attribute__((ext_vector_type(2)));
        const U32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        return static_cast<int64_t>((static_cast<uint64_t>(v[1]) << 32) | v[0]);
    } else {
        return static_cast<int64_t>(static_cast<I>(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0)));
    }
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

// The dense gradient gathers instead of scattering: the samples of each
// table row are listed -- by row ranges in one launch
// (embedding_plan_range_kernel) or, for batches too large for every block
// to read, by count, exclusive scan and fill over the whole table -- then
// one block per row writes the row once: the sum of its samples' dy rows in
// increasing sample order, or zeros.  The whole table is written exactly
// once and the result does not depend on timing.

// counts[idx[i]] += 1 for valid, non-padding indices.
template <typename I>
__global__ __launch_bounds__(kBlock) void embedding_count_kernel(const void* idx, int64_t n, int64_t V,
                                                                 int64_t padding_idx, int* counts) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const int64_t r = index_at<I>(idx, i);
    if (r >= 0 && r < V && r != padding_idx) atomicAdd(&counts[r], 1);
}

constexpr int kScanThreads = 1024;
constexpr int kScanPer = 16;  // counts per lane in a tile

// Inclusive prefix sum across the 64 lanes with DPP lane moves: shifts by
// 1, 2, 4 and 8 within each row of 16 lanes (a lane with no source adds 0),
// then lane 15 of rows 0 and 2 added to rows 1 and 3, then lane 31 to rows 2
// and 3.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); // row_bcast:31
    return v;
}

// offsets[0 .. V] = exclusive scan of counts[0 .. V), and counts zeroed (they
// become the fill cursors).  One block walks tiles of kScanThreads x
// kScanPer counts; wave w owns the tile's w-th run of kWave x kScanPer
// counts and reads it kWave at a time (lane l takes run index k kWave + l,
// so every access is one coalesced line), scanning each step across the
// wave; the waves' totals are scanned across the block and a carry moves to
// the next tile.
__global__ __launch_bounds__(kScanThreads) void embedding_scan_kernel(int* counts, int* offsets, int64_t V) {
    __shared__ int wave_tot[kScanThreads / kWave];
    __shared__ int carry_s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    if (threadIdx.x == 0) carry_s = 0;
    constexpr int64_t kRun = static_cast<int64_t>(kWave) * kScanPer;
    constexpr int64_t kTile = kRun * (kScanThreads / kWave);
    for (int64_t base = 0; base < V; base += kTile) {
        const int64_t run0 = base + wave * kRun;
        int v[kScanPer];
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) {
            const int64_t r = run0 + k * kWave + lane;
            v[k] = r < V ? counts[r] : 0;
        }
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) v[k] = wave_inclusive_scan(v[k]);
        int total = 0;
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) {
            const int step_total = __builtin_amdgcn_readlane(v[k], kWave - 1);
            v[k] += total;  // inclusive prefix within the wave's run
            total += step_total;
        }
        __syncthreads();  // carry_s and wave_tot of the previous tile are read
        if (lane == 0) wave_tot[wave] = total;
        __syncthreads();
        int before = carry_s;
        for (int w = 0; w < wave; ++w) before += wave_tot[w];
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) {
            const int64_t r = run0 + k * kWave + lane;
            if (r < V) {
                offsets[r + 1] = before + v[k];
                counts[r] = 0;
            }
        }
        __syncthreads();  // everyone has read carry_s
        if (threadIdx.x == kScanThreads - 1) carry_s = before + total;
    }
    if (threadIdx.x == 0) offsets[0] = 0;
}

// list[offsets[r] + k] = i, k the arrival order among row r's samples.
template <typename I>
__global__ __launch_bounds__(kBlock) void embedding_fill_kernel(const void* idx, int64_t n, int64_t V,
                                                                int64_t padding_idx, const int* offsets,
                                                                int* cursors, int* list) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const int64_t r = index_at<I>(idx, i);
    if (r >= 0 && r < V && r != padding_idx) {
        const int64_t pos = static_cast<int64_t>(offsets[r]) + atomicAdd(&cursors[r], 1);
        if (pos < n) list[pos] = static_cast<int>(i);  // always true; keeps the write inside `list`
    }
}

// Row `row` of the gradient = the sum of dy's rows entries[0 .. c) in that
// order (float32, from 0), times 1 / c with scale_grad_by_freq; the block's
// threads split the columns.
template <typename T, bool VEC, bool NT = true>
__device__ __forceinline__ void sum_row(const S_<T>* dy, const int* entries, int c, int64_t D,
                                        int scale_grad_by_freq, S_<T>* row) {
    constexpr int N = VEC ? Packet<T>::N : 1;
    const int64_t units = D / N;
    const float scale = scale_grad_by_freq ? 1.0f / static_cast<float>(c) : 1.0f;
    for (int64_t q = threadIdx.x; q < units; q += kBlock) {
        float acc[N];
#pragma unroll
        for (int j = 0; j < N; ++j) acc[j] = 0.0f;
        for (int k = 0; k < c; ++k) {
            const int64_t e = entries[k];
            if constexpr (VEC) {
                float v[N];
                unpack<T>(load_raw_nt(dy + e * D + q * N), v);
#pragma unroll
                for (int j = 0; j < N; ++j) acc[j] += v[j];
            } else {
                acc[0] += Elem<T>::load(dy[e * D + q]);
            }
        }
#pragma unroll
        for (int j = 0; j < N; ++j) acc[j] *= scale;
        if constexpr (VEC) {
            if constexpr (NT) store_raw_nt(row + q * N, pack<T>(acc));
            else *reinterpret_cast<uint4*>(row + q * N) = pack<T>(acc);
        } else {
            row[q] = Elem<T>::store(acc[0]);
        }
    }
}

// Row `row` of zeros (NT: non-temporal stores).
template <typename T, bool VEC, bool NT = true>
__device__ __forceinline__ void zero_row(int64_t D, S_<T>* row) {
    constexpr int N = VEC ? Packet<T>::N : 1;
    for (int64_t q = threadIdx.x; q < D / N; q += kBlock) {
        if constexpr (VEC) {
            if constexpr (NT) store_raw_nt(row + q * N, make_uint4(0u, 0u, 0u, 0u));
            else *reinterpret_cast<uint4*>(row + q * N) = make_uint4(0u, 0u, 0u, 0u);
        } else {
            row[q] = Elem<T>::store(0.0f);
        }
    }
}

constexpr int kSortCap = 2048;  // samples of one row ordered in LDS; more go through `sorted`

// Row r of the gradient (one block): the samples listed for r put in
// increasing order (each entry's rank among the row's entries, the entries
// being distinct), then each thread sums its columns over them in that
// order, scaled by 1 / count with scale_grad_by_freq.
template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void embedding_gather_kernel(const S_<T>* dy, const int* offsets,
                                                                  const int* list, int* sorted, int n_list,
                                                                  int64_t D, int scale_grad_by_freq,
                                                                  S_<T>* out) {
    __shared__ int stage[kSortCap];
    __shared__ int order[kSortCap];
    const int64_t r = blockIdx.x;
    // offsets rise from 0 to at most n; the clamps keep reads inside `list`
    const int off = max(offsets[r], 0);
    const int c = max(0, min(offsets[r + 1], n_list) - off);
    S_<T>* row = out + r * D;
    if (c == 0) {
        zero_row<T, VEC>(D, row);
        return;
    }
    const int* entries;
    if (c <= kSortCap) {
        for (int u = threadIdx.x; u < c; u += kBlock) stage[u] = list[off + u];
        __syncthreads();
        for (int u = threadIdx.x; u < c; u += kBlock) {
            const int e = stage[u];
            int rank = 0;
            for (int v = 0; v < c; ++v) rank += stage[v] < e;
            order[rank] = e;
        }
        __syncthreads();
        entries = order;
    } else {
        // Rank against the list in chunks staged through LDS; the ordered
        // entries go to this row's range of `sorted`.
        for (int u0 = 0; u0 < c; u0 += kBlock) {
            const int u = u0 + threadIdx.x;
            const int e = u < c ? list[off + u] : 0;
            int rank = 0;
            for (int v0 = 0; v0 < c; v0 += kSortCap) {
                const int len = c - v0 < kSortCap ? c - v0 : kSortCap;
                __syncthreads();
                for (int v = threadIdx.x; v < len; v += kBlock) stage[v] = list[off + v0 + v];
                __syncthreads();
                for (int v = 0; v < len; ++v) rank += stage[v] < e;
            }
            if (u < c) sorted[off + rank] = e;
        }
        __syncthreads();
        entries = sorted + off;
    }
    sum_row<T, VEC>(dy, entries, c, D, scale_grad_by_freq, row);
}

// The cursors of the range plan below: cursor g hands out the entries of
// list region g, each cursor on its own 128-byte line (atomics on one line
// serialize).  The ordered gather, which always follows the plan on the
// same stream, zeroes them for the next plan.
constexpr int kPlanCursors = 16;
constexpr int kCursorStride = 32;  // uint32 slots per 128-byte line
__device__ unsigned int embedding_plan_cursors[kPlanCursors * kCursorStride];

// The plan by row ranges, one launch, for batches whose indices every
// block can afford to read: block b owns table rows [b R, b R + R) and
// reads all n indices (from L2 once the first blocks have fetched them).
// Wave w takes the w-th sixteenth of the samples and counts its rows'
// samples in wave-private LDS counters; one scan gives each row its start
// and each (wave, row) its first slot, and one of `regions` device-wide
// cursors (block b takes cursor g = b % regions) gives the block its
// segment of list region g, entries [g n, g n + n).  A second pass places
// the samples (from registers when a wave's share is one step of
// kRangeBatch x 64 samples, else read again): a wave's samples after the
// previous waves', and inside a 64-sample step the lanes that share a row
// ranked by lane, so each row's samples are listed in increasing order and
// the gather needs no sort.  starts[r] and counts[r] locate row r's
// samples.  The ordered gather that follows resets the cursors for the next
// launch; launches on one device must not overlap (the library runs them
// on one stream).  One cursor for all 256 blocks, and an arrival count to
// reset it, cost about 2 us each (the blocks' atomics on one address
// serialize): measured 10.3 us a plan, against 7.8 and 8.2 us with either
// atomic taken out.
constexpr int kRangeRows = 128;  // most rows a block owns
constexpr int kRangeThreads = 1024;
constexpr int kRangeWaves = kRangeThreads / kWave;
constexpr int kRangeBatch = 8;  // index loads in flight per lane
constexpr int64_t kRangeReadCap = int64_t{128} << 20;  // bytes of indices all blocks read, each pass
constexpr int64_t kPlanListCap = int64_t{1} << 22;     // list entries beyond which fewer regions are used

template <typename I>
__global__ __launch_bounds__(kRangeThreads) void embedding_plan_range_kernel(const void* idx, int n, int64_t V,
                                                                      int64_t padding_idx, int rows_per_block,
                                                                      int regions, int* starts, int* counts,
                                                                      int* list) {
    __shared__ int cursor[kRangeWaves][kRangeRows];
    __shared__ int first[kRangeRows + 1];
    __shared__ int base_s;
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
    const int R = static_cast<int>(V - r0 < rows_per_block ? V - r0 : rows_per_block);
    for (int k = tid; k < kRangeWaves * kRangeRows; k += kRangeThreads) (&cursor[0][0])[k] = 0;
    __syncthreads();
    const int64_t share = (static_cast<int64_t>(n) + kRangeWaves - 1) / kRangeWaves;
    const int64_t s0 = min<int64_t>(n, wave * share), s1 = min<int64_t>(n, s0 + share);
    // the rows of a step of kRangeBatch x 64 samples relative to r0, -1 for
    // samples that are not this block's
    // The host takes this kernel only while n indices fit a 32-bit offset.
    const Rsrc ridx = buffer_over(idx, static_cast<uint32_t>(n) * static_cast<uint32_t>(sizeof(I)));
    auto step_rows = [&](int64_t base, int (&lr)[kRangeBatch]) {
        int64_t r[kRangeBatch];
#pragma unroll
        for (int u = 0; u < kRangeBatch; ++u) r[u] = index_load<I>(ridx, base + u * kWave + lane);
#pragma unroll
        for (int u = 0; u < kRangeBatch; ++u) {
            if (base + u * kWave + lane >= s1) r[u] = -1;
        }
#pragma unroll
        for (int u = 0; u < kRangeBatch; ++u)
            lr[u] = r[u] >= r0 && r[u] < r0 + R && r[u] != padding_idx ? static_cast<int>(r[u] - r0) : -1;
    };
    int first_step[kRangeBatch];  // kept for the placement pass
    for (int64_t base = s0; base < s1; base += kRangeBatch * kWave) {
        int lr[kRangeBatch];
        step_rows(base, lr);
#pragma unroll
        for (int u = 0; u < kRangeBatch; ++u) {
            if (lr[u] >= 0) atomicAdd(&cursor[wave][lr[u]], 1);
            if (base == s0) first_step[u] = lr[u];
        }
    }
    __syncthreads();
    if (wave == 0) {
        // first[l] = samples of rows before l; cursor[w][l] = where wave w's
        // samples of row l start
        int carry = 0;
        for (int c0 = 0; c0 < R; c0 += kWave) {
            const int l = c0 + lane;
            int c[kRangeWaves], tot = 0;
#pragma unroll
            for (int w = 0; w < kRangeWaves; ++w) {
                c[w] = l < R ? cursor[w][l] : 0;
                tot += c[w];
            }
            const int incl = wave_inclusive_scan(tot);
            int run = carry + incl - tot;
            if (l < R) {
                first[l] = run;
#pragma unroll
                for (int w = 0; w < kRangeWaves; ++w) {
                    cursor[w][l] = run;
                    run += c[w];
                }
            }
            carry += __builtin_amdgcn_readlane(incl, kWave - 1);
        }
        if (lane == 0) {
            first[R] = carry;
            const int g = static_cast<int>(blockIdx.x % static_cast<unsigned>(regions));
            base_s = static_cast<int>(__hip_atomic_fetch_add(&embedding_plan_cursors[g * kCursorStride],
                                                             static_cast<unsigned int>(carry), __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT));
        }
    }
    __syncthreads();
    // This block's segment: entries [base_b, base_b + its samples) of its
    // region, which starts at `region`; a region's segments hold at most n.
    const int base_b = base_s;
    const int region = static_cast<int>(blockIdx.x % static_cast<unsigned>(regions)) * n;
    for (int l = tid; l < R; l += kRangeThreads) {
        starts[r0 + l] = region + base_b + first[l];
        counts[r0 + l] = first[l + 1] - first[l];
    }
    for (int64_t base = s0; base < s1; base += kRangeBatch * kWave) {
        int lr[kRangeBatch];
        if (base == s0) {
#pragma unroll
            for (int u = 0; u < kRangeBatch; ++u) lr[u] = first_step[u];
        } else {
            step_rows(base, lr);
        }
#pragma unroll
        for (int u = 0; u < kRangeBatch; ++u) {
            uint64_t mask = __builtin_amdgcn_ballot_w64(lr[u] >= 0);
            int rank = 0, same = 0;
            while (mask) {
                const int j = __builtin_ctzll(mask);
                mask &= mask - 1;
                const int lj = __builtin_amdgcn_readlane(lr[u], j);
                same += lj == lr[u];
                rank += lj == lr[u] && j < lane;
            }
            if (lr[u] >= 0) {
                const int pos = cursor[wave][lr[u]] + rank;
                // a region's segments partition some of the valid samples: always < n
                if (base_b + pos < n) list[region + base_b + pos] = static_cast<int>(base + u * kWave + lane);
                if (rank == same - 1) cursor[wave][lr[u]] = pos + 1;
            }
        }
    }
}

// Row r of the gradient (one block) from a plan whose rows list their
// samples in increasing order: list[starts[r] .. starts[r] + counts[r]).
// NT selects non-temporal stores: the host takes them for a table larger
// than the 256 MB Infinity Cache, and the default policy for one that fits
// (measured on [32000, 4096] with 8192 random indices: bf16, 262 MB, 58.6 us
// against 69.8 us non-temporal; float32, 524 MB, 131.8 us against 138.1 us
// with the default policy).
constexpr int64_t kGatherCachedBytes = int64_t{256} << 20;

template <typename T, bool VEC, bool NT>
__global__ __launch_bounds__(kBlock) void embedding_gather_ordered_kernel(const S_<T>* dy, const int* starts,
                                                                          const int* counts, const int* list,
                                                                          int n_list, int64_t D,
                                                                          int scale_grad_by_freq, S_<T>* out) {
    const int64_t r = blockIdx.x;
    // starts and counts stay inside [0, n_list]; the clamps keep reads inside `list`
    const int off = min(max(starts[r], 0), n_list);
    const int c = max(0, min(counts[r], n_list - off));
    S_<T>* row = out + r * D;
    if (c == 0) {
        zero_row<T, VEC, NT>(D, row);
    } else {
        sum_row<T, VEC, NT>(dy, list + off, c, D, scale_grad_by_freq, row);
    }
    // Last, after every load: a store ahead of them would make the compiler
    // read starts and counts through vector memory instead of scalar loads
    // (measured 13 us slower for bf16 rows).
    if (r == 0 && threadIdx.x < kPlanCursors) {
        __hip_atomic_store(&embedding_plan_cursors[threadIdx.x * kCursorStride], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
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
// y[i]; otherwise each block writes its (sum loss, sum weight) to part, and
// the last block to arrive adds the partials in block order (thread t
// taking blocks t, t + kBlock, ..., then the block's lanes and waves in
// order) into y = sum loss (/ sum weight for the mean) and total = sum
// weight -- one launch.  The arrival order rests on the same gfx950
// guarantee as the reductions' one-launch folds: agent-scope stores are
// written through and acknowledged before s_waitcnt vmcnt(0) returns, so
// they precede the counter's atomic add, and agent-scope loads read the
// coherent level.  The counter is reset by its last arrival.
__device__ unsigned int nll_arrivals;
template <typename T, typename I>
__global__ __launch_bounds__(kBlock) void nll_kernel(const S_<T>* x, const void* target, const S_<T>* w,
                                                     int64_t n, int64_t C, int64_t ignore_index,
                                                     int reduction, S_<T>* y, S_<T>* total,
                                                     float* part) {
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
    __shared__ bool last;
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = 0.0f, b = 0.0f;
        for (int k = 0; k < kBlock / kWave; ++k) {
            a += s_loss[k];
            b += s_wt[k];
        }
        __hip_atomic_store(&part[2 * blockIdx.x], a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&part[2 * blockIdx.x + 1], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        last = __hip_atomic_fetch_add(&nll_arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               gridDim.x - 1;
        if (last) __hip_atomic_store(&nll_arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    float a = 0.0f, b = 0.0f;
    for (int64_t k = threadIdx.x; k < gridDim.x; k += kBlock) {
        a += __hip_atomic_load(&part[2 * k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        b += __hip_atomic_load(&part[2 * k + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    a = wave_allreduce(a, Plus{});
    b = wave_allreduce(b, Plus{});
    __syncthreads();  // every wave has read s_loss / s_wt above
    if (lane == 0) {
        s_loss[wave] = a;
        s_wt[wave] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ta = 0.0f, tb = 0.0f;
        for (int k = 0; k < kBlock / kWave; ++k) {
            ta += s_loss[k];
            tb += s_wt[k];
        }
        y[0] = Elem<T>::store(reduction == 1 ? ta / tb : ta);
        total[0] = Elem<T>::store(tb);
    }
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

// The same with dx as rows of 16-byte packets (C a multiple of the packet,
// dx aligned): a row takes `blocks_per_row` blocks, each thread one packet,
// holding the target's value if the target falls inside it.
template <typename T, typename I>
__global__ __launch_bounds__(kBlock) void nll_backward_rows_kernel(const S_<T>* grad, const void* target,
                                                                   const S_<T>* w, const S_<T>* total,
                                                                   int64_t C, uint32_t blocks_per_row,
                                                                   int64_t ignore_index, int reduction,
                                                                   S_<T>* dx) {
    constexpr int N = Packet<T>::N;
    const uint32_t i = blockIdx.x / blocks_per_row;
    const int64_t q = static_cast<int64_t>(blockIdx.x - i * blocks_per_row) * kBlock + threadIdx.x;
    if (q >= C / N) return;
    const int64_t t = index_at<I>(target, i);
    const bool bad = t != ignore_index && (t < 0 || t >= C);
    float v[N];
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = bad ? __builtin_nanf("") : 0.0f;
    const int64_t k = t - q * N;
    if (!bad && t != ignore_index && k >= 0 && k < N) {
        const float g = reduction == 0 ? Elem<T>::load(grad[i])
                        : reduction == 1 ? Elem<T>::load(grad[0]) / Elem<T>::load(total[0])
                                         : Elem<T>::load(grad[0]);
        const float val = opaque(-(w != nullptr ? Elem<T>::load(w[t]) : 1.0f) * g);
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = j == k ? val : v[j];
    }
    store_raw_nt(dx + static_cast<int64_t>(i) * C + q * N, pack<T>(v));
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
        const OnDevice scope(device);
        const int index = scope.index();
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
        const OnDevice scope(device);
        const int index = scope.index();
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
        const OnDevice scope(device);
        const int index = scope.index();
        const float scale = static_cast<float>(1.0 / (1.0 - p));
        // p 2^24 is exact in double; a 24-bit uniform u 2^-24 is >= p exactly
        // when u >= ceil(p 2^24) (at most 2^24, which keeps nothing).
        const uint32_t threshold = static_cast<uint32_t>(std::ceil(std::ldexp(p, 24)));
        TP_AMD_DISPATCH_NN(dtype, T, {
            constexpr int N = Packet<T>::N;
            const bool vec = aligned16(x) && aligned16(out) && reinterpret_cast<uintptr_t>(mask) % N == 0;
            dropout_kernel<T><<<blocks_for((n + N - 1) / N, kBlock), kBlock, 0, stream(index)>>>(
                static_cast<const S_<T>*>(x), static_cast<S_<T>*>(out), mask, n, threshold, scale,
                static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32),
                static_cast<uint32_t>(offset), static_cast<uint32_t>(offset >> 32), vec);
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_dropout_backward(int device, int dtype, int64_t n, const void* grad,
                                   const uint8_t* mask, double scale, void* out) {
    return guarded([&] {
        TP_AMD_CHECK(n >= 0, "dropout_backward: negative extent");
        if (n == 0) return;
        const OnDevice scope(device);
        const int index = scope.index();
        TP_AMD_DISPATCH_NN(dtype, T, {
            constexpr int N = Packet<T>::N;
            const bool vec = aligned16(grad) && aligned16(out) && reinterpret_cast<uintptr_t>(mask) % N == 0;
            dropout_backward_kernel<T><<<blocks_for((n + N - 1) / N, kBlock), kBlock, 0, stream(index)>>>(
                static_cast<const S_<T>*>(grad), mask, static_cast<S_<T>*>(out), n,
                static_cast<float>(scale), vec);
        });
        TP_AMD_HIP_CHECK(hipGetLastError());
    });
}

int tp_amd_launch_embedding(int device, int dtype, int64_t num_weights, int64_t dim, const void* weight,
                            int index_dtype, int64_t n, const void* indices, void* out) {
    return guarded([&] {
        TP_AMD_CHECK(num_weights >= 0 && dim >= 0 && n >= 0, "embedding: negative extent");
        if (n == 0 || dim == 0) return;
        const OnDevice scope(device);
        const int index = scope.index();
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
        TP_AMD_CHECK(n < 0x7fffffff && num_weights < 0x7fffffff,
                     "embedding_backward: at most 2^31 - 2 samples and table rows");
        const OnDevice scope(device);
        const int index = scope.index();
        hipStream_t st = stream(index);
        // The plan by row ranges (about one block per CU, at most kRangeRows
        // rows each) when its blocks' index reads stay under kRangeReadCap;
        // otherwise count, scan and fill over the whole table.
        const int64_t per_block = std::min<int64_t>(
            kRangeRows, std::max<int64_t>(1, blocks_for(num_weights, int64_t{cu_count(index)})));
        const int64_t range_blocks = blocks_for(num_weights, per_block);
        const int64_t index_bytes = index_dtype == TP_AMD_INT32 ? 4 : 8;
        if (range_blocks * n * index_bytes <= kRangeReadCap) {
            // starts [V], counts [V], list [regions x n]: up to kPlanCursors
            // regions while the list stays under kPlanListCap entries
            const int64_t regions = std::max<int64_t>(
                1, std::min<int64_t>({int64_t{kPlanCursors}, range_blocks, kPlanListCap / std::max<int64_t>(n, 1)}));
            Workspace ws(static_cast<size_t>(2 * num_weights + regions * n) * sizeof(int), index);
            int* starts = static_cast<int*>(ws.get());
            int* counts = starts + num_weights;
            int* list = counts + num_weights;
            dispatch_index<float>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                embedding_plan_range_kernel<I><<<range_blocks, kRangeThreads, 0, st>>>(
                    indices, static_cast<int>(n), num_weights, padding_idx, static_cast<int>(per_block),
                    static_cast<int>(regions), starts, counts, list);
            });
            TP_AMD_DISPATCH_NN(dtype, T, {
                const bool vec = dim % Packet<T>::N == 0 && aligned16(grad) && aligned16(out);
                const bool nt = num_weights * dim * static_cast<int64_t>(sizeof(S_<T>)) > kGatherCachedBytes;
                auto gather = [&](auto vec_tag, auto nt_tag) {
                    embedding_gather_ordered_kernel<T, decltype(vec_tag)::value, decltype(nt_tag)::value>
                        <<<num_weights, kBlock, 0, st>>>(static_cast<const S_<T>*>(grad), starts, counts, list,
                                                        static_cast<int>(regions * n), dim, scale_grad_by_freq,
                                                        static_cast<S_<T>*>(out));
                };
                using Yes = std::true_type;
                using No = std::false_type;
                if (vec) {
                    nt ? gather(Yes{}, Yes{}) : gather(Yes{}, No{});
                } else {
                    nt ? gather(No{}, Yes{}) : gather(No{}, No{});
                }
            });
            TP_AMD_HIP_CHECK(hipGetLastError());
            return;
        }
        // counts / cursors [V], offsets [V + 1], list and sorted [n]
        const size_t words = static_cast<size_t>(2 * num_weights + 1 + 2 * n);
        Workspace ws(words * sizeof(int), index);
        int* counts = static_cast<int*>(ws.get());
        int* offsets = counts + num_weights;
        int* list = offsets + num_weights + 1;
        int* sorted = list + n;
        zero_words_kernel<<<blocks_for(num_weights, kBlock), kBlock, 0, st>>>(
            reinterpret_cast<uint32_t*>(counts), num_weights);
        if (n > 0) {
            dispatch_index<float>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                embedding_count_kernel<I><<<blocks_for(n, kBlock), kBlock, 0, st>>>(indices, n, num_weights,
                                                                                   padding_idx, counts);
            });
        }
        embedding_scan_kernel<<<1, kScanThreads, 0, st>>>(counts, offsets, num_weights);
        if (n > 0) {
            dispatch_index<float>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                embedding_fill_kernel<I><<<blocks_for(n, kBlock), kBlock, 0, st>>>(
                    indices, n, num_weights, padding_idx, offsets, counts, list);
            });
        }
        TP_AMD_DISPATCH_NN(dtype, T, {
            const bool vec = dim % Packet<T>::N == 0 && aligned16(grad) && aligned16(out);
            if (vec) {
                embedding_gather_kernel<T, true><<<num_weights, kBlock, 0, st>>>(
                    static_cast<const S_<T>*>(grad), offsets, list, sorted, static_cast<int>(n), dim,
                    scale_grad_by_freq, static_cast<S_<T>*>(out));
            } else {
                embedding_gather_kernel<T, false><<<num_weights, kBlock, 0, st>>>(
                    static_cast<const S_<T>*>(grad), offsets, list, sorted, static_cast<int>(n), dim,
                    scale_grad_by_freq, static_cast<S_<T>*>(out));
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
        const OnDevice scope(device);
        const int index = scope.index();
        hipStream_t st = stream(index);
        const int64_t blocks = blocks_for(n, kBlock);
        TP_AMD_DISPATCH_NN(dtype, T, {
            Workspace part(reduction == 0 ? 0 : static_cast<size_t>(2 * blocks) * sizeof(float), index);
            dispatch_index<T>(index_dtype, [&](auto tag) {
                using I = decltype(tag);
                nll_kernel<T, I><<<blocks, kBlock, 0, st>>>(
                    static_cast<const S_<T>*>(x), target, static_cast<const S_<T>*>(weight), n, classes,
                    ignore_index, reduction, static_cast<S_<T>*>(y), static_cast<S_<T>*>(total_weight),
                    static_cast<float*>(part.get()));
            });
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
        const OnDevice scope(device);
        const int index = scope.index();
        const int64_t blocks = blocks_for(n * classes, kBlock);
        TP_AMD_DISPATCH_NN(dtype, T, {
            constexpr int N = Packet<T>::N;
            const int64_t per_row = blocks_for(classes / N, kBlock);
            if (classes % N == 0 && aligned16(dx) && n * per_row <= 0x7fffffff) {
                dispatch_index<T>(index_dtype, [&](auto tag) {
                    using I = decltype(tag);
                    nll_backward_rows_kernel<T, I><<<n * per_row, kBlock, 0, stream(index)>>>(
                        static_cast<const S_<T>*>(grad), target, static_cast<const S_<T>*>(weight),
                        static_cast<const S_<T>*>(total_weight), classes, static_cast<uint32_t>(per_row),
                        ignore_index, reduction, static_cast<S_<T>*>(dx));
                });
                break;
            }
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
