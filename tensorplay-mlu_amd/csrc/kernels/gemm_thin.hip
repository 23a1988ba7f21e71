// Thin products on the matrix cores (gfx950): C = alpha A B + beta Cin
// where one side of C is at most 64 long -- a decode step's x W^T, a
// matrix-vector product, the dX = dY W of an LM head, attention over one
// query.  Such a product reads its large operand once and does almost no
// arithmetic per byte, so it is bound by HBM; the tiled kernels
// (gemm_mfma.hip) give it a handful of 64- or 128-wide tiles that each walk
// all of K on one CU and reach a fifth of the bandwidth.
//
// Normal form.  The host turns every eligible product into
//   C'[i][j] = sum_k X[i][k] W[k][j],  i < m <= 64 ("thin" rows),
// X the small operand (any strides), W the wide one, stored K-major
// (element (k, j) at w + j ld + k: a Linear weight, or A of a product with
// few columns) or N-major (at w + k ld + j: a [K, N] row-major matrix).
// A product with few columns is taken as its transpose, C^T = B^T A^T, and
// stores C' transposed (the output strides are free).  A 16-bit product of
// more than 16 thin rows that gemm_mfma.hip's split over K spreads over
// every CU is left to that split (see launch_typed).
//
// Work split.  A column tile of W (64 or 128 columns) over a step of K (64
// of K for 16-bit types with W K-major) is one unit.  With at least as
// many tiles as blocks fit on the GPU at once, every block takes whole
// tiles; the tiles left over (fewer than a round) are first split into
// equal runs of units over the blocks (stream-K), so that their folds
// overlap the whole tiles still streaming.  With fewer tiles than that,
// every tile is split, into pieces of at least 64 KiB of W.  Within a
// block's piece of a tile the four waves take consecutive runs of steps,
// each with 16 x 16 MFMAs (the thin rows padded with zeros to 16, 32 or 64),
// the next batch of loads in flight; the waves' sums are added in LDS in a
// fixed tree.  A tile that one block covers whole is written at once.  A
// tile split between blocks gets a float32 partial from each, stored
// write-through; the last block to arrive (an arrival counter per tile)
// adds the partials in block order and writes the tile, so the bits do not
// depend on timing.
//
// Fragments (lane l, c = l % 16, g = l / 16; MFMA output lane l holds rows
// 4g..4g+3 of column c):
//   * 16-bit, W K-major: v_mfma_f32_16x16x32; lane l loads two 16-byte
//     packets of W column 16 cb + c, k = k0 + 16g .. +15, back to back,
//     and the same k of X row c, one MFMA a packet: the fragments need no
//     rearranging.
//   * 16-bit, W N-major: a lane loads 8 consecutive columns 8c .. 8c+7 at the
//     8 rows k0 + 8g + i and transposes the 8 x 8 block in registers; MFMA j
//     then multiplies tile columns 8c + j (c = 0..15).
//   * float32, W K-major: v_mfma_f32_16x16x4_f32; a 16-byte packet gives a
//     lane 4 consecutive k of one column, fed to 4 MFMAs (MFMA e takes the
//     packet's k e from X and W alike); two packets a step as for 16-bit,
//     one with more than 16 thin rows.
//   * float32, W N-major: a lane loads 4 consecutive columns 4c .. 4c+3 of
//     row k0 + g; MFMA j multiplies tile columns 4c + j.
// The sum pairs X and W elements of the same k in every case, whatever
// order the matrix core adds them in.

#include <algorithm>

#include "device_common.h"
#include "gemm.h"
#include "../allocator.h"
#include "../common.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the thin-product fold relies on gfx950's write-through ordering"
#endif

namespace tp_amd {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kThinWaves = 4;
constexpr int kThinThreads = kThinWaves * kWave;
constexpr int64_t kThinMaxRows = 64;
// One arrival counter per tile split between blocks, indexed by the first
// block that covers the tile (unique among split tiles), each on a 128-byte
// line of its own: atomics on one line serialize.
constexpr int kCounterStride = 32;
constexpr int kMaxThinBlocks = 4096;
constexpr int64_t kMinPieceBytes = int64_t(64) << 10;
constexpr int64_t kMinSplitBytes = int64_t(16) << 10;
constexpr int64_t kSplitTileBytes = int64_t(256) << 10;
// Least bytes of the wide operand for which a product takes this kernel:
// up to 16 thin rows, and more.
constexpr int64_t kMinWideBytes1 = int64_t(1) << 20;
constexpr int64_t kMinWideBytes2 = int64_t(8) << 20;
__device__ unsigned int thin_counters[kMaxThinBlocks * kCounterStride];

struct ThinArgs {
    int64_t m, n, k;    // thin rows (<= 64), columns, depth
    int64_t tiles;      // column tiles of one batch entry
    int64_t steps;      // K steps of a tile
    float alpha, beta;
    const void* x;      // X[i][k] at x + i x_m + k x_k (+ batch x_b)
    int64_t x_m, x_k, x_b;
    const void* w;      // W[k][j] at w + j ld + k (K-major) or w + k ld + j
    int64_t w_ld, w_b;
    const void* cin;    // read when beta != 0
    int64_t cin_m, cin_n, cin_b;
    void* c;            // C'[i][j] at c + i c_m + j c_n (+ batch c_b)
    int64_t c_m, c_n, c_b;
    float* part;        // [sk_blocks][2][m][TN] float32 partial tiles
    // Schedule: the first sk_tiles tiles are split into equal runs of
    // sk_units steps over blocks 0 .. sk_blocks - 1; each block then takes
    // dp_rounds whole tiles, sk_tiles + blockIdx.x + j gridDim.x.
    // (skipping tiles past all_tiles).
    int64_t sk_tiles, sk_units, sk_blocks, dp_rounds, all_tiles;
};

template <typename T, bool KMAJOR, int R, int CB>
struct Thin {
    using S = typename Elem<T>::storage;
    static constexpr bool k16 = sizeof(S) == 2;
    static constexpr int V = 16 / sizeof(S);               // elements per packet
    // MFMA column groups of 16: CB with W K-major (chosen by the host from
    // the product's width), fixed by the packet with W N-major.
    static constexpr int NB = KMAJOR ? CB : (k16 ? 8 : 4);
    static constexpr int TN = 16 * NB;                     // tile columns
    // K-major W: a step gives each lane HALVES packets of a column, lane g
    // taking packets HALVES g .. HALVES g + HALVES - 1 of the step's k, so
    // one column's packets of a step go out as back-to-back loads that
    // cover whole 128-byte lines (with one packet a lane, the two halves of
    // a line were requested a step apart and some lines were fetched twice:
    // FETCH_SIZE 1.116x the operand for bf16 1 x 4096 x 11008).  float32
    // with more than 16 rows keeps one packet, for registers.
    static constexpr int HALVES = KMAJOR && !(!k16 && R >= 2) ? 2 : 1;
    static constexpr int STEP = KMAJOR ? 4 * V * HALVES : (k16 ? 32 : 4);  // K per step
    static constexpr int WL = KMAJOR ? NB * HALVES : (k16 ? 8 : 1);       // W packets a step
    static constexpr int XL = KMAJOR ? HALVES : 1;                        // X fragments a row
    // Steps a batch of loads, and blocks a CU the registers are sized for
    // (float32 K-major with 17-32 rows: one packet a step at two blocks a
    // CU, 32 x 11008 x 4096 in 47 us against 58 us at two and one block;
    // 16-bit W N-major with up to 16 rows at two blocks a CU, the
    // accumulators moved from AGPRs into the 256 VGPRs: the LM-head dX
    // 1 x 50257 x 4096 80.5 against 84.8 us, other shapes level).
    static constexpr int U = KMAJOR ? (HALVES == 2 ? 8 : 4) / (NB * HALVES) : (k16 ? 1 : 8);
    static constexpr int OCCUPANCY = ((!k16 && KMAJOR && R == 2) || (k16 && !KMAJOR && R == 1)) ? 2 : 1;
    // X fragment: 8 (16-bit) or 4 (float32 K-major) consecutive k as one
    // packet, or one float.
    static constexpr bool kXPacket = k16 || KMAJOR;
};

template <typename T, bool KMAJOR, int R, int CB>
struct StepData {
    using P = Thin<T, KMAJOR, R, CB>;
    uint4 w[P::WL];
    typename std::conditional<P::kXPacket, uint4, float>::type x[R * P::XL];
};

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <typename T>
__device__ __forceinline__ f32x4 mma16(const uint4& a, const uint4& b, f32x4 c) {
    if constexpr (std::is_same<T, bf16_t>::value) {
        bf16x8 av, bv;
        __builtin_memcpy(&av, &a, 16);
        __builtin_memcpy(&bv, &b, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
    } else {
        f16x8 av, bv;
        __builtin_memcpy(&av, &a, 16);
        __builtin_memcpy(&bv, &b, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c, 0, 0, 0);
    }
}

__device__ __forceinline__ f32x4 mma32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Loads go through buffer resources: an offset at or past the resource's
// size reads zeros, so lanes outside the product (rows past m, columns past
// n, k past K or past the wave's run) load zeros without a branch, and the
// loop stays straight-line code whose wait counts the compiler keeps exact.
// Every valid offset is below 2^31 (checked on the host); kOob plus any
// offset added to it stays below 2^32.
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A wave's view of one piece of a tile: its resources and per-lane offsets.
template <typename T, bool KMAJOR, int R, int CB, bool XVEC>
struct ThinWave {
    using P = Thin<T, KMAJOR, R, CB>;
    using S = typename Elem<T>::storage;
    static constexpr int ES = sizeof(S);
    __amdgpu_buffer_rsrc_t wres, xres;
    uint32_t wlane[KMAJOR ? P::NB : 1];  // byte offset of the lane's W column(s), kOob outside the tile
    uint32_t xlane[R];                   // byte offset of the lane's X rows, kOob past m
    uint32_t wrow, xk;                   // N-major W bytes per row; X bytes per k
    int64_t k0, kend;                    // first k of the run; k past the run (and past K)
    int c, g;

    __device__ __forceinline__ void init(const ThinArgs& p, int64_t bi, int64_t col0, int64_t s_begin,
                                         int64_t s_end, int lane) {
        c = lane & 15;
        g = lane >> 4;
        k0 = s_begin * P::STEP;
        kend = s_end * P::STEP < p.k ? s_end * P::STEP : p.k;
        const int64_t ncols = p.n - col0 < P::TN ? p.n - col0 : P::TN;
        const S* W = static_cast<const S*>(p.w) + bi * p.w_b;
        if constexpr (KMAJOR) {
            wres = make_rsrc(W + col0 * p.w_ld, ((ncols - 1) * p.w_ld + p.k) * ES);
#pragma unroll
            for (int cb = 0; cb < P::NB; ++cb) {
                const int col = 16 * cb + c;
                wlane[cb] = col < ncols ? static_cast<uint32_t>(col * p.w_ld * ES) : kOob;
            }
        } else {
            // The resource covers rows k0 .. kend - 1: rows past the run read
            // zeros.
            const int64_t rows = kend - k0;
            wres = make_rsrc(W + k0 * p.w_ld + col0, rows > 0 ? ((rows - 1) * p.w_ld + ncols) * ES : 0);
            const int col = (P::k16 ? 8 : 4) * c;
            wlane[0] = col < ncols ? static_cast<uint32_t>(col * ES) : kOob;
            wrow = static_cast<uint32_t>(p.w_ld * ES);
        }
        const S* X = static_cast<const S*>(p.x) + bi * p.x_b;
        xres = make_rsrc(X, ((p.m - 1) * p.x_m + (p.k - 1) * p.x_k + 1) * ES);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = 16 * r + c;
            xlane[r] = row < p.m ? static_cast<uint32_t>(row * p.x_m * ES) : kOob;
        }
        xk = static_cast<uint32_t>(p.x_k * ES);
    }

    // The loads of step s.
    __device__ __forceinline__ void load(StepData<T, KMAJOR, R, CB>& d, int64_t s) const {
        constexpr int V = P::V, H = P::XL;
        if constexpr (P::kXPacket) {
            // This lane's packets: k = kv[h] .. kv[h] + V - 1.
            int64_t kv[H];
            bool ok[H];
#pragma unroll
            for (int h = 0; h < H; ++h) {
                kv[h] = s * P::STEP + V * (H * g + h);
                ok[h] = kv[h] < kend;  // K is a whole number of packets where it matters
            }
            if constexpr (KMAJOR) {
#pragma unroll
                for (int cb = 0; cb < P::NB; ++cb)
#pragma unroll
                    for (int h = 0; h < H; ++h)
                        d.w[cb * H + h] =
                            load16(wres, ok[h] ? wlane[cb] + static_cast<uint32_t>(kv[h] * ES) : kOob);
            } else {
                const uint32_t base = wlane[0] + static_cast<uint32_t>(kv[0] - k0) * wrow;
#pragma unroll
                for (int i = 0; i < 8; ++i) d.w[i] = load16(wres, base + i * wrow);
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    if constexpr (XVEC) {
                        d.x[r * H + h] = load16(xres, ok[h] ? xlane[r] + static_cast<uint32_t>(kv[h] * ES) : kOob);
                    } else {
                        S e[V];
#pragma unroll
                        for (int i = 0; i < V; ++i) {
                            const int64_t k = kv[h] + i;
                            const uint32_t off = k < kend ? xlane[r] + static_cast<uint32_t>(k) * xk : kOob;
                            if constexpr (ES == 2) {
                                e[i] = __builtin_amdgcn_raw_buffer_load_b16(xres, static_cast<int>(off), 0, 0);
                            } else {
                                e[i] = __uint_as_float(
                                    __builtin_amdgcn_raw_buffer_load_b32(xres, static_cast<int>(off), 0, 0));
                            }
                        }
                        __builtin_memcpy(&d.x[r * H + h], e, 16);
                    }
                }
        } else {
            // float32, W N-major: row k0 + g of the step, 4 columns a lane.
            const int64_t kv = s * P::STEP + g;
            d.w[0] = load16(wres, wlane[0] + static_cast<uint32_t>(kv - k0) * wrow);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t off = kv < kend ? xlane[r] + static_cast<uint32_t>(kv) * xk : kOob;
                d.x[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xres, static_cast<int>(off), 0, 0));
            }
        }
    }
};

template <typename T, bool KMAJOR, int R, int CB>
__device__ __forceinline__ void mma_step(const StepData<T, KMAJOR, R, CB>& d,
                                         f32x4 (&acc)[R][Thin<T, KMAJOR, R, CB>::NB]) {
    using P = Thin<T, KMAJOR, R, CB>;
    constexpr int H = P::XL;
    if constexpr (P::k16) {
        if constexpr (KMAJOR) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int cb = 0; cb < P::NB; ++cb)
#pragma unroll
                    for (int h = 0; h < H; ++h) acc[r][cb] = mma16<T>(d.x[r * H + h], d.w[cb * H + h], acc[r][cb]);
        } else {
            // 8 rows (k) x 8 columns -> column j's 8 consecutive k.
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t f[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t lo = word(d.w[2 * q], j / 2), hi = word(d.w[2 * q + 1], j / 2);
                    f[q] = (j & 1) ? (lo >> 16) | (hi & 0xffff0000u) : (lo & 0xffffu) | (hi << 16);
                }
                const uint4 b = make_uint4(f[0], f[1], f[2], f[3]);
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][j] = mma16<T>(d.x[r], b, acc[r][j]);
            }
        }
    } else if constexpr (KMAJOR) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int cb = 0; cb < P::NB; ++cb)
#pragma unroll
                for (int h = 0; h < H; ++h)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[r][cb] = mma32(__uint_as_float(word(d.x[r * H + h], e)),
                                           __uint_as_float(word(d.w[cb * H + h], e)), acc[r][cb]);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[r][j] = mma32(d.x[r], __uint_as_float(word(d.w[0], j)), acc[r][j]);
    }
}

// Steps [s, end) of one tile into acc: batches of U steps, the next batch's
// loads issued before the current one's MFMAs (steps past `end` load zeros).
template <typename T, bool KMAJOR, int R, int CB, bool XVEC>
__device__ __forceinline__ void run_steps(const ThinWave<T, KMAJOR, R, CB, XVEC>& wv, int64_t s, int64_t end,
                                          f32x4 (&acc)[R][Thin<T, KMAJOR, R, CB>::NB]) {
    constexpr int U = Thin<T, KMAJOR, R, CB>::U;
    if (s >= end) return;
    StepData<T, KMAJOR, R, CB> a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) wv.load(a[u], s + u);
    for (;;) {
#pragma unroll
        for (int u = 0; u < U; ++u) wv.load(b[u], s + U + u);
#pragma unroll
        for (int u = 0; u < U; ++u) mma_step<T, KMAJOR, R, CB>(a[u], acc);
        s += U;
        if (s >= end) break;
#pragma unroll
        for (int u = 0; u < U; ++u) wv.load(a[u], s + U + u);
#pragma unroll
        for (int u = 0; u < U; ++u) mma_step<T, KMAJOR, R, CB>(b[u], acc);
        s += U;
        if (s >= end) break;
    }
}

// Block holding unit u of `units` split over `blocks` blocks: the largest b
// with b units / blocks <= u.
__device__ __forceinline__ int64_t block_of(int64_t u, int64_t units, int64_t blocks) {
    return ((u + 1) * blocks - 1) / units;
}

template <typename T>
__device__ __forceinline__ void store_c(const ThinArgs& p, int64_t bi, int64_t i, int64_t j, float v) {
    using S = typename Elem<T>::storage;
    const float a = p.alpha * v;
    float out = a;
    if (p.beta != 0.0f) {
        const S* cin = static_cast<const S*>(p.cin);
        out = fmaf(p.beta, Elem<T>::load(cin[bi * p.cin_b + i * p.cin_m + j * p.cin_n]), a);
    }
    static_cast<S*>(p.c)[bi * p.c_b + i * p.c_m + j * p.c_n] = Elem<T>::store(out);
}

template <typename T, bool KMAJOR, int R, int CB, bool XVEC>
__global__ __launch_bounds__(kThinThreads, (Thin<T, KMAJOR, R, CB>::OCCUPANCY)) void gemm_thin_kernel(
    ThinArgs p) {
    using P = Thin<T, KMAJOR, R, CB>;
    constexpr int NB = P::NB, TN = P::TN;
    // Row groups reduced together (the LDS tree's slots hold RC of them), and
    // fold elements a thread, taken FC at a time.
    constexpr int RC = R < 16 / NB ? R : 16 / NB;
    constexpr int EPT = (16 * R * TN + kThinThreads - 1) / kThinThreads;
    constexpr int FC = EPT < 8 ? EPT : 8;
    static_assert(R % RC == 0 && EPT % FC == 0, "row groups and fold chunks divide evenly");
    __shared__ float red[kThinWaves / 2][RC * NB * 4][kWave];
    __shared__ float tile[16 * R][TN + 1];
    __shared__ bool last;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int c = lane & 15, g = lane >> 4;
    const int64_t blocks = p.sk_blocks;
    const int64_t u_begin = blockIdx.x < blocks ? static_cast<int64_t>(blockIdx.x) * p.sk_units / blocks : 0;
    const int64_t u_end = blockIdx.x < blocks ? (static_cast<int64_t>(blockIdx.x) + 1) * p.sk_units / blocks : 0;
    // Steps [s0, s1) of tile t (batch-major).  first_piece: the block's
    // first piece of its split run (its partial slot).
    auto piece = [&](int64_t t, int64_t s0, int64_t s1, bool first_piece) {
        const int64_t bi = t / p.tiles, col0 = (t - bi * p.tiles) * TN;
        // This wave's run of the block's steps.
        const int64_t len = s1 - s0, q = (len + kThinWaves - 1) / kThinWaves;
        const int64_t ws0 = s0 + std::min(len, wave * q), ws1 = s0 + std::min(len, (wave + 1) * q);
        f32x4 acc[R][NB];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[r][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (ws0 < ws1) {
            ThinWave<T, KMAJOR, R, CB, XVEC> wv;
            wv.init(p, bi, col0, ws0, ws1, lane);
            run_steps<T, KMAJOR, R, CB, XVEC>(wv, ws0, ws1, acc);
        }
        // Waves' sums in a fixed tree, (w0 + w2) + (w1 + w3), RC row groups
        // at a time.
#pragma unroll
        for (int r0 = 0; r0 < R; r0 += RC) {
#pragma unroll
            for (int half = kThinWaves / 2; half >= 1; half /= 2) {
                if (wave >= half && wave < 2 * half) {
#pragma unroll
                    for (int r = 0; r < RC; ++r)
#pragma unroll
                        for (int j = 0; j < NB; ++j)
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                red[wave - half][(r * NB + j) * 4 + i][lane] = acc[r0 + r][j][i];
                }
                __syncthreads();
                if (wave < half) {
#pragma unroll
                    for (int r = 0; r < RC; ++r)
#pragma unroll
                        for (int j = 0; j < NB; ++j)
#pragma unroll
                            for (int i = 0; i < 4; ++i) acc[r0 + r][j][i] += red[wave][(r * NB + j) * 4 + i][lane];
                }
                __syncthreads();
            }
        }
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int j = 0; j < NB; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = 16 * r + 4 * g + i;
                        const int col = KMAJOR ? 16 * j + c : NB * c + j;
                        tile[row][col] = acc[r][j][i];
                    }
        }
        __syncthreads();
        const int64_t elems = p.m * TN;
        if (s0 == 0 && s1 == p.steps) {
            for (int64_t e = tid; e < elems; e += kThinThreads) {
                const int64_t i = e / TN, jl = e - i * TN;
                if (col0 + jl < p.n) store_c<T>(p, bi, i, col0 + jl, tile[i][jl]);
            }
        } else {
            // A piece of a tile shared with other blocks: this block's
            // partial goes to its slot (0 for its first piece, 1 for its last).
            float* mine = p.part + (static_cast<int64_t>(blockIdx.x) * 2 + (first_piece ? 0 : 1)) * elems;
            for (int64_t e = tid; e < elems; e += kThinThreads) {
                const int64_t i = e / TN, jl = e - i * TN;
                __hip_atomic_store(mine + e, tile[i][jl], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // The partial is written through before the block counts its
            // arrival; the last arrival's agent-scope loads read it there.
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            const int64_t first = block_of(t * p.steps, p.sk_units, blocks);
            const int64_t final_b = block_of((t + 1) * p.steps - 1, p.sk_units, blocks);
            if (tid == 0) {
                unsigned int* ctr = &thin_counters[first * kCounterStride];
                last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       static_cast<unsigned int>(final_b - first);
                if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (last) {
                // Partials of blocks first..final_b added in block order; each
                // thread's elements of four blocks are loaded before any add.
                const int64_t tile_start = t * p.steps;
                for (int e0 = 0; e0 < EPT; e0 += FC) {
                    if (static_cast<int64_t>(e0) * kThinThreads >= elems) break;
                    float v[FC];
#pragma unroll
                    for (int q2 = 0; q2 < FC; ++q2) v[q2] = 0.0f;
                    for (int64_t b0 = first; b0 <= final_b; b0 += 4) {
                        float h[4][FC];
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            const int64_t b = b0 + d;
                            // Tile t is block b's first piece when b starts inside it.
                            const int slot = b * p.sk_units / blocks >= tile_start ? 0 : 1;
                            const float* src = p.part + (b * 2 + slot) * elems;
#pragma unroll
                            for (int q2 = 0; q2 < FC; ++q2) {
                                const int64_t e = tid + (e0 + q2) * kThinThreads;
                                h[d][q2] = b <= final_b && e < elems
                                               ? __hip_atomic_load(src + e, __ATOMIC_RELAXED,
                                                                   __HIP_MEMORY_SCOPE_AGENT)
                                               : 0.0f;
                            }
                        }
#pragma unroll
                        for (int d = 0; d < 4; ++d)
#pragma unroll
                            for (int q2 = 0; q2 < FC; ++q2)
                                if (b0 + d <= final_b) v[q2] += h[d][q2];
                    }
#pragma unroll
                    for (int q2 = 0; q2 < FC; ++q2) {
                        const int64_t e = tid + (e0 + q2) * kThinThreads;
                        if (e < elems) {
                            const int64_t i = e / TN, jl = e - i * TN;
                            if (col0 + jl < p.n) store_c<T>(p, bi, i, col0 + jl, v[q2]);
                        }
                    }
                }
            }
        }
        __syncthreads();  // tile and red are reused by the next piece
    };
    // Split tiles first, so that their folds overlap the whole tiles other
    // blocks are still streaming; whole tiles last.
    for (int64_t u = u_begin; u < u_end;) {
        const int64_t t = u / p.steps;
        const int64_t s0 = u - t * p.steps;
        const int64_t s1 = std::min(p.steps, s0 + (u_end - u));
        piece(t, s0, s1, u == u_begin);
        u += s1 - s0;
    }
    for (int64_t j = 0; j < p.dp_rounds; ++j) {
        const int64_t t = p.sk_tiles + blockIdx.x + j * static_cast<int64_t>(gridDim.x);
        if (t < p.all_tiles) piece(t, 0, p.steps, false);
    }
}

template <typename T, bool KMAJOR, int R, int CB, bool XVEC>
int blocks_per_cu() {
    static const int n = [] {
        int b = 0;
        TP_AMD_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, reinterpret_cast<const void*>(gemm_thin_kernel<T, KMAJOR, R, CB, XVEC>), kThinThreads, 0));
        return std::max(b, 1);
    }();
    return n;
}

template <typename T, bool KMAJOR, int R, int CB, bool XVEC>
int64_t thin_slots(int device) {
    return std::min<int64_t>(static_cast<int64_t>(blocks_per_cu<T, KMAJOR, R, CB, XVEC>()) * cu_count(device),
                             kMaxThinBlocks);
}

// The schedule (see ThinArgs) over `slots` blocks resident at once.
//   * At least a round of tiles: every block takes whole tiles, and the
//     tiles left over from the last round (fewer than a round) are split
//     over the blocks first.  Their folds then overlap the whole tiles other
//     blocks are still streaming, and no fold remains at the end.
//   * Fewer tiles than blocks: every tile is split, into pieces of at least
//     kMinPieceBytes of W -- a tile cut into many small pieces pays for their
//     fold (a write-through, an atomic and the reads, each a trip to the
//     coherent level) more than they gain.
template <typename T, bool KMAJOR, int R, int CB, bool XVEC>
void launch_kernel(ThinArgs q, int64_t batch, hipStream_t stream) {
    using P = Thin<T, KMAJOR, R, CB>;
    int device = 0;
    TP_AMD_HIP_CHECK(hipGetDevice(&device));
    q.tiles = (q.n + P::TN - 1) / P::TN;
    q.steps = (q.k + P::STEP - 1) / P::STEP;
    const int64_t slots = thin_slots<T, KMAJOR, R, CB, XVEC>(device);
    const int64_t tiles = batch * q.tiles;
    const int64_t step_bytes = P::STEP * P::TN * static_cast<int64_t>(sizeof(typename Elem<T>::storage));
    int64_t grid;
    q.all_tiles = tiles;
    if (tiles >= slots && step_bytes * q.steps < kSplitTileBytes) {
        // Small tiles: whole tiles dealt round the blocks (a fold would cost
        // more than the last round's imbalance).
        grid = slots;
        q.sk_tiles = q.sk_units = q.sk_blocks = 0;
        q.dp_rounds = (tiles + slots - 1) / slots;
    } else if (tiles >= slots) {
        grid = slots;
        q.sk_tiles = tiles % slots;
        q.dp_rounds = tiles / slots;
        q.sk_units = q.sk_tiles * q.steps;
        // The left-over tiles over every block, in pieces of at least
        // kMinSplitBytes (the fold of a tile reads every piece).
        q.sk_blocks = std::min(grid, std::max<int64_t>(q.sk_tiles, q.sk_units / std::max<int64_t>(1, kMinSplitBytes / step_bytes)));
    } else {
        // Every tile split, over at most one block a CU for 16-bit types
        // and two for float32: more blocks (more, smaller pieces, each
        // folded) measured slower, e.g. bf16 1 x 4096 x 4096 10.5 us on one
        // block a CU, 11.9 us on two; float32 1 x 11008 x 4096 35.3 us on
        // two, 38.4 us on three.
        q.sk_tiles = tiles;
        q.dp_rounds = 0;
        q.sk_units = tiles * q.steps;
        const int64_t cap = std::min<int64_t>(slots, (P::k16 ? 1 : 2) * static_cast<int64_t>(cu_count(device)));
        grid = std::min(cap, std::max<int64_t>(tiles, q.sk_units / std::max<int64_t>(1, kMinPieceBytes / step_bytes)));
        q.sk_blocks = grid;
    }
    Workspace ws;
    q.part = nullptr;
    // Partials exist only when some tile is split between blocks.
    if (q.sk_blocks > 0 && (q.sk_units % q.sk_blocks != 0 || (q.sk_units / q.sk_blocks) % q.steps != 0)) {
        ws = Workspace(static_cast<size_t>(q.sk_blocks) * 2 * q.m * P::TN * sizeof(float), device);
        q.part = static_cast<float*>(ws.get());
    }
    gemm_thin_kernel<T, KMAJOR, R, CB, XVEC><<<static_cast<unsigned>(grid), kThinThreads, 0, stream>>>(q);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

// Four column groups a wave with W K-major (64-wide tiles).  One group
// (16-wide tiles, so that more products have a whole tile for every block)
// measured slower: bf16 1 x 4096 x 11008 21.3 -> 23.1 us, 32 rows
// 28.9 -> 42.4 us.
constexpr int kColumnGroups = 4;

template <typename T, bool KMAJOR, int R>
void launch_x(const ThinArgs& q, bool xvec, int64_t batch, hipStream_t stream) {
    constexpr int CB = kColumnGroups;
    xvec ? launch_kernel<T, KMAJOR, R, CB, true>(q, batch, stream)
         : launch_kernel<T, KMAJOR, R, CB, false>(q, batch, stream);
}

// Most thin rows a variant takes (rows are padded to 16, 32 or 64).  W
// N-major in 16-bit types holds 8 column groups a wave and spills from 64
// rows on.  128 rows (8 row groups) compiled without spills for W K-major
// but ran no faster than the tiled kernels (bf16 128 x 4096 x 11008 64.8 us
// against 57.8 us): every wave reads its own 128 rows of X for 64 columns
// of W, twice the bytes of W, from L2.
int thin_max_rows(bool k16, bool kmajor) { return !kmajor && k16 ? 32 : 64; }

template <typename T, bool KMAJOR>
void launch_rows(const ThinArgs& q, bool xvec, int64_t batch, hipStream_t stream) {
    constexpr bool k16 = sizeof(typename Elem<T>::storage) == 2;
    if (q.m > 32) {
        if constexpr (KMAJOR || !k16) launch_x<T, KMAJOR, 4>(q, xvec, batch, stream);
    } else if (q.m > 16) {
        launch_x<T, KMAJOR, 2>(q, xvec, batch, stream);
    } else {
        launch_x<T, KMAJOR, 1>(q, xvec, batch, stream);
    }
}

template <typename T>
bool launch_typed(const GemmArgs& p, hipStream_t stream) {
    using S = typename Elem<T>::storage;
    constexpr int V = 16 / sizeof(S);
    constexpr int64_t kLimit = int64_t(1) << 31;
    if (p.k <= 0 || p.m <= 0 || p.n <= 0 || p.batch <= 0 || p.trans_c) return false;
    const bool thin_m = p.m <= kThinMaxRows, thin_n = p.n <= kThinMaxRows;
    if (!thin_m && !thin_n) return false;
    ThinArgs q{};
    q.k = p.k;
    q.alpha = p.alpha;
    q.beta = p.beta;
    q.cin = p.cin;
    bool kmajor;
    if (thin_m && (!thin_n || p.m <= p.n)) {
        // X = A, W = B.
        q.m = p.m;
        q.n = p.n;
        q.x = p.a;
        q.x_m = p.trans_a ? 1 : p.lda;
        q.x_k = p.trans_a ? p.lda : 1;
        q.x_b = p.stride_a;
        q.w = p.b;
        q.w_ld = p.ldb;
        q.w_b = p.stride_b;
        kmajor = p.trans_b;
        q.c_m = p.ldc;
        q.c_n = 1;
        q.cin_m = p.cin_rs;
        q.cin_n = p.cin_cs;
    } else {
        // C^T = B^T A^T: X = B^T, W = A^T.
        q.m = p.n;
        q.n = p.m;
        q.x = p.b;
        q.x_m = p.trans_b ? p.ldb : 1;
        q.x_k = p.trans_b ? 1 : p.ldb;
        q.x_b = p.stride_b;
        q.w = p.a;
        q.w_ld = p.lda;
        q.w_b = p.stride_a;
        kmajor = !p.trans_a;
        q.c_m = 1;
        q.c_n = p.ldc;
        q.cin_m = p.cin_cs;
        q.cin_n = p.cin_rs;
    }
    q.c = p.c;
    q.c_b = p.stride_c;
    q.cin_b = p.cin_stride_b;
    // The wide operand is read in 16-byte packets along its contiguous axis,
    // its rows apart (no overlap), and every byte offset within a tile's
    // resource (and the X resource) below 2^31.
    constexpr int64_t ES = sizeof(S);
    if (!aligned16(q.w) || q.w_ld % V != 0 || q.w_b % V != 0 || (kmajor ? q.k : q.n) % V != 0) return false;
    if (kmajor ? (q.w_ld < q.k || (64 * q.w_ld + q.k) * ES >= kLimit)
               : (q.w_ld < q.n || ((q.k + 64) * q.w_ld + 128) * ES >= kLimit)) {
        return false;
    }
    if (q.x_m < 0 || q.x_k < 0 || ((q.m - 1) * q.x_m + (q.k + 16) * std::max<int64_t>(q.x_k, 1)) * ES >= kLimit) {
        return false;
    }
    // Small products stay on the tiled kernels: below these sizes of the wide
    // operand the thin kernel's fixed costs (resources, the LDS tree, a fold)
    // outweigh what it saves (measured: bf16 32 x 2048 x 256 6.4 us tiled,
    // 10.5 us thin; float32 32 x 1024 x 1024 15.9 us tiled, 18.0 us thin;
    // bf16 16 x 512 x 512 7.9 us tiled, 10.1 us thin; bf16 1 x 1024 x 1024
    // 12.3 us tiled, 7.9 us thin).
    const int64_t wbytes = (q.w_b == 0 ? 1 : p.batch) * q.n * q.k * ES;
    if (wbytes < (q.m > 16 ? kMinWideBytes2 : kMinWideBytes1)) return false;
    const bool xvec = q.x_k == 1 && q.k % V == 0 && aligned16(q.x) && (q.m == 1 || q.x_m % V == 0) &&
                      (p.batch == 1 || q.x_b % V == 0);
    if (q.m > thin_max_rows(sizeof(S) == 2, kmajor)) return false;
    // A 16-bit product of more than 16 rows that the split over K spreads
    // over every CU runs faster there; from 17 to 32 rows with W K-major
    // only when it takes at most eight slices.  Each wave here reads its
    // rows of X again for every 64 columns of W, which costs more as the
    // rows grow, and a long K splits into many slices, each adding a
    // float32 partial of C.  Measured (bf16, W rotated beyond the Infinity
    // Cache, x W^T / x W, us):
    //   33-64 x 11008 x 4096 (86 tiles x 5 slices):  split 31-32 / 35-36, here 41-44 / -
    //   33-64 x 4096 x 11008 (32 tiles x 16 slices): split 31-32 / 33-35, here 34-38 / -
    //   17-32 x 11008 x 4096 (86 x 5):  split 26-29 / 30-32, here 29-31 / 33-35
    //   17-32 x 4096 x 11008 (32 x 16): split 28-29 / 31-32, here 27-30 / 34-35
    if (sizeof(S) == 2 && q.m > 16) {
        int device = 0;
        TP_AMD_HIP_CHECK(hipGetDevice(&device));
        int64_t slices = 1;
        const int64_t blocks = splitk16_blocks(p, device, &slices);
        if (blocks >= cu_count(device) && (q.m > 32 || !kmajor || slices <= 8)) return false;
    }
    if (sizeof(S) == 4 && q.m > 32) {
        int device = 0;
        TP_AMD_HIP_CHECK(hipGetDevice(&device));
        if (splitk32_takes(p, device)) return false;
    }
    if (kmajor) {
        launch_rows<T, true>(q, xvec, p.batch, stream);
    } else {
        // float32 with W N-major reads one X element a step either way.
        launch_rows<T, false>(q, xvec && sizeof(S) == 2, p.batch, stream);
    }
    return true;
}

}  // namespace

bool launch_gemm_thin(int dtype, const GemmArgs& p, hipStream_t stream) {
    switch (dtype) {
        case TP_AMD_FLOAT32: return launch_typed<float>(p, stream);
        case TP_AMD_BFLOAT16: return launch_typed<bf16_t>(p, stream);
        case TP_AMD_FLOAT16: return launch_typed<f16_t>(p, stream);
        default: return false;
    }
}

}  // namespace tp_amd
