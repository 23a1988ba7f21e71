// Elementwise kernels for gfx950: broadcasting binary arithmetic, the
// affine transform behind the scalar forms, unary math and activations, and
// the activation backward kernels.
//
// Streaming design (HBM-bound): every thread moves 16-byte packets (4 fp32 or
// 8 bf16/fp16), issues all of its loads before any arithmetic so several
// packets per thread are in flight, and one block covers a contiguous span of
// kUnroll * 256 packets so a wavefront's accesses are fully coalesced.  After
// coalescing, broadcasting reduces to a 2-D [R, C] index space in which each
// operand is full, a row broadcast (b[c]), a column broadcast (b[r]) or a
// scalar; anything else takes the general strided kernel.

#include "device_common.h"
#include "layout.h"
#include "math_ops.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kBlock = 256;
// Packets per thread of the dense kernels.  One 16-byte packet per thread
// over a grid that covers the tensor streamed at 82 % of HBM on MI355X in a
// copy of 2 x 256 MB, against 77 % with four packets per thread.
constexpr int kUnroll = 1;

// 16-bit storage takes the fast transcendental forms (math_ops.h).
template <typename T>
constexpr bool kFast = sizeof(typename Elem<T>::storage) == 2;

#define TP_AMD_DISPATCH_FLOAT(dtype, T, ...)                                      \
    switch (dtype) {                                                              \
        case TP_AMD_FLOAT32: { using T = float; __VA_ARGS__; break; }             \
        case TP_AMD_BFLOAT16: { using T = bf16_t; __VA_ARGS__; break; }           \
        case TP_AMD_FLOAT16: { using T = f16_t; __VA_ARGS__; break; }             \
        default: TP_AMD_CHECK(false, "elementwise kernels take float32, float16 or " \
                              "bfloat16, got ", dtype_name(dtype));               \
    }

// ---- dense kernels: NIN inputs, one output, all contiguous ---------------
//
// Inputs load with the default cache policy, the output stores
// non-temporally.  On [8192, 8192] float32 a copy-like launch takes 72 us
// this way and 81 us with non-temporal loads: inputs read again soon (the
// next launch over the same tensor, the next op of a step) partly come from
// the 256 MB Infinity Cache.  A 1 GiB copy, which cannot stay there, is
// 5 % faster with non-temporal loads (4.9 against 4.8 TB/s).

template <typename T, int NIN, typename F>
__global__ __launch_bounds__(kBlock) void flat_kernel(const typename Elem<T>::storage* in0,
                                                      const typename Elem<T>::storage* in1,
                                                      typename Elem<T>::storage* out,
                                                      int64_t npackets, int64_t n, F f) {
    constexpr int N = Packet<T>::N;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
    Packet<T> x0[kUnroll], x1[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t p = base + k * kBlock;
        if (p < npackets) {
            x0[k] = load_packet<T>(in0 + p * N);
            if constexpr (NIN == 2) x1[k] = load_packet<T>(in1 + p * N);
        }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t p = base + k * kBlock;
        if (p < npackets) {
            float y[N];
#pragma unroll
            for (int j = 0; j < N; ++j) {
                if constexpr (NIN == 1) y[j] = f(Elem<T>::load(x0[k].v[j]));
                else y[j] = f(Elem<T>::load(x0[k].v[j]), Elem<T>::load(x1[k].v[j]));
            }
            store_raw_nt(out + p * N, pack<T>(y));
        }
    }
    // The n % N trailing elements, one per thread of block 0.
    if (blockIdx.x == 0) {
        const int64_t i = npackets * N + threadIdx.x;
        if (i < n) {
            float v;
            if constexpr (NIN == 1) v = f(Elem<T>::load(in0[i]));
            else v = f(Elem<T>::load(in0[i]), Elem<T>::load(in1[i]));
            out[i] = Elem<T>::store(v);
        }
    }
}

// ---- broadcasting binary over [R, C] ---------------------------------------

enum Mode { kFull = 0, kRowB = 1, kColB = 2, kScal = 3 };

template <typename T, int MODE, bool BIG>
__device__ __forceinline__ Packet<T> fetch(const typename Elem<T>::storage* x, int64_t i,
                                           int64_t r, int64_t c) {
    if constexpr (MODE == kFull) {
        return load_packet<T>(x + i);
    } else if constexpr (MODE == kRowB) {
        return load_packet<T>(x + c);
    } else {
        const typename Elem<T>::storage s = MODE == kColB ? x[r] : x[0];
        Packet<T> p;
#pragma unroll
        for (int j = 0; j < Packet<T>::N; ++j) p.v[j] = s;
        return p;
    }
}

// C % N == 0, so a packet never crosses a row.  BIG selects 64-bit index
// math for index spaces of 2^31 elements or more.
template <typename T, int MA, int MB, bool BIG, typename F>
__global__ __launch_bounds__(kBlock) void binary2d_kernel(const typename Elem<T>::storage* a,
                                                          const typename Elem<T>::storage* b,
                                                          typename Elem<T>::storage* out,
                                                          int64_t npackets, int64_t C,
                                                          FastDiv cdiv, F f) {
    constexpr int N = Packet<T>::N;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
    Packet<T> xa[kUnroll], xb[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t p = base + k * kBlock;
        if (p < npackets) {
            const int64_t i = p * N;
            int64_t r, c;
            if constexpr (BIG) {
                r = i / C;
            } else {
                r = fastdiv(static_cast<uint32_t>(i), cdiv);
            }
            c = i - r * C;
            xa[k] = fetch<T, MA, BIG>(a, i, r, c);
            xb[k] = fetch<T, MB, BIG>(b, i, r, c);
        }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
        const int64_t p = base + k * kBlock;
        if (p < npackets) {
            float y[N];
#pragma unroll
            for (int j = 0; j < N; ++j) {
                y[j] = f(Elem<T>::load(xa[k].v[j]), Elem<T>::load(xb[k].v[j]));
            }
            store_raw_nt(out + p * N, pack<T>(y));
        }
    }
}

// ---- general strided index space --------------------------------------------

// Operand 0 is the output; operands 1..NIN the inputs.  The index splits
// into its coordinates with divisions in I: 32-bit when the element count
// allows (a 64-bit division is several times the instructions).
template <typename T, int NIN, typename F, typename I>
__global__ __launch_bounds__(kBlock) void nd_kernel(NdParams<NIN + 1> p,
                                                    typename Elem<T>::storage* out,
                                                    const typename Elem<T>::storage* in0,
                                                    const typename Elem<T>::storage* in1,
                                                    int64_t n, F f) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += stride) {
        I rem = static_cast<I>(i);
        int64_t off[NIN + 1] = {};
        for (int d = p.ndim - 1; d >= 0; --d) {
            const I size = static_cast<I>(p.sizes[d]);
            const I q = rem / size;
            const int64_t idx = static_cast<int64_t>(rem - q * size);
            rem = q;
#pragma unroll
            for (int k = 0; k <= NIN; ++k) off[k] += idx * p.strides[k][d];
        }
        float v;
        if constexpr (NIN == 1) v = f(Elem<T>::load(in0[off[1]]));
        else v = f(Elem<T>::load(in0[off[1]]), Elem<T>::load(in1[off[2]]));
        out[off[0]] = Elem<T>::store(v);
    }
}

// Layouts whose innermost dimension is contiguous in the output and in
// each input, or repeats one input element along it (inner stride 0): the
// inner dimension moves in 16-byte packets, one a thread, and only the
// outer coordinates come from divisions (32-bit, once a packet).  `p`
// holds the outer dimensions; bit k - 1 of `rep` marks input k as
// repeated.  A broadcast add of [B, M, N] and [B, 1, N] is the common case.
template <typename T, int NIN, typename F>
__global__ __launch_bounds__(kBlock) void rows_nd_kernel(NdParams<NIN + 1> p, uint32_t per_row, uint32_t rep,
                                                         typename Elem<T>::storage* out,
                                                         const typename Elem<T>::storage* in0,
                                                         const typename Elem<T>::storage* in1, uint32_t total,
                                                         F f) {
    constexpr int N = Packet<T>::N;
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= total) return;
    uint32_t row = i / per_row;
    const int64_t e = static_cast<int64_t>(i - row * per_row) * N;
    int64_t off[NIN + 1] = {};
    for (int d = p.ndim - 1; d >= 0; --d) {
        const uint32_t size = static_cast<uint32_t>(p.sizes[d]);
        const uint32_t q = row / size;
        const int64_t idx = static_cast<int64_t>(row - q * size);
        row = q;
#pragma unroll
        for (int k = 0; k <= NIN; ++k) off[k] += idx * p.strides[k][d];
    }
    auto fetch_in = [&](const typename Elem<T>::storage* x, int64_t o, bool repeated) {
        Packet<T> v;
        if (repeated) {
            const typename Elem<T>::storage s = x[o];
#pragma unroll
            for (int j = 0; j < N; ++j) v.v[j] = s;
        } else {
            v = load_packet<T>(x + o + e);
        }
        return v;
    };
    const Packet<T> x0 = fetch_in(in0, off[1], rep & 1u);
    float y[N];
    if constexpr (NIN == 1) {
#pragma unroll
        for (int j = 0; j < N; ++j) y[j] = f(Elem<T>::load(x0.v[j]));
    } else {
        const Packet<T> x1 = fetch_in(in1, off[2], rep & 2u);
#pragma unroll
        for (int j = 0; j < N; ++j) y[j] = f(Elem<T>::load(x0.v[j]), Elem<T>::load(x1.v[j]));
    }
    store_raw_nt(out + off[0] + e, pack<T>(y));
}

int64_t flat_grid(int64_t npackets) {
    const int64_t per_block = static_cast<int64_t>(kBlock) * kUnroll;
    const int64_t blocks = (npackets + per_block - 1) / per_block;
    return blocks > 0 ? blocks : 1;
}

int64_t nd_grid(int64_t n, int device) {
    const int64_t want = (n + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(cu_count(device)) * 32;
    return want < cap ? (want > 0 ? want : 1) : cap;
}

// nd_kernel over the n elements of layout l, with 32-bit index arithmetic
// when n allows.
template <typename T, int NIN, typename F>
void launch_nd(int device, const Layout<NIN + 1>& l, void* out, const void* in0, const void* in1, int64_t n,
               F f) {
    using S = typename Elem<T>::storage;
    if (n <= int64_t{0xffffffff}) {
        nd_kernel<T, NIN, F, uint32_t><<<nd_grid(n, device), kBlock, 0, stream(device)>>>(
            nd_params(l), static_cast<S*>(out), static_cast<const S*>(in0), static_cast<const S*>(in1), n, f);
    } else {
        nd_kernel<T, NIN, F, int64_t><<<nd_grid(n, device), kBlock, 0, stream(device)>>>(
            nd_params(l), static_cast<S*>(out), static_cast<const S*>(in0), static_cast<const S*>(in1), n, f);
    }
}

// rows_nd_kernel when the layout allows it (see above); false otherwise.
template <typename T, int NIN, typename F>
bool try_rows_nd(int device, const Layout<NIN + 1>& l, void* out, const void* in0, const void* in1, int64_t n,
                 F f) {
    using S = typename Elem<T>::storage;
    constexpr int N = Packet<T>::N;
    constexpr int64_t kEs = sizeof(S);
    if (l.ndim < 2 || n > int64_t{0xffffffff}) return false;
    const int last = l.ndim - 1;
    const int64_t C = l.sizes[last];
    if (C % N != 0) return false;
    const void* base[3] = {out, in0, in1};
    uint32_t rep = 0;
    for (int k = 0; k <= NIN; ++k) {
        if (k > 0 && l.strides[k][last] == 0) {
            rep |= 1u << (k - 1);
            continue;
        }
        if (l.strides[k][last] != 1 || !aligned16(base[k])) return false;
        for (int d = 0; d < last; ++d) {
            if ((l.strides[k][d] * kEs) % 16 != 0) return false;
        }
    }
    Layout<NIN + 1> outer;
    outer.ndim = last;
    for (int d = 0; d < last; ++d) {
        outer.sizes[d] = l.sizes[d];
        for (int k = 0; k <= NIN; ++k) outer.strides[k][d] = l.strides[k][d];
    }
    const uint32_t total = static_cast<uint32_t>(n / N);
    rows_nd_kernel<T, NIN, F><<<(total + kBlock - 1) / kBlock, kBlock, 0, stream(device)>>>(
        nd_params(outer), static_cast<uint32_t>(C / N), rep, static_cast<S*>(out), static_cast<const S*>(in0),
        static_cast<const S*>(in1), total, f);
    return true;
}

template <typename T, int NIN, typename F>
void launch_flat(int device, const void* in0, const void* in1, void* out, int64_t n, F f) {
    using S = typename Elem<T>::storage;
    constexpr int N = Packet<T>::N;
    const bool vec = aligned16(in0) && aligned16(out) && (NIN == 1 || aligned16(in1));
    const int64_t npackets = vec ? n / N : 0;
    if (!vec) {
        // Unaligned views: the general kernel over one dense dimension.
        Layout<NIN + 1> l;
        l.ndim = 1;
        l.sizes[0] = n;
        for (int k = 0; k <= NIN; ++k) l.strides[k][0] = 1;
        launch_nd<T, NIN, F>(device, l, out, in0, in1, n, f);
    } else {
        flat_kernel<T, NIN, F><<<flat_grid(npackets), kBlock, 0, stream(device)>>>(
            static_cast<const S*>(in0), static_cast<const S*>(in1), static_cast<S*>(out),
            npackets, n, f);
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

int mode_of(const int64_t* strides, int64_t C, bool two_d) {
    const int64_t sr = two_d ? strides[0] : 0;
    const int64_t sc = two_d ? strides[1] : strides[0];
    if (sc == 1 && (!two_d || sr == C)) return kFull;
    if (sc == 1 && sr == 0) return kRowB;
    if (sc == 0 && sr == 1 && two_d) return kColB;
    if (sc == 0 && sr == 0) return kScal;
    return -1;
}

template <typename T, int MA, int MB, typename F>
void launch_binary2d(int device, const void* a, const void* b, void* out, int64_t n, int64_t C,
                     F f) {
    using S = typename Elem<T>::storage;
    constexpr int N = Packet<T>::N;
    const int64_t npackets = n / N;
    const bool big = n >= (int64_t(1) << 31);
    const FastDiv cdiv = make_fastdiv(static_cast<uint32_t>(big ? 1 : C));
    if (big) {
        binary2d_kernel<T, MA, MB, true, F><<<flat_grid(npackets), kBlock, 0, stream(device)>>>(
            static_cast<const S*>(a), static_cast<const S*>(b), static_cast<S*>(out), npackets,
            C, cdiv, f);
    } else {
        binary2d_kernel<T, MA, MB, false, F><<<flat_grid(npackets), kBlock, 0, stream(device)>>>(
            static_cast<const S*>(a), static_cast<const S*>(b), static_cast<S*>(out), npackets,
            C, cdiv, f);
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

// Mode pairs with a specialised kernel; other combinations take nd_kernel.
template <typename T, typename F>
bool try_binary2d(int device, int ma, int mb, const void* a, const void* b, void* out,
                  int64_t n, int64_t C, F f) {
#define TP_AMD_PAIR(MA, MB)                                                       \
    if (ma == MA && mb == MB) {                                                   \
        launch_binary2d<T, MA, MB, F>(device, a, b, out, n, C, f);                \
        return true;                                                              \
    }
    TP_AMD_PAIR(kFull, kFull)
    TP_AMD_PAIR(kFull, kRowB)
    TP_AMD_PAIR(kFull, kColB)
    TP_AMD_PAIR(kFull, kScal)
    TP_AMD_PAIR(kRowB, kFull)
    TP_AMD_PAIR(kColB, kFull)
    TP_AMD_PAIR(kScal, kFull)
    TP_AMD_PAIR(kColB, kRowB)
    TP_AMD_PAIR(kRowB, kColB)
#undef TP_AMD_PAIR
    return false;
}

// out [rows][cols] (row stride ldo) = f(a, b), where an input is read
// row-major (element (r, c) at x[r ld + c]; ld may be 0, a row broadcast) or
// column-major (at x[c ld + r]: a transposed view such as x.t() + y).  One
// 64 x 64 tile a block: the column-major inputs are read along r, their
// unit-stride axis, into LDS as floats; then consecutive threads walk c for
// the row-major inputs and the output, so every HBM access is coalesced.
// The tile rows are 65 floats apart, so the transposed LDS reads of a wave
// fall in 64 different banks.  Tiles run in diagonal order (block b takes
// tile row b % gy, tile column (b / gy + b % gy) % gx) so that blocks that
// run together read the column-major inputs at different offsets.
constexpr int kTTile = 64;

template <typename T, bool ACOL, bool BCOL, typename F>
__global__ __launch_bounds__(kBlock) void binary_transposed_kernel(
    const typename Elem<T>::storage* __restrict__ a, int64_t lda,
    const typename Elem<T>::storage* __restrict__ b, int64_t ldb,
    typename Elem<T>::storage* __restrict__ out, int64_t ldo, int64_t rows, int64_t cols, F f) {
    using S = typename Elem<T>::storage;
    constexpr int kStep = kBlock / kTTile;  // 4 rows of the tile at a time
    constexpr int kPer = kTTile / kStep;    // 16 elements a thread
    __shared__ float ta[ACOL ? kTTile : 1][kTTile + 1];
    __shared__ float tb[BCOL ? kTTile : 1][kTTile + 1];
    const int64_t bid = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    const int64_t ty_tile = bid % gridDim.y, tx_tile = (bid / gridDim.y + ty_tile) % gridDim.x;
    const int64_t r0 = ty_tile * kTTile, c0 = tx_tile * kTTile;
    const int tx = threadIdx.x % kTTile, ty = threadIdx.x / kTTile;
    const bool full = r0 + kTTile <= rows && c0 + kTTile <= cols;
    auto stage = [&](const S* x, int64_t ld, float (*tile)[kTTile + 1]) {
        S v[kPer];
        if (full) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) v[k] = x[(c0 + ty + k * kStep) * ld + r0 + tx];
        } else {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int64_t r = r0 + tx, c = c0 + ty + k * kStep;
                v[k] = r < rows && c < cols ? x[c * ld + r] : S{};
            }
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) tile[ty + k * kStep][tx] = Elem<T>::load(v[k]);
    };
    const int64_t c = c0 + tx;
    S ra[kPer], rb[kPer];
    auto load_rows = [&] {
        if constexpr (!ACOL || !BCOL) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int64_t r = r0 + ty + k * kStep;
                const bool in = full || (r < rows && c < cols);
                if constexpr (!ACOL) ra[k] = in ? a[r * lda + c] : S{};
                if constexpr (!BCOL) rb[k] = in ? b[r * ldb + c] : S{};
            }
        }
    };
    // 4-byte types load the row-major input before staging, so its reads
    // overlap the staging reads (fp32 x.t() + y 4096^2: 31.4 -> 29.8 us);
    // 16-bit types measured slower that way (24.8 -> 27.9 us) and load it
    // after the barrier.
    constexpr bool kEarly = sizeof(S) == 4;
    if constexpr (kEarly) load_rows();
    if constexpr (ACOL) stage(a, lda, ta);
    if constexpr (BCOL) stage(b, ldb, tb);
    __syncthreads();
    if constexpr (!kEarly) load_rows();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int64_t r = r0 + ty + k * kStep;
        const float va = ACOL ? ta[tx][ty + k * kStep] : Elem<T>::load(ra[k]);
        const float vb = BCOL ? tb[tx][ty + k * kStep] : Elem<T>::load(rb[k]);
        if (full || (r < rows && c < cols)) out[r * ldo + c] = Elem<T>::store(f(va, vb));
    }
}

// The two-dimensional case with a row-major output and at least one
// column-major input; false when the layout is anything else.
template <typename T, typename F>
bool try_binary_transposed(int device, const Layout<3>& l, const void* a, const void* b, void* out,
                           F f) {
    using S = typename Elem<T>::storage;
    if constexpr (sizeof(S) > 4) {
        return false;
    } else {
        if (l.ndim != 2) return false;
        const int64_t R = l.sizes[0], C = l.sizes[1];
        const int64_t* so = l.strides[0];
        const int64_t* sa = l.strides[1];
        const int64_t* sb = l.strides[2];
        if (so[1] != 1 || so[0] < C) return false;
        auto col = [&](const int64_t* st) { return st[0] == 1 && st[1] >= R; };
        auto row = [&](const int64_t* st) { return st[1] == 1 && st[0] >= 0; };
        const bool acol = col(sa), bcol = col(sb);
        if (!(acol || bcol) || !(acol || row(sa)) || !(bcol || row(sb))) return false;
        const int64_t gx = (C + kTTile - 1) / kTTile, gy = (R + kTTile - 1) / kTTile;
        if (gy > 65535 || gx * gy >= (int64_t(1) << 31)) return false;
        const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
        const S* pa = static_cast<const S*>(a);
        const S* pb = static_cast<const S*>(b);
        S* po = static_cast<S*>(out);
        const int64_t lda = acol ? sa[1] : sa[0], ldb = bcol ? sb[1] : sb[0];
        hipStream_t st = stream(device);
        if (acol && bcol) {
            binary_transposed_kernel<T, true, true, F><<<grid, kBlock, 0, st>>>(pa, lda, pb, ldb, po, so[0], R, C, f);
        } else if (acol) {
            binary_transposed_kernel<T, true, false, F><<<grid, kBlock, 0, st>>>(pa, lda, pb, ldb, po, so[0], R, C, f);
        } else {
            binary_transposed_kernel<T, false, true, F><<<grid, kBlock, 0, st>>>(pa, lda, pb, ldb, po, so[0], R, C, f);
        }
        TP_AMD_HIP_CHECK(hipGetLastError());
        return true;
    }
}

template <typename T, typename F>
void binary_typed(int device, int ndim, const int64_t* sizes, const void* a,
                  const int64_t* as, const void* b, const int64_t* bs, void* out,
                  const int64_t* os, F f) {
    constexpr int N = Packet<T>::N;
    const int64_t* strides[3] = {os, as, bs};
    const Layout<3> l = coalesce<3>(ndim, sizes, strides);
    const int64_t n = l.numel();
    if (n == 0) return;
    if (l.ndim <= 2) {
        const bool two_d = l.ndim == 2;
        const int64_t C = l.ndim == 0 ? 1 : l.sizes[l.ndim - 1];
        int64_t zero[2] = {0, 0};
        const int64_t* so = l.ndim == 0 ? zero : l.strides[0];
        const int64_t* sa = l.ndim == 0 ? zero : l.strides[1];
        const int64_t* sb = l.ndim == 0 ? zero : l.strides[2];
        const int mo = l.ndim == 0 ? kFull : mode_of(so, C, two_d);
        const int ma = l.ndim == 0 ? kFull : mode_of(sa, C, two_d);
        const int mb = l.ndim == 0 ? kFull : mode_of(sb, C, two_d);
        const bool packets = C % N == 0 && aligned16(out) &&
                             (ma == kColB || ma == kScal || aligned16(a)) &&
                             (mb == kColB || mb == kScal || aligned16(b));
        if (mo == kFull && ma >= 0 && mb >= 0 && packets &&
            try_binary2d<T>(device, ma, mb, a, b, out, n, C, f)) {
            return;
        }
    }
    if (try_binary_transposed<T, F>(device, l, a, b, out, f)) return;
    if (!try_rows_nd<T, 2, F>(device, l, out, a, b, n, f)) launch_nd<T, 2, F>(device, l, out, a, b, n, f);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template <typename T, typename F>
void unary_typed(int device, int ndim, const int64_t* sizes, const void* x, const int64_t* xs,
                 void* y, F f) {
    int64_t ys[TP_AMD_MAX_DIMS];
    contiguous_strides(ndim, sizes, ys);
    const int64_t* strides[2] = {ys, xs};
    const Layout<2> l = coalesce<2>(ndim, sizes, strides);
    const int64_t n = l.numel();
    if (n == 0) return;
    if (l.ndim == 0 || (l.ndim == 1 && l.strides[0][0] == 1 && l.strides[1][0] == 1)) {
        launch_flat<T, 1, F>(device, x, nullptr, y, n, f);
        return;
    }
    if (!try_rows_nd<T, 1, F>(device, l, y, x, nullptr, n, f)) launch_nd<T, 1, F>(device, l, y, x, nullptr, n, f);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

#define TP_AMD_UNARY_CASE(OP)                                                         \
    case OP:                                                                          \
        unary_typed<T>(index, ndim, sizes, x, x_strides, y, UnaryFn<OP, kFast<T>>{param}); \
        break;

template <typename T>
void unary_dispatch(int index, int op, int ndim, const int64_t* sizes, const void* x,
                    const int64_t* x_strides, void* y, float param) {
    switch (op) {
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_EXP)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_LOG)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_SQRT)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_RSQRT)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_NEG)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_ABS)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_SQUARE)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_POW)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_RELU)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_SIGMOID)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_TANH)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_SILU)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_GELU)
        TP_AMD_UNARY_CASE(TP_AMD_UNARY_GELU_TANH)
        default: TP_AMD_CHECK(false, "unknown unary op ", op);
    }
}
#undef TP_AMD_UNARY_CASE

#define TP_AMD_BWD_CASE(OP)                                                            \
    case OP:                                                                           \
        launch_flat<T, 2>(index, grad, saved, dx, n, BackwardFn<OP, kFast<T>>{param}); \
        break;

template <typename T>
void backward_dispatch(int index, int op, int64_t n, const void* grad, const void* saved,
                       void* dx, float param) {
    switch (op) {
        TP_AMD_BWD_CASE(TP_AMD_BACKWARD_THRESHOLD)
        TP_AMD_BWD_CASE(TP_AMD_BACKWARD_SIGMOID)
        TP_AMD_BWD_CASE(TP_AMD_BACKWARD_TANH)
        TP_AMD_BWD_CASE(TP_AMD_BACKWARD_GELU)
        TP_AMD_BWD_CASE(TP_AMD_BACKWARD_GELU_TANH)
        TP_AMD_BWD_CASE(TP_AMD_BACKWARD_SILU)
        default: TP_AMD_CHECK(false, "unknown backward op ", op);
    }
}
#undef TP_AMD_BWD_CASE

}  // namespace

}  // namespace tp_amd

using namespace tp_amd;

extern "C" {

int tp_amd_launch_binary(int device, int op, int dtype, int ndim, const int64_t* sizes,
                         const void* a, const int64_t* a_strides, const void* b,
                         const int64_t* b_strides, void* out, const int64_t* out_strides,
                         float alpha) {
    return guarded([&] {
        const OnDevice scope(device);
        const int index = scope.index();
        TP_AMD_DISPATCH_FLOAT(dtype, T, {
            switch (op) {
                case TP_AMD_BINARY_ADD:
                    binary_typed<T>(index, ndim, sizes, a, a_strides, b, b_strides, out,
                                    out_strides, BinaryFn<TP_AMD_BINARY_ADD>{alpha});
                    break;
                case TP_AMD_BINARY_MUL:
                    binary_typed<T>(index, ndim, sizes, a, a_strides, b, b_strides, out,
                                    out_strides, BinaryFn<TP_AMD_BINARY_MUL>{alpha});
                    break;
                case TP_AMD_BINARY_DIV:
                    binary_typed<T>(index, ndim, sizes, a, a_strides, b, b_strides, out,
                                    out_strides, BinaryFn<TP_AMD_BINARY_DIV>{alpha});
                    break;
                default: TP_AMD_CHECK(false, "unknown binary op ", op);
            }
        });
    });
}

int tp_amd_launch_affine(int device, int dtype, int64_t n, const void* x, float alpha,
                         float beta, void* y) {
    return guarded([&] {
        TP_AMD_CHECK(n >= 0, "negative element count");
        if (n == 0) return;
        const OnDevice scope(device);
        const int index = scope.index();
        TP_AMD_DISPATCH_FLOAT(dtype, T,
                              launch_flat<T, 1>(index, x, nullptr, y, n, AffineFn{alpha, beta}));
    });
}

int tp_amd_launch_unary(int device, int op, int dtype, int ndim, const int64_t* sizes,
                        const void* x, const int64_t* x_strides, void* y, float param) {
    return guarded([&] {
        const OnDevice scope(device);
        const int index = scope.index();
        TP_AMD_DISPATCH_FLOAT(dtype, T,
                              unary_dispatch<T>(index, op, ndim, sizes, x, x_strides, y, param));
    });
}

int tp_amd_launch_activation_backward(int device, int op, int dtype, int64_t n,
                                      const void* grad, const void* saved, void* dx,
                                      float param) {
    return guarded([&] {
        TP_AMD_CHECK(n >= 0, "negative element count");
        if (n == 0) return;
        const OnDevice scope(device);
        const int index = scope.index();
        TP_AMD_DISPATCH_FLOAT(dtype, T,
                              backward_dispatch<T>(index, op, n, grad, saved, dx, param));
    });
}

}  // extern "C"
