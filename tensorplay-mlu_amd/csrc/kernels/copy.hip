// Fill, dtype conversion and strided copy kernels for gfx950.
//
// * Fill writes 16-byte packets of the replicated element pattern when the
//   view is dense, the strided kernel otherwise.
// * Conversion covers every pair of the ten dtypes; each thread converts
//   kPerThread elements with coalesced accesses.  Float to narrower float
//   rounds to nearest even, float to integer truncates toward zero
//   (saturating to int64, NaN to 0) and wraps to the target width, anything
//   to bool is x != 0.
// * Strided copy merges dimensions first; a dense copy is one device memcpy,
//   a 2-D transpose goes through a padded LDS tile so both the read and the
//   write side are coalesced, anything else takes the general kernel.

#include <cstring>

#include "device_common.h"
#include "layout.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kBlock = 256;

template <int BYTES>
struct Raw;
template <>
struct Raw<1> { using type = uint8_t; };
template <>
struct Raw<2> { using type = uint16_t; };
template <>
struct Raw<4> { using type = uint32_t; };
template <>
struct Raw<8> { using type = uint64_t; };

int64_t grid_for(int64_t work, int64_t per_block, int device) {
    int64_t blocks = (work + per_block - 1) / per_block;
    const int64_t cap = static_cast<int64_t>(cu_count(device)) * 64;
    if (blocks > cap) blocks = cap;
    return blocks > 0 ? blocks : 1;
}

// ---- fill --------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void fill_dense_kernel(uint4* dst, int64_t npackets,
                                                            uint4 pattern) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < npackets;
         i += stride) {
        dst[i] = pattern;
    }
}

template <typename R>
__global__ __launch_bounds__(kBlock) void fill_nd_kernel(NdParams<1> p, R* dst, int64_t n,
                                                         R value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += stride) {
        int64_t rem = i, off = 0;
        for (int d = p.ndim - 1; d >= 0; --d) {
            const int64_t q = rem / p.sizes[d];
            off += (rem - q * p.sizes[d]) * p.strides[0][d];
            rem = q;
        }
        dst[off] = value;
    }
}

template <typename R>
void fill_typed(int device, const void* value, int ndim, const int64_t* sizes, void* dst,
                const int64_t* strides) {
    R v;
    std::memcpy(&v, value, sizeof(R));
    const int64_t* s[1] = {strides};
    const Layout<1> l = coalesce<1>(ndim, sizes, s);
    const int64_t n = l.numel();
    if (n == 0) return;
    hipStream_t st = stream(device);
    const bool dense = l.ndim == 0 || (l.ndim == 1 && l.strides[0][0] == 1);
    if (dense && aligned16(dst)) {
        uint4 pattern;
        R rep[16 / sizeof(R)];
        for (auto& r : rep) r = v;
        std::memcpy(&pattern, rep, 16);
        const int64_t npackets = n * static_cast<int64_t>(sizeof(R)) / 16;
        if (npackets > 0) {
            fill_dense_kernel<<<grid_for(npackets, kBlock * 4, device), kBlock, 0, st>>>(
                static_cast<uint4*>(dst), npackets, pattern);
            TP_AMD_HIP_CHECK(hipGetLastError());
        }
        const int64_t done = npackets * 16 / static_cast<int64_t>(sizeof(R));
        if (done < n) {
            Layout<1> tail;
            tail.ndim = 1;
            tail.sizes[0] = n - done;
            tail.strides[0][0] = 1;
            fill_nd_kernel<R><<<1, kBlock, 0, st>>>(nd_params(tail), static_cast<R*>(dst) + done,
                                                    n - done, v);
            TP_AMD_HIP_CHECK(hipGetLastError());
        }
        return;
    }
    fill_nd_kernel<R><<<grid_for(n, kBlock * 4, device), kBlock, 0, st>>>(
        nd_params(l), static_cast<R*>(dst), n, v);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

// ---- conversion ----------------------------------------------------------

// Device element types by dtype code.
struct F32 { using S = float; };
struct F16 { using S = uint16_t; };
struct BF16 { using S = uint16_t; };
struct F64 { using S = double; };
struct I8 { using S = int8_t; };
struct I16 { using S = int16_t; };
struct I32 { using S = int32_t; };
struct I64 { using S = int64_t; };
struct U8 { using S = uint8_t; };
struct B1 { using S = uint8_t; };

template <typename D>
constexpr bool is_float_tag() {
    return std::is_same<D, F32>::value || std::is_same<D, F16>::value ||
           std::is_same<D, BF16>::value || std::is_same<D, F64>::value;
}

// Read an element as either a double (float sources) or an int64 (integer
// and bool sources).  float16 and bfloat16 widen exactly.
template <typename D>
__device__ __forceinline__ double read_float(typename D::S v) {
    if constexpr (std::is_same<D, F16>::value) return f16_to_float(v);
    else if constexpr (std::is_same<D, BF16>::value) return bf16_to_float(v);
    else return static_cast<double>(v);
}

template <typename D>
__device__ __forceinline__ typename D::S write_from_float(double x) {
    if constexpr (std::is_same<D, F64>::value) {
        return x;
    } else if constexpr (std::is_same<D, F32>::value) {
        return static_cast<float>(x);
    } else if constexpr (std::is_same<D, F16>::value) {
        // Through float32: the source is float32 or narrower except for
        // float64 sources, which the operator layer routes through float32.
        return float_to_f16(static_cast<float>(x));
    } else if constexpr (std::is_same<D, BF16>::value) {
        return float_to_bf16(static_cast<float>(x));
    } else if constexpr (std::is_same<D, B1>::value) {
        return static_cast<uint8_t>(x != 0.0 ? 1 : 0);
    } else {
        // Truncate toward zero into int64 (saturating, NaN -> 0), then wrap.
        int64_t t;
        if (!(x == x)) t = 0;
        else if (x >= 9223372036854775807.0) t = INT64_MAX;
        else if (x <= -9223372036854775808.0) t = INT64_MIN;
        else t = static_cast<int64_t>(x);
        return static_cast<typename D::S>(t);
    }
}

template <typename D>
__device__ __forceinline__ typename D::S write_from_int(int64_t x) {
    if constexpr (std::is_same<D, F64>::value) return static_cast<double>(x);
    else if constexpr (std::is_same<D, F32>::value) return static_cast<float>(x);
    else if constexpr (std::is_same<D, F16>::value) return float_to_f16(static_cast<float>(x));
    else if constexpr (std::is_same<D, BF16>::value) return float_to_bf16(static_cast<float>(x));
    else if constexpr (std::is_same<D, B1>::value) return static_cast<uint8_t>(x != 0 ? 1 : 0);
    else return static_cast<typename D::S>(x);
}

// float32 -> float16 / bfloat16 directly from a float (the hot casts).
template <typename Src, typename Dst>
__device__ __forceinline__ typename Dst::S convert(typename Src::S v) {
    if constexpr (std::is_same<Src, Dst>::value && !std::is_same<Src, B1>::value) {
        return v;
    } else if constexpr (std::is_same<Src, F32>::value && std::is_same<Dst, BF16>::value) {
        return float_to_bf16(v);
    } else if constexpr (std::is_same<Src, F32>::value && std::is_same<Dst, F16>::value) {
        return float_to_f16(v);
    } else if constexpr (std::is_same<Src, B1>::value) {
        return write_from_int<Dst>(v != 0 ? 1 : 0);
    } else if constexpr (is_float_tag<Src>()) {
        return write_from_float<Dst>(read_float<Src>(v));
    } else {
        return write_from_int<Dst>(static_cast<int64_t>(v));
    }
}

constexpr int kPerThread = 8;

template <typename Src, typename Dst>
__global__ __launch_bounds__(kBlock) void cast_kernel(const typename Src::S* src,
                                                      typename Dst::S* dst, int64_t n) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kBlock * kPerThread) + threadIdx.x;
    typename Src::S v[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const int64_t i = base + k * kBlock;
        if (i < n) v[k] = src[i];
    }
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const int64_t i = base + k * kBlock;
        if (i < n) dst[i] = convert<Src, Dst>(v[k]);
    }
}

// Between 2- and 4-byte types with both buffers 16-byte aligned: a thread
// converts the elements of one 16-byte packet of the wider type (4 for
// float32 <-> 16-bit, 8 or 4 when both sides are alike), so each load and
// store instruction covers one contiguous span (the scalar kernel's lanes
// move 2 or 4 bytes an access).  Same conversions, same bits.
template <typename Src, typename Dst>
constexpr int packed_elems() {
    return 16 / static_cast<int>(sizeof(typename Src::S) > sizeof(typename Dst::S) ? sizeof(typename Src::S)
                                                                                     : sizeof(typename Dst::S));
}

template <int BYTES>
__device__ __forceinline__ void load_bytes(void* dst, const void* src) {
    if constexpr (BYTES == 16) {
        const uint4 v = *static_cast<const uint4*>(src);
        __builtin_memcpy(dst, &v, 16);
    } else {
        const uint2 v = *static_cast<const uint2*>(src);
        __builtin_memcpy(dst, &v, 8);
    }
}

template <int BYTES>
__device__ __forceinline__ void store_bytes_nt(void* dst, const void* src) {
    if constexpr (BYTES == 16) {
        uint4 v;
        __builtin_memcpy(&v, src, 16);
        store_raw_nt(dst, v);
    } else {
        uint64_t v;
        __builtin_memcpy(&v, src, 8);
        __builtin_nontemporal_store(v, static_cast<uint64_t*>(dst));
    }
}

template <typename Src, typename Dst>
__global__ __launch_bounds__(kBlock) void cast_packed_kernel(const typename Src::S* src,
                                                             typename Dst::S* dst, int64_t groups) {
    using SS = typename Src::S;
    using DS = typename Dst::S;
    constexpr int E = packed_elems<Src, Dst>();
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (g >= groups) return;
    SS v[E];
    DS o[E];
    load_bytes<E * sizeof(SS)>(v, src + g * E);
#pragma unroll
    for (int j = 0; j < E; ++j) o[j] = convert<Src, Dst>(v[j]);
    store_bytes_nt<E * sizeof(DS)>(dst + g * E, o);
}

template <typename Src, typename Dst>
void cast_typed(int device, int64_t n, const void* src, void* dst) {
    using SS = typename Src::S;
    using DS = typename Dst::S;
    const SS* s = static_cast<const SS*>(src);
    DS* d = static_cast<DS*>(dst);
    constexpr bool kPackable = (sizeof(SS) == 2 || sizeof(SS) == 4) && (sizeof(DS) == 2 || sizeof(DS) == 4) &&
                               !std::is_same<Src, B1>::value && !std::is_same<Dst, B1>::value;
    if constexpr (kPackable) {
        constexpr int E = packed_elems<Src, Dst>();
        const int64_t groups = n / E;
        if (groups > 0 && aligned16(src) && aligned16(dst)) {
            const int64_t blocks = (groups + kBlock - 1) / kBlock;
            cast_packed_kernel<Src, Dst><<<blocks, kBlock, 0, stream(device)>>>(s, d, groups);
            TP_AMD_HIP_CHECK(hipGetLastError());
            s += groups * E;  // the last n % E elements below
            d += groups * E;
            n -= groups * E;
            if (n == 0) return;
        }
    }
    const int64_t per_block = static_cast<int64_t>(kBlock) * kPerThread;
    const int64_t blocks = (n + per_block - 1) / per_block;
    cast_kernel<Src, Dst><<<blocks, kBlock, 0, stream(device)>>>(s, d, n);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template <typename Src>
void cast_from(int device, int dst_dtype, int64_t n, const void* src, void* dst) {
    switch (dst_dtype) {
        case TP_AMD_FLOAT32: cast_typed<Src, F32>(device, n, src, dst); break;
        case TP_AMD_FLOAT16: cast_typed<Src, F16>(device, n, src, dst); break;
        case TP_AMD_BFLOAT16: cast_typed<Src, BF16>(device, n, src, dst); break;
        case TP_AMD_FLOAT64: cast_typed<Src, F64>(device, n, src, dst); break;
        case TP_AMD_INT8: cast_typed<Src, I8>(device, n, src, dst); break;
        case TP_AMD_INT16: cast_typed<Src, I16>(device, n, src, dst); break;
        case TP_AMD_INT32: cast_typed<Src, I32>(device, n, src, dst); break;
        case TP_AMD_INT64: cast_typed<Src, I64>(device, n, src, dst); break;
        case TP_AMD_UINT8: cast_typed<Src, U8>(device, n, src, dst); break;
        case TP_AMD_BOOL: cast_typed<Src, B1>(device, n, src, dst); break;
        default: TP_AMD_CHECK(false, "unknown destination dtype ", dst_dtype);
    }
}

// ---- strided copy ------------------------------------------------------------

// The general case, one element a lane.  The index splits into its
// coordinates with divisions in I: 32-bit when the element count allows
// (a 64-bit division is several times the instructions).
template <typename R, typename I>
__global__ __launch_bounds__(kBlock) void copy_nd_kernel(NdParams<2> p, R* dst, const R* src,
                                                         int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += stride) {
        I rem = static_cast<I>(i);
        int64_t od = 0, os = 0;
        for (int d = p.ndim - 1; d >= 0; --d) {
            const I size = static_cast<I>(p.sizes[d]);
            const I q = rem / size;
            const int64_t idx = static_cast<int64_t>(rem - q * size);
            od += idx * p.strides[0][d];
            os += idx * p.strides[1][d];
            rem = q;
        }
        dst[od] = src[os];
    }
}

// Rows of whole 16-byte packets (a row-padded slice, a narrow): packet c
// of row r at dst[r * ld_dst + c] and src[r * ld_src + c].  One packet a
// lane, blockIdx.y walking the rows, no division.
// (Restrict: without it a store may alias the next load, and the compiler
// copies the packet as four dependent 4-byte loads and stores.)
__global__ __launch_bounds__(kBlock) void copy_rows_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                           int64_t rows, int64_t cols, int64_t ld_dst,
                                                           int64_t ld_src) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= cols) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const uint4 v = src[r * ld_src + c];
        store_raw_nt(dst + r * ld_dst + c, v);
    }
}

// dst[r, c] (row stride ld_dst, unit column stride) = src[r, c] read with
// unit row stride and column stride ld_src: a transpose.  64x64 tiles staged
// through LDS with one element of padding per row.
constexpr int kTile = 64;

// A thread's 16 loads go out together before any LDS write (a loop of
// load, wait, write left one in flight at a time), and full tiles skip the
// bounds tests.
template <typename R>
__global__ __launch_bounds__(kBlock) void transpose_kernel(R* __restrict__ dst, const R* __restrict__ src,
                                                           int64_t rows, int64_t cols, int64_t ld_dst,
                                                           int64_t ld_src) {
    constexpr int kStep = kBlock / kTile;  // 4 rows of the tile at a time
    constexpr int kPer = kTile / kStep;    // 16 elements a thread
    __shared__ R tile[kTile][kTile + 1];
    // Diagonal tile order: block b takes tile row b % gy and tile column
    // (b / gy + b % gy) % gx (a bijection), so blocks that run together
    // read the source's strided rows at different offsets.
    const int64_t b = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    const int64_t ty_tile = b % gridDim.y, tx_tile = (b / gridDim.y + ty_tile) % gridDim.x;
    const int64_t r0 = ty_tile * kTile;
    const int64_t c0 = tx_tile * kTile;
    const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;  // 64 x 4
    const bool full = r0 + kTile <= rows && c0 + kTile <= cols;
    R v[kPer];
    // Read: consecutive threads walk r (the source's unit-stride axis).
    if (full) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) v[k] = src[(c0 + ty + k * kStep) * ld_src + r0 + tx];
    } else {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int64_t r = r0 + tx, c = c0 + ty + k * kStep;
            v[k] = r < rows && c < cols ? src[c * ld_src + r] : R{};
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) tile[ty + k * kStep][tx] = v[k];
    __syncthreads();
    // Write: consecutive threads walk c (the destination's unit-stride axis).
#pragma unroll
    for (int k = 0; k < kPer; ++k) v[k] = tile[tx][ty + k * kStep];
    if (full) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) dst[(r0 + ty + k * kStep) * ld_dst + c0 + tx] = v[k];
    } else {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int64_t r = r0 + ty + k * kStep, c = c0 + tx;
            if (r < rows && c < cols) dst[r * ld_dst + c] = v[k];
        }
    }
}

template <typename R>
void copy_typed(int device, const Layout<2>& l, void* dst, const void* src) {
    const int64_t n = l.numel();
    hipStream_t st = stream(device);
    if (l.ndim == 2 && l.strides[0][1] == 1 && l.strides[1][0] == 1 &&
        l.strides[0][0] >= l.sizes[1] && l.strides[1][1] >= l.sizes[0]) {
        const dim3 grid(static_cast<unsigned>((l.sizes[1] + kTile - 1) / kTile),
                        static_cast<unsigned>((l.sizes[0] + kTile - 1) / kTile));
        if (grid.y < 65536u) {
            transpose_kernel<R><<<grid, kBlock, 0, st>>>(static_cast<R*>(dst),
                                                         static_cast<const R*>(src), l.sizes[0],
                                                         l.sizes[1], l.strides[0][0],
                                                         l.strides[1][1]);
            TP_AMD_HIP_CHECK(hipGetLastError());
            return;
        }
    }
    if (n <= int64_t{0xffffffff}) {
        copy_nd_kernel<R, uint32_t><<<grid_for(n, kBlock * 4, device), kBlock, 0, st>>>(
            nd_params(l), static_cast<R*>(dst), static_cast<const R*>(src), n);
    } else {
        copy_nd_kernel<R, int64_t><<<grid_for(n, kBlock * 4, device), kBlock, 0, st>>>(
            nd_params(l), static_cast<R*>(dst), static_cast<const R*>(src), n);
    }
    TP_AMD_HIP_CHECK(hipGetLastError());
}

// The layout in 16-byte elements, when the innermost dimension is
// contiguous in both operands and the row bytes, every other stride in
// bytes and both base addresses are multiples of 16; otherwise ndim 0.
Layout<2> in_packets(const Layout<2>& l, int elem_size, const void* dst, const void* src) {
    Layout<2> w;
    const int last = l.ndim - 1;
    if (l.ndim < 2 || l.strides[0][last] != 1 || l.strides[1][last] != 1 || !aligned16(dst) ||
        !aligned16(src) || (l.sizes[last] * elem_size) % 16 != 0) {
        return w;
    }
    for (int d = 0; d < last; ++d) {
        for (int k = 0; k < 2; ++k) {
            if ((l.strides[k][d] * elem_size) % 16 != 0) return w;
        }
    }
    w.ndim = l.ndim;
    for (int d = 0; d < last; ++d) {
        w.sizes[d] = l.sizes[d];
        for (int k = 0; k < 2; ++k) w.strides[k][d] = l.strides[k][d] * elem_size / 16;
    }
    w.sizes[last] = l.sizes[last] * elem_size / 16;
    w.strides[0][last] = w.strides[1][last] = 1;
    return w;
}

void copy_packets(int device, const Layout<2>& w, void* dst, const void* src) {
    hipStream_t st = stream(device);
    if (w.ndim == 2) {
        const int64_t cols = w.sizes[1], rows = w.sizes[0];
        const dim3 grid(static_cast<unsigned>((cols + kBlock - 1) / kBlock),
                        static_cast<unsigned>(rows < 65535 ? rows : 65535));
        if ((cols + kBlock - 1) / kBlock < (int64_t{1} << 31)) {
            copy_rows_kernel<<<grid, kBlock, 0, st>>>(static_cast<uint4*>(dst), static_cast<const uint4*>(src),
                                                      rows, cols, w.strides[0][0], w.strides[1][0]);
            TP_AMD_HIP_CHECK(hipGetLastError());
            return;
        }
    }
    copy_typed<uint4>(device, w, dst, src);
}

}  // namespace

}  // namespace tp_amd

using namespace tp_amd;

extern "C" {

int tp_amd_launch_fill(int device, int elem_size, const void* value, int ndim,
                       const int64_t* sizes, void* dst, const int64_t* dst_strides) {
    return guarded([&] {
        TP_AMD_CHECK(value != nullptr, "tp_amd_launch_fill: null value");
        const OnDevice scope(device);
        const int index = scope.index();
        switch (elem_size) {
            case 1: fill_typed<uint8_t>(index, value, ndim, sizes, dst, dst_strides); break;
            case 2: fill_typed<uint16_t>(index, value, ndim, sizes, dst, dst_strides); break;
            case 4: fill_typed<uint32_t>(index, value, ndim, sizes, dst, dst_strides); break;
            case 8: fill_typed<uint64_t>(index, value, ndim, sizes, dst, dst_strides); break;
            default: TP_AMD_CHECK(false, "fill: element size ", elem_size, " not 1/2/4/8");
        }
    });
}

int tp_amd_launch_cast(int device, int src_dtype, int dst_dtype, int64_t n, const void* src,
                       void* dst) {
    return guarded([&] {
        TP_AMD_CHECK(n >= 0, "negative element count");
        if (n == 0) return;
        const OnDevice scope(device);
        const int index = scope.index();
        switch (src_dtype) {
            case TP_AMD_FLOAT32: cast_from<F32>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_FLOAT16: cast_from<F16>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_BFLOAT16: cast_from<BF16>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_FLOAT64: cast_from<F64>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_INT8: cast_from<I8>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_INT16: cast_from<I16>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_INT32: cast_from<I32>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_INT64: cast_from<I64>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_UINT8: cast_from<U8>(index, dst_dtype, n, src, dst); break;
            case TP_AMD_BOOL: cast_from<B1>(index, dst_dtype, n, src, dst); break;
            default: TP_AMD_CHECK(false, "unknown source dtype ", src_dtype);
        }
    });
}

int tp_amd_launch_strided_copy(int device, int elem_size, int ndim, const int64_t* sizes,
                               void* dst, const int64_t* dst_strides, const void* src,
                               const int64_t* src_strides) {
    return guarded([&] {
        const OnDevice scope(device);
        const int index = scope.index();
        const int64_t* s[2] = {dst_strides, src_strides};
        const Layout<2> l = coalesce<2>(ndim, sizes, s);
        const int64_t n = l.numel();
        if (n == 0) return;
        if (l.ndim == 0 || (l.ndim == 1 && l.strides[0][0] == 1 && l.strides[1][0] == 1)) {
            copy_on_device(dst, src, static_cast<size_t>(n) * elem_size, index);
            return;
        }
        const Layout<2> w = in_packets(l, elem_size, dst, src);
        if (w.ndim > 0) {
            copy_packets(index, w, dst, src);
            return;
        }
        switch (elem_size) {
            case 1: copy_typed<uint8_t>(index, l, dst, src); break;
            case 2: copy_typed<uint16_t>(index, l, dst, src); break;
            case 4: copy_typed<uint32_t>(index, l, dst, src); break;
            case 8: copy_typed<uint64_t>(index, l, dst, src); break;
            default: TP_AMD_CHECK(false, "copy: element size ", elem_size, " not 1/2/4/8");
        }
    });
}

}  // extern "C"
