// Device-side building blocks shared by the gfx950 kernels: element
// conversions (float32 compute, round-to-nearest-even stores), 16-byte
// vector packets, and magic-number division for index math.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace tp_amd {

// Storage types.  bfloat16 and float16 are carried as raw 16-bit patterns
// and converted explicitly, so rounding is exactly round-to-nearest-even
// with NaN kept quiet, independent of compiler defaults.
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round to nearest even, NaN kept quiet (sign and the payload's high bits
// kept, quiet bit set): v_cvt_pk_bf16_f32, which gives exactly these bits
// for every float32 input -- the same as the integer form
// u + 0x7fff + ((u >> 16) & 1) for non-NaN u, (u >> 16) | 0x40 for NaN.
__device__ __forceinline__ uint16_t float_to_bf16(float f) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float floatx2 __attribute__((ext_vector_type(2)));
    const floatx2 v = {f, 0.0f};
    const bf16x2 b = __builtin_convertvector(v, bf16x2);
    uint32_t u;
    __builtin_memcpy(&u, &b, 4);
    return static_cast<uint16_t>(u & 0xffffu);
}

__device__ __forceinline__ float f16_to_float(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t float_to_f16(float f) {
    // v_cvt_f16_f32 rounds to nearest even (the default round mode).
    _Float16 v = static_cast<_Float16>(f);
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

template <typename T>
struct Elem;

template <>
struct Elem<float> {
    using storage = float;
    __device__ __forceinline__ static float load(float v) { return v; }
    __device__ __forceinline__ static float store(float f) { return f; }
};
template <>
struct Elem<bf16_t> {
    using storage = uint16_t;
    __device__ __forceinline__ static float load(uint16_t v) { return bf16_to_float(v); }
    __device__ __forceinline__ static uint16_t store(float f) { return float_to_bf16(f); }
};
template <>
struct Elem<f16_t> {
    using storage = uint16_t;
    __device__ __forceinline__ static float load(uint16_t v) { return f16_to_float(v); }
    __device__ __forceinline__ static uint16_t store(float f) { return float_to_f16(f); }
};

// A 16-byte packet of N = 16 / sizeof(storage) elements.
template <typename T>
struct Packet {
    using S = typename Elem<T>::storage;
    static constexpr int N = 16 / sizeof(S);
    S v[N];
};

template <typename T>
__device__ __forceinline__ Packet<T> load_packet(const typename Elem<T>::storage* p) {
    Packet<T> out;
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    __builtin_memcpy(&out, &raw, 16);
    return out;
}

template <typename T>
__device__ __forceinline__ void store_packet(typename Elem<T>::storage* p, const Packet<T>& v) {
    uint4 raw;
    __builtin_memcpy(&raw, &v, 16);
    *reinterpret_cast<uint4*>(p) = raw;
}

// Streaming variants: the data is touched once, so keep it out of the
// caches' way (nontemporal loads/stores).
template <typename T>
__device__ __forceinline__ Packet<T> load_packet_nt(const typename Elem<T>::storage* p) {
    Packet<T> out;
    uint4 raw;
    const uint4* q = reinterpret_cast<const uint4*>(p);
    raw.x = __builtin_nontemporal_load(&q->x);
    raw.y = __builtin_nontemporal_load(&q->y);
    raw.z = __builtin_nontemporal_load(&q->z);
    raw.w = __builtin_nontemporal_load(&q->w);
    __builtin_memcpy(&out, &raw, 16);
    return out;
}

template <typename T>
__device__ __forceinline__ void store_packet_nt(typename Elem<T>::storage* p, const Packet<T>& v) {
    uint4 raw;
    __builtin_memcpy(&raw, &v, 16);
    uint4* q = reinterpret_cast<uint4*>(p);
    __builtin_nontemporal_store(raw.x, &q->x);
    __builtin_nontemporal_store(raw.y, &q->y);
    __builtin_nontemporal_store(raw.z, &q->z);
    __builtin_nontemporal_store(raw.w, &q->w);
}

// Raw 16-byte packets converted to and from float32 lanes, for kernels whose
// per-element arithmetic is the limit (softmax, transcendental activations):
// bfloat16 unpacks with one shift or mask per element and packs two elements
// per v_cvt_pk_bf16_f32 (round to nearest even, as float_to_bf16 for every
// non-NaN input); float16 converts with v_cvt_f16_f32 (round to nearest even).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ void unpack(const uint4& raw, float (&f)[Packet<T>::N]) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(typename Elem<T>::storage) == 4) {
            f[i] = __uint_as_float(w[i]);
        } else if constexpr (std::is_same_v<T, bf16_t>) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        } else {
            f[2 * i] = f16_to_float(static_cast<uint16_t>(w[i] & 0xffffu));
            f[2 * i + 1] = f16_to_float(static_cast<uint16_t>(w[i] >> 16));
        }
    }
}

template <typename T>
__device__ __forceinline__ uint4 pack(const float (&f)[Packet<T>::N]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(typename Elem<T>::storage) == 4) {
            w[i] = __float_as_uint(f[i]);
        } else if constexpr (std::is_same_v<T, bf16_t>) {
            const floatx2_t v = {f[2 * i], f[2 * i + 1]};
            const bf16x2_t b = __builtin_convertvector(v, bf16x2_t);
            __builtin_memcpy(&w[i], &b, 4);
        } else {
            const floatx2_t v = {f[2 * i], f[2 * i + 1]};
            const f16x2_t h = __builtin_convertvector(v, f16x2_t);
            __builtin_memcpy(&w[i], &h, 4);
        }
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint4 load_raw_nt(const void* p) {
    const uint4* q = static_cast<const uint4*>(p);
    uint4 raw;
    raw.x = __builtin_nontemporal_load(&q->x);
    raw.y = __builtin_nontemporal_load(&q->y);
    raw.z = __builtin_nontemporal_load(&q->z);
    raw.w = __builtin_nontemporal_load(&q->w);
    return raw;
}

__device__ __forceinline__ void store_raw_nt(void* p, const uint4& raw) {
    uint4* q = static_cast<uint4*>(p);
    __builtin_nontemporal_store(raw.x, &q->x);
    __builtin_nontemporal_store(raw.y, &q->y);
    __builtin_nontemporal_store(raw.z, &q->z);
    __builtin_nontemporal_store(raw.w, &q->w);
}

// Unsigned division by a runtime constant d (1 <= d < 2^31) for numerators
// n < 2^31: with s = ceil(log2 d) and m = ceil(2^(31+s) / d) (which fits in
// 32 bits), floor(n / d) = (n * m) >> (31 + s).  The rounding error of m
// adds less than n / 2^(31+s) < 2^-s <= 1/d to n/d, which cannot carry
// floor(n/d) to the next integer.
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t shift;  // 31 + s
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) ++s;
    const uint64_t m = ((uint64_t(1) << (31 + s)) + d - 1) / d;
    return FastDiv{d, static_cast<uint32_t>(m), 31 + s};
}

__device__ __forceinline__ uint32_t fastdiv(uint32_t n, const FastDiv& f) {
    return static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> f.shift);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Wavefront size on gfx9 / CDNA.
constexpr int kWave = 64;

template <typename T>
__device__ __forceinline__ T wave_shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

// Lane value rotated right by N within each row of 16 lanes (DPP row_ror).
template <int N>
__device__ __forceinline__ float row_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xf, 0xf,
                                                      false));
}

// Reduction of v over the 64 lanes of the wave with an associative and
// commutative op, returned to every lane: four DPP rotations combine each
// row of 16 lanes, then the four row results are read as scalars.  A
// handful of cycles, where a shuffle ladder pays LDS latency six times.
template <typename Op>
__device__ __forceinline__ float wave_allreduce(float v, Op op) {
    v = op(v, row_ror<8>(v));
    v = op(v, row_ror<4>(v));
    v = op(v, row_ror<2>(v));
    v = op(v, row_ror<1>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(a, b), op(c, d));
}

// ---- buffer access ------------------------------------------------------------
//
// Row kernels address rows through buffer resources: a 16-byte access past
// the resource's range is dropped by the hardware (a load gives zeros), so a
// thread issues its loads and stores without a branch around each, and the
// compiler can count the outstanding ones exactly -- it waits for a
// prefetched row without also waiting for the stores issued after it.

using Rsrc = __amdgpu_buffer_rsrc_t;
typedef unsigned int U32x4 __attribute__((ext_vector_type(4)));
constexpr int kNt = 2;  // cache policy: non-temporal

// A resource over `bytes` bytes at `base`; 0 bytes makes every access out of
// range (nothing is read or written).
__device__ __forceinline__ Rsrc buffer_over(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buffer_load16(Rsrc r, uint32_t offset) {
    const U32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kNt);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// The same with the default cache policy: the lines are allocated like any
// other, so an operand re-read soon (by the next launch over the same
// tensor, or by the next op) can come from the 256 MB Infinity Cache.
__device__ __forceinline__ uint4 buffer_load16_cached(Rsrc r, uint32_t offset) {
    const U32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ void buffer_store16(Rsrc r, uint32_t offset, const uint4& v) {
    const U32x4 d = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(d, r, offset, 0, kNt);
}

__device__ __forceinline__ float buffer_load_f32(Rsrc r, uint32_t offset) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0));
}

__device__ __forceinline__ void buffer_store_f32(Rsrc r, uint32_t offset, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, offset, 0, 0);
}

// A wave-uniform 64-bit value in scalar registers.
__device__ __forceinline__ int64_t uniform(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

constexpr uint32_t kOutOfRange = 0xfffffff0u;  // an offset past any resource used here

// Waits for every outstanding memory operation.  Before a software-pipelined
// row loop this leaves nothing pending on entry, so the waits the compiler
// places at the loop head follow the loop's own issue order alone.
__device__ __forceinline__ void drain() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace tp_amd
