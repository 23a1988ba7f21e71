// Pointwise math on float32, shared by the forward and backward kernels.
// Formulas follow the reference operators' definitions
// (tensorplay_mlu/csrc/UnaryKernels.cpp:106-287, BinaryKernels.cpp:44-87).
//
// Two precisions of the transcendental functions, chosen by the storage
// dtype (FAST = 16-bit storage):
//   * float32 storage: ROCm's device math library (expf, logf, tanhf, powf),
//     accurate to an ulp or two, except the normal CDF and density of gelu's
//     erf form and its backward (normal_f32 below: a few ulps, at HBM speed);
//   * bfloat16 / float16 storage, where the result keeps 8 or 11 significant
//     bits and the library functions' instruction count, not HBM, would set
//     the pace: the hardware v_exp_f32 / v_log_f32 / v_sqrt_f32 / v_rcp_f32
//     and, for the normal CDF, the Chebyshev-fitted erfc of Numerical Recipes
//     in C (2nd ed., section 6.2, "erfcc": relative error below 1.2e-7 for
//     every argument).  Their float32 errors (a few 1e-7 relative) move a
//     16-bit result by at most one unit in its last place, which the GPU
//     tests check at every finite 16-bit input.
#pragma once

#include <hip/hip_runtime.h>

#include "tp_amd_kernels.h"

namespace tp_amd {

constexpr float kSqrt1_2 = 0.70710678118654752440f;    // 1/sqrt(2)
constexpr float kInvSqrt2Pi = 0.39894228040143267794f; // 1/sqrt(2 pi)
constexpr float kSqrt2OverPi = 0.79788456080286535588f; // sqrt(2/pi)
constexpr float kGeluTanhC = 0.044715f;

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;

// 1 / (1 + e^-x) from e = e^-|x| <= 1: for x < 0 it is e / (1 + e), so the
// exponential never overflows and a sigmoid far below 1 keeps its value
// (1 / (1 + inf) would give 0 below x = -88.7, where the result is a float32
// subnormal).
__device__ __forceinline__ float sigmoidf(float x) {
    const float e = expf(-fabsf(x));
    const float r = 1.0f / (1.0f + e);
    return x >= 0.0f ? r : e * r;
}

// ---- fast forms (16-bit storage) ------------------------------------------------
//
// v_exp_f32 returns 0 for results below 2^-126, where bfloat16 (float32's
// exponent range) still has subnormal values, and v_sqrt_f32 reads a
// subnormal input as 0 (both measured over every bfloat16 value).

// e^x as (2^(a/2))^2, a = x log2 e: the halves stay normal down to a = -252
// and their product underflows gradually.  One multiply and about one
// float32 ulp more than 2^a alone, where a select between a raised and a
// plain argument cost five instructions (bfloat16 gelu 46 -> 59 us).
__device__ __forceinline__ float exp_fast(float x) {
    const float h = __builtin_amdgcn_exp2f(x * (0.5f * kLog2e));
    return h * h;
}

// sqrt on v_sqrt_f32, a subnormal x scaled by 2^32 first and the root by 2^-16 after.
__device__ __forceinline__ float sqrt_fast(float x) {
    const bool tiny = x < 0x1p-126f;
    const float r = __builtin_amdgcn_sqrtf(tiny ? x * 0x1p32f : x);
    return tiny ? r * 0x1p-16f : r;
}

// ln x on v_log_f32 (log2); subnormal inputs are scaled into the normal range
// first, so they are not flushed.
__device__ __forceinline__ float log_fast(float x) {
    const bool tiny = x < 1.17549435e-38f;
    const float l = __builtin_amdgcn_logf(tiny ? x * 16777216.0f : x);
    return (tiny ? l - 24.0f : l) * kLn2;
}

// sigmoidf's form on the hardware exponential and reciprocal.
__device__ __forceinline__ float sigmoid_fast(float x) {
    const float e = exp_fast(-fabsf(x));
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    return x >= 0.0f ? r : e * r;
}

// P(t) of erfc(z) = t exp(-z^2 + P(t)), t = 1 / (1 + z/2), z >= 0: the
// degree-9 Chebyshev fit of Numerical Recipes' erfcc.
__device__ __forceinline__ float erfc_fit(float t) {
    float p = 0.17087277f;
    p = fmaf(p, t, -0.82215223f);
    p = fmaf(p, t, 1.48851587f);
    p = fmaf(p, t, -1.13520398f);
    p = fmaf(p, t, 0.27886807f);
    p = fmaf(p, t, -0.18628806f);
    p = fmaf(p, t, 0.09678418f);
    p = fmaf(p, t, 0.37409196f);
    p = fmaf(p, t, 1.00002368f);
    return fmaf(p, t, -1.26551223f);
}

// x Phi(x) for a 16-bit result.  Phi(x) = 1 - q (x >= 0) or q (x < 0) with
// q = erfc(|x| / sqrt 2) / 2 = t e^(-x^2 / 2 + P(t)) / 2 and
// t = 1 / (1 + |x| / (2 sqrt 2)), P of degree 5 fitted here (least squares
// on 2000 Chebyshev nodes, reweighted towards the largest errors) to
// log(erfcx(z) / t) for z = |x| / sqrt 2 in [0, 9.5], where erfc reaches
// bfloat16's smallest values: erfc's relative error is at most 7.6e-6
// (degree 9: 1.2e-7), far under half a 16-bit ulp.  The exponential runs as
// h^2 with h = 2^(-(x k)^2 + P'(t)), k^2 = log2(e) / 4 and P' = (P log2(e)
// - 1) / 2 (the factor 1/2 folded in): h stays normal where q is
// subnormal.  18 VALU operations a value against 26 for x * phi(x) on the
// degree-9 P; an operator whose VALU work otherwise exceeds its memory time.
// (The derivative keeps the degree-9 P: near its zero at x = -0.75,
// cdf + x pdf cancels, and a degree-5 P gave 21 fp16 ulps there in a float32
// emulation.)
__device__ __forceinline__ float gelu16(float x) {
    const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(x), 0.35355339f, 1.0f));  // 1 / (2 sqrt 2)
    const float xs = x * 0.60056120f;                                          // sqrt(log2(e) / 4)
    float p = 0.16503832f;
    p = fmaf(p, t, -0.51157612f);
    p = fmaf(p, t, 0.34227800f);
    p = fmaf(p, t, 0.18354011f);
    p = fmaf(p, t, 0.73434204f);
    p = fmaf(p, t, -1.41361678f);
    const float h = __builtin_amdgcn_exp2f(fmaf(-xs, xs, p));
    const float q = t * (h * h);
    return x * (x >= 0.0f ? 1.0f - q : q);
}

// Phi(x) and the density phi(x) = e^(-x^2/2) / sqrt(2 pi) together: with
// z = x / sqrt 2, erfc(|z|) = t e^(-z^2) e^P(t) shares e^(-z^2) with the
// density (e^P(t) lies in [0.28, 1], so it takes the plain instruction).
__device__ __forceinline__ float phi_pdf_fast(float x, float& pdf) {
    const float z = x * kSqrt1_2;
    const float az = fabsf(z);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, az, 1.0f));
    const float e = exp_fast(-az * az);  // e^(-z^2)
    const float c = t * e * __builtin_amdgcn_exp2f(erfc_fit(t) * kLog2e);
    pdf = kInvSqrt2Pi * e;
    return z >= 0.0f ? fmaf(-0.5f, c, 1.0f) : 0.5f * c;
}

// 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3), evaluated as
// x * sigmoid(2u), the same function without the cancellation of 1 + tanh(u)
// for large negative x.
__device__ __forceinline__ float gelu_tanhf(float x) {
    const float u = kSqrt2OverPi * (x + kGeluTanhC * x * x * x);
    return x * sigmoidf(2.0f * u);
}

// The normal CDF Phi(x) for float32 storage and, with WANT_PDF, the density
// phi(x) in *pdf.  The library form 0.5 erfc(-x / sqrt 2) loses accuracy
// before erfcf runs: rounding z = x / sqrt 2 to float32 moves erfc(z) by
// 2 z^2 times z's relative error (14-23 ulps at 1 <= |x| < 5, ~200 at
// |x| > 8), and erfcf's instruction count made float32 gelu compute-bound.
// Here z = zh + zlo with zlo the rounding error of zh (1/sqrt 2 carried to
// 48 bits), and erfc(z) = t exp(-z^2 + P(t)) with the erfcc fit above:
// z^2 = zz + zl exactly (zz = zh^2 rounded, zl its rounding error plus
// 2 zh zlo), e^-zz is reduced by n ln 2 (Cody and Waite: n = rint(-zz
// log2 e); ln 2 split so that n ln2_hi is exact for |n| < 2^12) and the
// small rest, r - zl + P(t), goes to v_exp_f32 and v_ldexp_f32.  The density
// shares the reduction: phi(x) = e^(-z^2) / sqrt(2 pi).  Emulated in float64
// against scipy.special.erfc over |x| <= 14: gelu within 9 ulps everywhere
// (the library form: 14-200), the density within 3.  Measured on [8192,
// 8192] float32: gelu 74.7-75.6 us against 88-98 us with erfcf, the
// backward 133-139 us against 156-165 us (relu 72.6 us).
template <bool WANT_PDF>
__device__ __forceinline__ float normal_f32(float x, float* pdf) {
    constexpr float kSqrt1_2Lo = 1.21016175e-08f;  // 1/sqrt(2) - kSqrt1_2
    constexpr float kLn2Hi = 0.69311523f;          // ln 2 with 12 trailing zero bits
    constexpr float kLn2Lo = 3.1946183e-05f;       // ln 2 - kLn2Hi
    const float ax = fabsf(x);
    const float zh = ax * kSqrt1_2;
    const float zlo = fmaf(ax, kSqrt1_2, -zh) + ax * kSqrt1_2Lo;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, zh, 1.0f));
    const float p = erfc_fit(t);
    // Beyond z = 10.5 erfc and the density are below float32's range (and an
    // infinite z would make NaN of the reduction): both are 0 there.
    const bool live = zh < 10.5f;
    const float zs = live ? zh : 0.0f;
    const float zz = zs * zs;
    const float zl = fmaf(zs, zs, -zz) + 2.0f * zs * (live ? zlo : 0.0f);
    const float n = rintf(-zz * kLog2e);
    const float r = fmaf(-n, kLn2Lo, fmaf(-n, kLn2Hi, -zz));
    const int ni = static_cast<int>(n);
    const float c = live ? t * __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((r + (p - zl)) * kLog2e), ni) : 0.0f;
    if constexpr (WANT_PDF) {
        *pdf = live ? kInvSqrt2Pi * __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((r - zl) * kLog2e), ni) : 0.0f;
    }
    return x >= 0.0f ? fmaf(-0.5f, c, 1.0f) : 0.5f * c;
}

template <int OP>
struct BinaryFn;

template <>
struct BinaryFn<TP_AMD_BINARY_ADD> {
    float alpha;
    __device__ __forceinline__ float operator()(float a, float b) const {
        return fmaf(alpha, b, a);
    }
};
template <>
struct BinaryFn<TP_AMD_BINARY_MUL> {
    float alpha;
    __device__ __forceinline__ float operator()(float a, float b) const { return a * b; }
};
template <>
struct BinaryFn<TP_AMD_BINARY_DIV> {
    float alpha;
    __device__ __forceinline__ float operator()(float a, float b) const { return a / b; }
};

struct AffineFn {
    float alpha, beta;
    __device__ __forceinline__ float operator()(float x) const { return fmaf(alpha, x, beta); }
};

template <int OP, bool FAST = false>
struct UnaryFn {
    float param;
    __device__ __forceinline__ float operator()(float x) const {
        if constexpr (OP == TP_AMD_UNARY_EXP) return FAST ? exp_fast(x) : expf(x);
        else if constexpr (OP == TP_AMD_UNARY_LOG) return FAST ? log_fast(x) : logf(x);
        else if constexpr (OP == TP_AMD_UNARY_SQRT) return FAST ? sqrt_fast(x) : sqrtf(x);
        else if constexpr (OP == TP_AMD_UNARY_RSQRT) return 1.0f / sqrtf(x);
        else if constexpr (OP == TP_AMD_UNARY_NEG) return -x;
        else if constexpr (OP == TP_AMD_UNARY_ABS) return fabsf(x);
        else if constexpr (OP == TP_AMD_UNARY_SQUARE) return x * x;
        else if constexpr (OP == TP_AMD_UNARY_POW) return powf(x, param);
        else if constexpr (OP == TP_AMD_UNARY_RELU) return x > 0.0f ? x : 0.0f;
        else if constexpr (OP == TP_AMD_UNARY_SIGMOID) return FAST ? sigmoid_fast(x) : sigmoidf(x);
        else if constexpr (OP == TP_AMD_UNARY_TANH) return tanhf(x);
        else if constexpr (OP == TP_AMD_UNARY_SILU) {
            return FAST ? x * sigmoid_fast(x) : x / (1.0f + expf(-x));
        } else if constexpr (OP == TP_AMD_UNARY_GELU) {
            if constexpr (FAST) return gelu16(x);
            else return x * normal_f32<false>(x, nullptr);
        } else {
            if constexpr (FAST) {
                const float u = kSqrt2OverPi * (x + kGeluTanhC * x * x * x);
                return x * sigmoid_fast(2.0f * u);
            } else {
                return gelu_tanhf(x);
            }
        }
    }
};

// dx from the upstream gradient g and the saved operand s (input or output).
template <int OP, bool FAST = false>
struct BackwardFn {
    float param;
    __device__ __forceinline__ float sigmoid(float x) const {
        return FAST ? sigmoid_fast(x) : sigmoidf(x);
    }
    __device__ __forceinline__ float operator()(float g, float s) const {
        if constexpr (OP == TP_AMD_BACKWARD_THRESHOLD) {
            return s > param ? g : 0.0f;
        } else if constexpr (OP == TP_AMD_BACKWARD_SIGMOID) {
            return g * s * (1.0f - s);
        } else if constexpr (OP == TP_AMD_BACKWARD_TANH) {
            return g * (1.0f - s * s);
        } else if constexpr (OP == TP_AMD_BACKWARD_GELU) {
            float cdf, pdf;
            if constexpr (FAST) {
                cdf = phi_pdf_fast(s, pdf);
            } else {
                cdf = normal_f32<true>(s, &pdf);
            }
            return g * (cdf + s * pdf);
        } else if constexpr (OP == TP_AMD_BACKWARD_GELU_TANH) {
            // Beyond |s| = 20 the derivative rounds to 1 (s > 0) or to 0
            // (s < 0) in float32; s is held there so that s^2 and du stay
            // finite (past |s| = 1.8e19, s^2 overflows and 0 * inf would give
            // NaN).  A NaN s stays NaN.
            s = fabsf(s) > 20.0f ? copysignf(20.0f, s) : s;
            const float x2 = s * s;
            const float u = kSqrt2OverPi * (s + kGeluTanhC * x2 * s);
            const float sg = sigmoid(2.0f * u);
            const float du = kSqrt2OverPi * (1.0f + 3.0f * kGeluTanhC * x2);
            return g * (sg + s * sg * (1.0f - sg) * 2.0f * du);
        } else {
            const float sg = sigmoid(s);
            return g * sg * (1.0f + s * (1.0f - sg));
        }
    }
};

}  // namespace tp_amd
