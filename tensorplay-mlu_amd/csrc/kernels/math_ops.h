// Pointwise math on float32, shared by the forward and backward kernels.
// Formulas follow the reference operators' definitions
// (tensorplay_mlu/csrc/UnaryKernels.cpp:106-287, BinaryKernels.cpp:44-87).
//
// Two precisions of the transcendental functions, chosen by the storage
// dtype (FAST = 16-bit storage):
//   * float32 storage: ROCm's device math library (expf, logf, erfcf, tanhf,
//     powf), accurate to an ulp or two;
//   * bfloat16 / float16 storage, where the result keeps 8 or 11 significant
//     bits and the library functions' instruction count, not HBM, would set
//     the pace: the hardware v_exp_f32 / v_log_f32 / v_sqrt_f32 / v_rcp_f32
//     and, for the normal CDF, the Chebyshev-fitted erfc of Numerical Recipes
//     in C (2nd ed., section 6.2, "erfcc": relative error below 1.2e-7 for
//     every argument).  Their float32 errors (a few 1e-7 relative) move a
//     16-bit result by at most one unit in its last place.
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

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---- fast forms (16-bit storage) ------------------------------------------------

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// ln x on v_log_f32 (log2); subnormal inputs are scaled into the normal range
// first, so they are not flushed.
__device__ __forceinline__ float log_fast(float x) {
    const bool tiny = x < 1.17549435e-38f;
    const float l = __builtin_amdgcn_logf(tiny ? x * 16777216.0f : x);
    return (tiny ? l - 24.0f : l) * kLn2;
}

__device__ __forceinline__ float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + exp_fast(-x));
}

// erfc(z) for z >= 0: t exp(-z^2 + P(t)), t = 1 / (1 + z/2), P the degree-9
// Chebyshev fit of Numerical Recipes' erfcc.
__device__ __forceinline__ float erfc_pos_fast(float z) {
    const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
    float p = 0.17087277f;
    p = fmaf(p, t, -0.82215223f);
    p = fmaf(p, t, 1.48851587f);
    p = fmaf(p, t, -1.13520398f);
    p = fmaf(p, t, 0.27886807f);
    p = fmaf(p, t, -0.18628806f);
    p = fmaf(p, t, 0.09678418f);
    p = fmaf(p, t, 0.37409196f);
    p = fmaf(p, t, 1.00002368f);
    p = fmaf(p, t, -1.26551223f);
    return t * exp_fast(fmaf(-z, z, p));
}

// Normal CDF Phi(x) = erfc(-x / sqrt(2)) / 2.
__device__ __forceinline__ float phi_fast(float x) {
    const float z = x * 0.70710678118654752440f;  // -(-x / sqrt 2)
    const float c = erfc_pos_fast(fabsf(z));      // erfc(|z|)
    return 0.5f * (z >= 0.0f ? 2.0f - c : c);
}

// 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3), evaluated as
// x * sigmoid(2u), the same function without the cancellation of 1 + tanh(u)
// for large negative x.
__device__ __forceinline__ float gelu_tanhf(float x) {
    const float u = kSqrt2OverPi * (x + kGeluTanhC * x * x * x);
    return x * sigmoidf(2.0f * u);
}

// x Phi(x) = 0.5 x erfc(-x / sqrt(2)).
__device__ __forceinline__ float gelu_erff(float x) { return 0.5f * x * erfcf(-x * kSqrt1_2); }

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
        else if constexpr (OP == TP_AMD_UNARY_SQRT) return FAST ? __builtin_amdgcn_sqrtf(x) : sqrtf(x);
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
            return FAST ? x * phi_fast(x) : gelu_erff(x);
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
            const float cdf = FAST ? phi_fast(s) : 0.5f * erfcf(-s * kSqrt1_2);
            const float pdf = kInvSqrt2Pi * (FAST ? exp_fast(-0.5f * s * s) : expf(-0.5f * s * s));
            return g * (cdf + s * pdf);
        } else if constexpr (OP == TP_AMD_BACKWARD_GELU_TANH) {
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
