// Pointwise math on float32, shared by the forward and backward kernels.
// Formulas follow the reference operators' definitions
// (tensorplay_mlu/csrc/UnaryKernels.cpp:106-287, BinaryKernels.cpp:44-87);
// the transcendental functions are ROCm's device math library (expf, logf,
// erfcf, tanhf, powf).
#pragma once

#include <hip/hip_runtime.h>

#include "tp_amd_kernels.h"

namespace tp_amd {

constexpr float kSqrt1_2 = 0.70710678118654752440f;    // 1/sqrt(2)
constexpr float kInvSqrt2Pi = 0.39894228040143267794f; // 1/sqrt(2 pi)
constexpr float kSqrt2OverPi = 0.79788456080286535588f; // sqrt(2/pi)
constexpr float kGeluTanhC = 0.044715f;

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

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

template <int OP>
struct UnaryFn {
    float param;
    __device__ __forceinline__ float operator()(float x) const {
        if constexpr (OP == TP_AMD_UNARY_EXP) return expf(x);
        else if constexpr (OP == TP_AMD_UNARY_LOG) return logf(x);
        else if constexpr (OP == TP_AMD_UNARY_SQRT) return sqrtf(x);
        else if constexpr (OP == TP_AMD_UNARY_RSQRT) return 1.0f / sqrtf(x);
        else if constexpr (OP == TP_AMD_UNARY_NEG) return -x;
        else if constexpr (OP == TP_AMD_UNARY_ABS) return fabsf(x);
        else if constexpr (OP == TP_AMD_UNARY_SQUARE) return x * x;
        else if constexpr (OP == TP_AMD_UNARY_POW) return powf(x, param);
        else if constexpr (OP == TP_AMD_UNARY_RELU) return x > 0.0f ? x : 0.0f;
        else if constexpr (OP == TP_AMD_UNARY_SIGMOID) return sigmoidf(x);
        else if constexpr (OP == TP_AMD_UNARY_TANH) return tanhf(x);
        else if constexpr (OP == TP_AMD_UNARY_SILU) return x / (1.0f + expf(-x));
        else if constexpr (OP == TP_AMD_UNARY_GELU) return gelu_erff(x);
        else return gelu_tanhf(x);
    }
};

// dx from the upstream gradient g and the saved operand s (input or output).
template <int OP>
struct BackwardFn {
    float param;
    __device__ __forceinline__ float operator()(float g, float s) const {
        if constexpr (OP == TP_AMD_BACKWARD_THRESHOLD) {
            return s > param ? g : 0.0f;
        } else if constexpr (OP == TP_AMD_BACKWARD_SIGMOID) {
            return g * s * (1.0f - s);
        } else if constexpr (OP == TP_AMD_BACKWARD_TANH) {
            return g * (1.0f - s * s);
        } else if constexpr (OP == TP_AMD_BACKWARD_GELU) {
            const float cdf = 0.5f * erfcf(-s * kSqrt1_2);
            const float pdf = kInvSqrt2Pi * expf(-0.5f * s * s);
            return g * (cdf + s * pdf);
        } else if constexpr (OP == TP_AMD_BACKWARD_GELU_TANH) {
            const float x2 = s * s;
            const float u = kSqrt2OverPi * (s + kGeluTanhC * x2 * s);
            const float sg = sigmoidf(2.0f * u);
            const float du = kSqrt2OverPi * (1.0f + 3.0f * kGeluTanhC * x2);
            return g * (sg + s * sg * (1.0f - sg) * 2.0f * du);
        } else {
            const float sg = sigmoidf(s);
            return g * sg * (1.0f + s * (1.0f - sg));
        }
    }
};

}  // namespace tp_amd
