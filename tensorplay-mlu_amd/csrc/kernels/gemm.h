// Shared argument block and launch entry of the GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tp_amd {

struct GemmArgs {
    int64_t batch, m, n, k;
    float alpha, beta;
    const void* a;
    int64_t lda, stride_a;
    const void* b;
    int64_t ldb, stride_b;
    const void* cin;
    int64_t cin_rs, cin_cs, cin_stride_b;
    void* c;
    int64_t ldc, stride_c;
    bool trans_a, trans_b;
    // C stored transposed: element (i, j) of the product at c + j ldc + i
    // (gemm_mfma_kernel only; set by the dispatch when it computes C^T).
    bool trans_c = false;
};

// Any shape, stride and alignment (gemm.hip).
template <typename T>
void launch_gemm_general(const GemmArgs& p, hipStream_t stream);

// Products with at most 64 rows or 64 columns whose large operand the
// matrix cores can read in place (gemm_thin.hip); false when not eligible.
bool launch_gemm_thin(int dtype, const GemmArgs& p, hipStream_t stream);

// Picks the matrix-core kernel when the operands allow it, the general one
// otherwise (gemm_mfma.hip).
void launch_gemm(int dtype, const GemmArgs& p, hipStream_t stream);

}  // namespace tp_amd
