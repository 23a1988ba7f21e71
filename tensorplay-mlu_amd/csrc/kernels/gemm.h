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
    // Split-K partials of a 16-bit product (gemm_mfma_kernel's float32
    // output): the product's whole K; batch entry s covers k = s k ..
    // min((s + 1) k, k_total).
    int64_t k_total = 0;
};

// Any shape, stride and alignment (gemm.hip).
template <typename T>
void launch_gemm_general(const GemmArgs& p, hipStream_t stream);

// Products with at most 64 rows or 64 columns whose large operand the
// matrix cores can read in place (gemm_thin.hip); false when not eligible.
bool launch_gemm_thin(int dtype, const GemmArgs& p, hipStream_t stream);

// The blocks (128 x 128 tiles times K slices) that the 16-bit split over K
// launches for a product of one matrix, 0 when it does not split, and the
// slices (gemm_mfma.hip).  The thin kernel leaves products to the split
// when these are enough to fill the CUs.
int64_t splitk16_blocks(const GemmArgs& p, int device, int64_t* slices);

// True when a float32 product of 33-64 thin rows against a wide operand
// goes to gemm_mfma.hip's split over K on 64 x 64 tiles.
bool splitk32_takes(const GemmArgs& p, int device);

// Picks the matrix-core kernel when the operands allow it, the general one
// otherwise (gemm_mfma.hip).
void launch_gemm(int dtype, const GemmArgs& p, hipStream_t stream);

}  // namespace tp_amd
