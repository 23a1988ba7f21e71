// Matrix products for gfx950 (the reference's cnnlMatMul_v2 /
// cnnlStrideBatchMatMul_v3, tensorplay_mlu/csrc/BlasKernels.cpp:202-242).
//
// C[b] = alpha * op(A[b]) op(B[b]) + beta * Cin[b], float32 accumulation,
// result rounded once to the dtype.  Transposed operands are read in place:
// the tile loaders index the stored matrix directly.
//
// This file holds the general kernel: 64x64 output tiles, 256 threads each
// owning a 4x4 patch, K staged through LDS 16 at a time, any leading
// dimension and alignment, bounds-checked edges.

#include "device_common.h"
#include "gemm.h"
#include "../runtime.h"
#include "tp_amd_kernels.h"

namespace tp_amd {

namespace {

constexpr int kGBlock = 256;
constexpr int kGTile = 64;
constexpr int kGK = 16;

template <typename T>
__global__ __launch_bounds__(kGBlock) void gemm_general_kernel(GemmArgs p) {
    using S = typename Elem<T>::storage;
    __shared__ float As[kGK][kGTile + 4];
    __shared__ float Bs[kGK][kGTile + 4];
    const S* A = static_cast<const S*>(p.a);
    const S* B = static_cast<const S*>(p.b);
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kGTile;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kGTile;
    for (int64_t bi = blockIdx.z; bi < p.batch; bi += gridDim.z) {
        const S* Ab = A + bi * p.stride_a;
        const S* Bb = B + bi * p.stride_b;
        float acc[4][4] = {};
        for (int64_t k0 = 0; k0 < p.k; k0 += kGK) {
#pragma unroll
            for (int q = 0; q < (kGTile * kGK) / kGBlock; ++q) {
                const int e = threadIdx.x + q * kGBlock;
                // A tile: rows along the contiguous axis when A is stored
                // transposed (K x M), along K otherwise.
                int i, kk;
                if (p.trans_a) {
                    i = e % kGTile;
                    kk = e / kGTile;
                } else {
                    kk = e % kGK;
                    i = e / kGK;
                }
                const int64_t gm = m0 + i, gk = k0 + kk;
                float va = 0.0f;
                if (gm < p.m && gk < p.k) {
                    va = Elem<T>::load(p.trans_a ? Ab[gk * p.lda + gm] : Ab[gm * p.lda + gk]);
                }
                As[kk][i] = va;
                int j, kb;
                if (p.trans_b) {
                    kb = e % kGK;
                    j = e / kGK;
                } else {
                    j = e % kGTile;
                    kb = e / kGTile;
                }
                const int64_t gn = n0 + j, gkb = k0 + kb;
                float vb = 0.0f;
                if (gn < p.n && gkb < p.k) {
                    vb = Elem<T>::load(p.trans_b ? Bb[gn * p.ldb + gkb] : Bb[gkb * p.ldb + gn]);
                }
                Bs[kb][j] = vb;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < kGK; ++kk) {
                float av[4], bv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) av[r] = As[kk][ty * 4 + r];
#pragma unroll
                for (int c = 0; c < 4; ++c) bv[c] = Bs[kk][tx * 4 + c];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(av[r], bv[c], acc[r][c]);
            }
            __syncthreads();
        }
        S* C = static_cast<S*>(p.c) + bi * p.stride_c;
        const S* Cin = static_cast<const S*>(p.cin);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t gm = m0 + ty * 4 + r;
            if (gm >= p.m) continue;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t gn = n0 + tx * 4 + c;
                if (gn >= p.n) continue;
                float v = p.alpha * acc[r][c];
                if (p.beta != 0.0f) {
                    v = fmaf(p.beta,
                             Elem<T>::load(Cin[bi * p.cin_stride_b + gm * p.cin_rs + gn * p.cin_cs]),
                             v);
                }
                C[gm * p.ldc + gn] = Elem<T>::store(v);
            }
        }
    }
}

}  // namespace

template <typename T>
void launch_gemm_general(const GemmArgs& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((p.n + kGTile - 1) / kGTile),
                    static_cast<unsigned>((p.m + kGTile - 1) / kGTile),
                    static_cast<unsigned>(p.batch < 65535 ? p.batch : 65535));
    gemm_general_kernel<T><<<grid, kGBlock, 0, stream>>>(p);
    TP_AMD_HIP_CHECK(hipGetLastError());
}

template void launch_gemm_general<float>(const GemmArgs&, hipStream_t);
template void launch_gemm_general<bf16_t>(const GemmArgs&, hipStream_t);
template void launch_gemm_general<f16_t>(const GemmArgs&, hipStream_t);

}  // namespace tp_amd

using namespace tp_amd;

extern "C" {

int tp_amd_launch_gemm(int device, int dtype, int64_t batch, int64_t m, int64_t n, int64_t k,
                       float alpha, const void* a, int64_t lda, int64_t stride_a, int trans_a,
                       const void* b, int64_t ldb, int64_t stride_b, int trans_b, float beta,
                       const void* cin, int64_t cin_rs, int64_t cin_cs, int64_t cin_stride_b,
                       void* c, int64_t ldc, int64_t stride_c) {
    return guarded([&] {
        TP_AMD_CHECK(batch >= 0 && m >= 0 && n >= 0 && k >= 0, "negative GEMM extent");
        if (batch == 0 || m == 0 || n == 0) return;
        TP_AMD_CHECK(beta == 0.0f || cin != nullptr, "beta != 0 needs an input C");
        TP_AMD_CHECK(lda >= (trans_a ? m : k) || k == 0, "lda too small");
        TP_AMD_CHECK(ldb >= (trans_b ? k : n) || k == 0, "ldb too small");
        TP_AMD_CHECK(ldc >= n, "ldc too small");
        const OnDevice scope(device);
        const int index = scope.index();
        GemmArgs p{};
        p.batch = batch;
        p.m = m;
        p.n = n;
        p.k = k;
        p.alpha = alpha;
        p.beta = beta;
        p.a = a;
        p.lda = lda;
        p.stride_a = stride_a;
        p.trans_a = trans_a != 0;
        p.b = b;
        p.ldb = ldb;
        p.stride_b = stride_b;
        p.trans_b = trans_b != 0;
        p.cin = cin;
        p.cin_rs = cin_rs;
        p.cin_cs = cin_cs;
        p.cin_stride_b = cin_stride_b;
        p.c = c;
        p.ldc = ldc;
        p.stride_c = stride_c;
        launch_gemm(dtype, p, stream(index));
    });
}

}  // extern "C"
