/* CPU oracle for the TensorPlay PrivateUse1 hot path -- TEST INFRASTRUCTURE.
 *
 * Only the tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or, for cpu_baseline, as the
 * timed CPU port).  The device backend never calls it and must not fall back
 * to it.
 *
 * What it restates.  The reference computes each hot-path operator with one
 * Cambricon CNNL call whose compute type is float32 and whose result is
 * rounded to the tensor's dtype (tensorplay_mlu/csrc/BinaryKernels.cpp:76,
 * UnaryKernels.cpp:57-59, ReduceKernels.cpp:33-36, BlasKernels.cpp:113,159).
 * CNNL is closed, so its exact float32 operation order is unknowable; the
 * oracle states the operator's mathematical definition, evaluates it in
 * double precision, rounds once to float32 (the compute type) and then to the
 * storage dtype.  Each function cites the reference lines it follows.
 *
 * How it is pinned (tests/test_oracle.py, golden fixtures in tests/golden/):
 *   orc_binary, orc_affine       numpy float64 broadcasting arithmetic; the
 *                                scalar folds (1/s multiply, rsub) against
 *                                hand-derived closed forms
 *   orc_unary                    numpy / scipy.special float64 functions and
 *                                closed-form points (sigmoid(0) = 1/2, ...)
 *   orc_activation_backward      central finite differences of the forward
 *   orc_reduce                   math.fsum / numpy max, closed forms
 *                                (sum of ones, arange), signed-zero and NaN
 *                                cases by hand
 *   orc_softmax(_backward)       scipy.special softmax / log_softmax, the
 *                                explicit Jacobian (diag(y) - y y^T) product
 *   orc_gemm, orc_gemm_entries   numpy float64 matmul, identity/permutation
 *                                and transpose identities
 *   orc_cast, rounding helpers   numpy astype (float16, integers); bfloat16 by
 *                                brute force over all 2^16 patterns and the
 *                                nearest-neighbour/ties-to-even property
 * NaN semantics of amax/amin/relu against TensorPlay's host kernels, and
 * integer conversions outside the target range, are "parity unpinned": no
 * reference test or fixture fixes them.
 */
#ifndef TP_AMD_ORACLE_H
#define TP_AMD_ORACLE_H

#include <stdint.h>

/* dtype codes (same numbering as the library's tp_amd_dtype) */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_F64 = 3, ORC_I8 = 4,
    ORC_I16 = 5, ORC_I32 = 6, ORC_I64 = 7, ORC_U8 = 8, ORC_BOOL = 9
};

int orc_num_threads(void);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);

void orc_binary(int op, int dtype, int ndim, const int64_t* sizes, const void* a,
                const int64_t* a_strides, const void* b, const int64_t* b_strides, void* out,
                const int64_t* out_strides, float alpha);
void orc_affine(int dtype, int64_t n, const void* x, float alpha, float beta, void* y);
void orc_unary(int op, int dtype, int64_t n, const void* x, void* y, float param);
void orc_activation_backward(int op, int dtype, int64_t n, const void* grad, const void* saved,
                             void* dx, float param);
void orc_reduce(int op, int dtype, int64_t outer, int64_t r, int64_t inner, const void* x,
                void* out);
void orc_softmax(int log, int dtype, int64_t outer, int64_t dim, int64_t inner, const void* x,
                 void* y);
void orc_softmax_backward(int log, int dtype, int64_t outer, int64_t dim, int64_t inner,
                          const void* y, const void* dy, void* dx);
void orc_gemm(int dtype, int64_t batch, int64_t m, int64_t n, int64_t k, float alpha,
              const void* a, int64_t lda, int64_t stride_a, int trans_a, const void* b,
              int64_t ldb, int64_t stride_b, int trans_b, float beta, const void* cin,
              int64_t cin_rs, int64_t cin_cs, int64_t cin_stride_b, void* c, int64_t ldc,
              int64_t stride_c);
void orc_gemm_entries(int dtype, int64_t k, float alpha, const void* a, int64_t lda,
                      int64_t stride_a, int trans_a, const void* b, int64_t ldb, int64_t stride_b,
                      int trans_b, float beta, const void* cin, int64_t cin_rs, int64_t cin_cs,
                      int64_t cin_stride_b, const int64_t* bij, int64_t count, double* out);
void orc_cast(int src_dtype, int dst_dtype, int64_t n, const void* src, void* dst);

#endif
