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
 *   orc_layer_norm(_backward)    torch float64 layer_norm and its autograd
 *                                gradients; central finite differences of the
 *                                float64 forward; shift/scale invariance and
 *                                the constant row (tests/test_oracle_nn.py)
 *   orc_philox4x32_10            the Random123 known-answer vectors
 *   orc_dropout(_backward)       the first Philox block's words by hand, the
 *                                keep fraction, out = x mask / (1 - p)
 *   orc_embedding(_backward)     numpy fancy indexing; torch float64 autograd
 *                                with padding_idx and scale_grad_by_freq; the
 *                                one-hot product onehot(idx)^T dy
 *   orc_nll_loss(_backward)      torch float64 nll_loss (weights, ignore_index,
 *                                the three reductions) and its autograd
 *                                gradient; -sum x[i, t_i] by hand
 * NaN semantics of amax/amin/relu against TensorPlay's host kernels, and
 * integer conversions outside the target range, are "parity unpinned": no
 * reference test or fixture fixes them.  So are the NN layers' results for
 * an index or target outside its table (the host kernels raise, the device
 * returns NaN), and dropout's exact random stream: CNNL's Philox stream is
 * closed, so the oracle fixes the published Philox4x32-10 and the tests
 * check the mask's distribution and out = x mask / (1 - p).
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

void orc_layer_norm(int dtype, int64_t rows, int64_t D, const void* x, const void* w,
                    const void* b, double eps, void* y, void* mean, void* rstd);
void orc_layer_norm_backward(int dtype, int64_t rows, int64_t D, const void* dy, const void* x,
                             const void* mean, const void* rstd, const void* w, void* dx,
                             void* dw, void* db);
void orc_philox4x32_10(const uint32_t* ctr, const uint32_t* key, uint32_t* out);
void orc_dropout(int dtype, int64_t n, const void* x, double p, uint64_t seed, uint64_t offset,
                 void* out, uint8_t* mask);
void orc_dropout_backward(int dtype, int64_t n, const void* grad, const uint8_t* mask,
                          double scale, void* out);
void orc_embedding(int dtype, int64_t V, int64_t D, const void* weight, int index_dtype,
                   int64_t n, const void* idx, void* out);
void orc_embedding_backward(int dtype, int64_t n, int64_t D, const void* dy, int index_dtype,
                            const void* idx, int64_t V, int64_t padding_idx,
                            int scale_grad_by_freq, void* out);
void orc_nll_loss(int dtype, int64_t n, int64_t C, const void* x, int index_dtype,
                  const void* target, const void* w, int reduction, int64_t ignore_index,
                  void* y, void* total);
void orc_nll_loss_backward(int dtype, int64_t n, int64_t C, const void* grad, int index_dtype,
                           const void* target, const void* w, int reduction, int64_t ignore_index,
                           const void* total, void* dx);

#endif
