/* Thin kernel-level C-ABI of libtp_amd.so: one entry per device computation
 * the reference delegates to a CNNL call.  These take raw device addresses,
 * sizes and element strides, issue hand-written gfx950 HIP kernels on the
 * device's single stream and return without waiting.  The host-side
 * operator layer (tp_amd_ops.h) is built on these; they are exported so a
 * caller can drive a kernel directly.
 *
 * ``device`` < 0 means the current device.  Every pointer must be device
 * memory of that device (or NULL where stated).  Return codes as in
 * tp_amd_types.h.
 */
#ifndef TP_AMD_KERNELS_H
#define TP_AMD_KERNELS_H

#include "tp_amd_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Binary operations (BinaryKernels.cpp:44-87). */
typedef enum tp_amd_binary_op {
    TP_AMD_BINARY_ADD = 0, /* out = a + alpha * b  (sub passes -alpha, :82) */
    TP_AMD_BINARY_MUL = 1, /* out = a * b          (CNNL_OP_TENSOR_MUL) */
    TP_AMD_BINARY_DIV = 2  /* out = a / b          (CNNL_DIV_TRUE, :60-61) */
} tp_amd_binary_op;

/* Replaces launch_binary's cnnlOpTensor / cnnlDiv_v3 (BinaryKernels.cpp:44-87).
 * out[i] = a[i] op b[i] over the ``ndim``-d index space ``sizes``; each
 * operand has its own element strides (0 for a broadcast dimension, the
 * reference's padded descriptors :49-52).  a, b and out share ``dtype``
 * (float32, float16 or bfloat16); arithmetic is float32, rounded once to
 * ``dtype`` (compute type CNNL_DTYPE_FLOAT, :76).  ``out`` may alias ``a`` or
 * ``b`` element for element (the in-place forms). */
int tp_amd_launch_binary(int device, int op, int dtype, int ndim, const int64_t* sizes,
                         const void* a, const int64_t* a_strides, const void* b,
                         const int64_t* b_strides, void* out, const int64_t* out_strides,
                         float alpha);

/* Replaces affine's cnnlTransform_v2 (BinaryKernels.cpp:30-40): y = alpha * x
 * + beta over ``n`` dense elements, float32 arithmetic, alpha and beta
 * already rounded to float32 by the caller (:113-140, :189-248). */
int tp_amd_launch_affine(int device, int dtype, int64_t n, const void* x, float alpha,
                         float beta, void* y);

/* Unary forward operations (UnaryKernels.cpp:106-214). */
typedef enum tp_amd_unary_op {
    TP_AMD_UNARY_EXP = 0,
    TP_AMD_UNARY_LOG = 1,
    TP_AMD_UNARY_SQRT = 2,
    TP_AMD_UNARY_RSQRT = 3,
    TP_AMD_UNARY_NEG = 4,
    TP_AMD_UNARY_ABS = 5,
    TP_AMD_UNARY_SQUARE = 6,   /* pow(x, 2) (cnnlSquare, :150) */
    TP_AMD_UNARY_POW = 7,      /* pow(x, param) (cnnlPow, :176) */
    TP_AMD_UNARY_RELU = 8,
    TP_AMD_UNARY_SIGMOID = 9,
    TP_AMD_UNARY_TANH = 10,
    TP_AMD_UNARY_SILU = 11,
    TP_AMD_UNARY_GELU = 12,      /* erf form, approximate="none" */
    TP_AMD_UNARY_GELU_TANH = 13, /* tanh form, approximate="tanh" */
    TP_AMD_UNARY_NUM_OPS = 14
} tp_amd_unary_op;

/* Replaces the CNNL unary and activation-forward calls
 * (UnaryKernels.cpp:29-80, 106-214).  y (dense, row-major over ``sizes``) =
 * f(x) with x read through ``x_strides``; float32 arithmetic rounded once to
 * ``dtype``.  ``param`` is the exponent for TP_AMD_UNARY_POW. */
int tp_amd_launch_unary(int device, int op, int dtype, int ndim, const int64_t* sizes,
                        const void* x, const int64_t* x_strides, void* y, float param);

/* Activation backward operations (UnaryKernels.cpp:83-104, 222-287). */
typedef enum tp_amd_backward_op {
    TP_AMD_BACKWARD_THRESHOLD = 0, /* dx = saved > param ? dy : 0, saved = input */
    TP_AMD_BACKWARD_SIGMOID = 1,   /* dx = dy * y * (1 - y), saved = output */
    TP_AMD_BACKWARD_TANH = 2,      /* dx = dy * (1 - y^2), saved = output */
    TP_AMD_BACKWARD_GELU = 3,      /* dx = dy * (Phi(x) + x phi(x)), saved = input */
    TP_AMD_BACKWARD_GELU_TANH = 4, /* derivative of the tanh form, saved = input */
    TP_AMD_BACKWARD_SILU = 5       /* dx = dy * s * (1 + x (1 - s)), saved = input */
} tp_amd_backward_op;

/* Replaces cnnlThresholdBackward (UnaryKernels.cpp:239) and
 * cnnlActivationBackward (:97).  All three arrays dense with ``n`` elements
 * of ``dtype``; ``param`` is the threshold for TP_AMD_BACKWARD_THRESHOLD
 * (already rounded to ``dtype`` by the caller, :229-236). */
int tp_amd_launch_activation_backward(int device, int op, int dtype, int64_t n,
                                      const void* grad, const void* saved, void* dx,
                                      float param);

/* Reductions (ReduceKernels.cpp:21-44, CNNL_REDUCE_ADD/AVG/MAX/MIN). */
typedef enum tp_amd_reduce_op {
    TP_AMD_REDUCE_SUM = 0,
    TP_AMD_REDUCE_MEAN = 1,
    TP_AMD_REDUCE_AMAX = 2,
    TP_AMD_REDUCE_AMIN = 3
} tp_amd_reduce_op;

/* Replaces launch_reduce's cnnlReduce_v2 (ReduceKernels.cpp:21-44).  ``x`` is
 * a dense [outer, r, inner] array of ``dtype``; out[o, i] = reduce over j of
 * x[o, j, i], written dense [outer, inner] in ``dtype``.  float32 arithmetic;
 * NaN inputs are skipped by amax/amin (CNNL_NOT_PROPAGATE_NAN, :33-36) and
 * max(-0, +0) = +0, min(-0, +0) = -0, so the result does not depend on the
 * order of evaluation.  r == 0 gives 0 for sum/mean. */
int tp_amd_launch_reduce(int device, int op, int dtype, int64_t outer, int64_t r,
                         int64_t inner, const void* x, void* out);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The same reduction as tp_amd_launch_reduce, with the
 * same kernels and bit-identical results, but the float32 partials of a split
 * reduction live in a static device array of
 * tp_amd_reduce_noalloc_scratch_bytes() bytes per GPU (1 MiB, held until the
 * process ends) instead of coming from the caching allocator; nothing is
 * allocated or freed.  A reduction that would need more partials than that
 * returns TP_AMD_ERROR.  Every call on one GPU shares that GPU's array, so
 * calls that overlap on one device (other streams, other processes' copies
 * aside) race; calls on the library's single stream are ordered and safe. */
int tp_amd_launch_reduce_noalloc(int device, int op, int dtype, int64_t outer, int64_t r,
                                 int64_t inner, const void* x, void* out);

/* Size in bytes of the static partials array of tp_amd_launch_reduce_noalloc. */
size_t tp_amd_reduce_noalloc_scratch_bytes(void);

/* No counterpart in the reference: a planning query for callers of
 * tp_amd_launch_reduce_noalloc.  The bytes of float32 partials that a
 * reduction of dense [outer, r, inner] ``dtype`` with a 16-byte aligned input
 * uses on a GPU with ``compute_units`` CUs (0 when it runs without partials;
 * -1 for an unknown dtype or a negative extent).  The allocation-free entry
 * refuses the shapes whose figure exceeds tp_amd_reduce_noalloc_scratch_bytes();
 * pure host arithmetic, no GPU needed. */
int64_t tp_amd_reduce_partial_bytes(int compute_units, int dtype, int64_t outer, int64_t r,
                                    int64_t inner);

/* Replaces cnnlSoftmaxForward (ReduceKernels.cpp:171-183): x, y dense
 * [outer, dim, inner] of ``dtype``; softmax (log_softmax when ``log``) along
 * the middle axis, float32 arithmetic. */
int tp_amd_launch_softmax(int device, int log, int dtype, int64_t outer, int64_t dim,
                          int64_t inner, const void* x, void* y);

/* Replaces cnnlSoftmaxBackward (ReduceKernels.cpp:185-199): from the forward
 * output y and the upstream gradient dy, dx = y * (dy - sum(dy * y)) for
 * softmax, dx = dy - exp(y) * sum(dy) for log_softmax (sums along the
 * middle axis).  All dense [outer, dim, inner] of ``dtype``. */
int tp_amd_launch_softmax_backward(int device, int log, int dtype, int64_t outer,
                                   int64_t dim, int64_t inner, const void* y,
                                   const void* dy, void* dx);

/* Replaces cnnlMatMul_v2 / cnnlStrideBatchMatMul_v3 (BlasKernels.cpp:202-242).
 * For each of ``batch`` problems:
 *   C[b] (M x N, row stride ldc) = alpha * op(A[b]) op(B[b]) + beta * Cin[b]
 * op(A) is M x K: A stored row-major M x K (lda >= K) or, when trans_a, the
 * transpose of a row-major K x M matrix (lda >= M) -- read in place, never
 * copied (as_operand, :38-54).  op(B) likewise K x N from a row-major K x N
 * (ldb >= N) or, when trans_b, a row-major N x K (ldb >= K).  Batch strides
 * are in elements; 0 repeats one matrix for every batch (:221-222).  ``cin``
 * (may be NULL when beta == 0, may equal ``c``) is read at
 * cin[b * cin_stride_b + i * cin_rs + j * cin_cs], so a bias row broadcast
 * over M is cin_rs = 0, cin_cs = 1.  dtype float32, float16 or bfloat16;
 * accumulation in float32 (CNNL_DTYPE_FLOAT compute, :113,159), result
 * rounded once to ``dtype``; float32 inputs are multiplied in full float32
 * (no reduced-precision mode; gfx950 has no TF32 matrix instruction). */
int tp_amd_launch_gemm(int device, int dtype, int64_t batch, int64_t m, int64_t n,
                       int64_t k, float alpha, const void* a, int64_t lda, int64_t stride_a,
                       int trans_a, const void* b, int64_t ldb, int64_t stride_b, int trans_b,
                       float beta, const void* cin, int64_t cin_rs, int64_t cin_cs,
                       int64_t cin_stride_b, void* c, int64_t ldc, int64_t stride_c);

/* Replaces cnnlCastDataType (CopyKernels.cpp:125-139): ``n`` dense elements
 * converted from ``src_dtype`` to ``dst_dtype``.  Float to narrower float
 * rounds to nearest even (NaN stays NaN, overflow gives infinity); float to
 * integer truncates toward zero; anything to bool is (x != 0); integer to
 * float rounds to nearest even.  Any pair of the ten dtypes is accepted. */
int tp_amd_launch_cast(int device, int src_dtype, int dst_dtype, int64_t n, const void* src,
                       void* dst);

/* Replaces cnnlFill_v3 (CopyKernels.cpp:266-299): every element of the
 * strided view (sizes/strides over ``ndim`` dims) set to the ``elem_size``
 * bytes at ``value`` (1, 2, 4 or 8 bytes; the caller encodes the value per
 * dtype, :272-283). */
int tp_amd_launch_fill(int device, int elem_size, const void* value, int ndim,
                       const int64_t* sizes, void* dst, const int64_t* dst_strides);

/* Replaces strided_copy's cnnlCopy_v2 / memcpy fast path
 * (Cnnl.cpp:127-176): dst[idx] = src[idx] over ``sizes`` for elements of
 * ``elem_size`` bytes, each side with its own strides (src strides may be 0
 * for an expanded view).  Dimensions laid out back to back in both are
 * merged first; a dense-to-dense copy is one device memcpy. */
int tp_amd_launch_strided_copy(int device, int elem_size, int ndim, const int64_t* sizes,
                               void* dst, const int64_t* dst_strides, const void* src,
                               const int64_t* src_strides);

/* ---- neural-network layers (NNKernels.cpp:57-395) ------------------------ */

/* Replaces cnnlLayerNormForward (NNKernels.cpp:88-94): x dense [rows, dim] of
 * ``dtype``; per row mean = sum(x) / dim, var = sum((x - mean)^2) / dim (the
 * biased variance), rstd = 1 / sqrt(var + eps), and
 * y = (x - mean) * rstd * weight + bias.  ``weight`` / ``bias`` ([dim] of
 * ``dtype``) may be NULL for 1 / 0.  mean and rstd ([rows]) are float32 for
 * every dtype (stats_dtype, :52-54); float32 arithmetic. */
int tp_amd_launch_layer_norm(int device, int dtype, int64_t rows, int64_t dim, const void* x,
                             const void* weight, const void* bias, double eps, void* y,
                             float* mean, float* rstd);

/* Replaces cnnlLayerNormBackward_v2 (NNKernels.cpp:139-143): from the
 * forward's input x, its float32 mean and rstd, and grad_out, with
 * xhat = (x - mean) * rstd and g = grad_out * weight,
 *   dx      = rstd * (g - mean_row(g) - xhat * mean_row(g * xhat)),
 *   dweight = sum over rows of grad_out * xhat,
 *   dbias   = sum over rows of grad_out.
 * Any of dx, dweight, dbias may be NULL (not computed); ``weight`` may be
 * NULL for 1.  rows == 0 gives zero parameter gradients. */
int tp_amd_launch_layer_norm_backward(int device, int dtype, int64_t rows, int64_t dim,
                                      const void* grad_out, const void* x, const float* mean,
                                      const float* rstd, const void* weight, void* dx,
                                      void* dweight, void* dbias);

/* Replaces cnnlFusedDropout_v3 (NNKernels.cpp:184-186): element e of the
 * dense ``x`` is kept when the uniform (w >> 8) * 2^-24 is >= p, w being word
 * e % 4 of Philox4x32-10 (Salmon et al., SC 2011) on the counter
 * (e / 4 low, e / 4 high, offset low, offset high) under the key (seed low,
 * seed high).  out = keep ? x / (1 - p) : 0 (the scale rounded to float32),
 * mask = keep (one byte, 0 or 1).  0 <= p < 1. */
int tp_amd_launch_dropout(int device, int dtype, int64_t n, const void* x, double p,
                          uint64_t seed, uint64_t offset, void* out, uint8_t* mask);

/* Replaces scaled_product's cnnlOpTensor (NNKernels.cpp:196-220): out = grad *
 * mask * scale over n dense elements, mask bytes 0 / 1. */
int tp_amd_launch_dropout_backward(int device, int dtype, int64_t n, const void* grad,
                                   const uint8_t* mask, double scale, void* out);

/* Replaces cnnlEmbeddingForward_v2 (NNKernels.cpp:254-256): out[i, :] =
 * weight[indices[i], :] for the n indices (``index_dtype`` int32 or int64);
 * weight dense [num_weights, dim].  An index outside [0, num_weights) writes
 * a row of NaN and reads nothing. */
int tp_amd_launch_embedding(int device, int dtype, int64_t num_weights, int64_t dim,
                            const void* weight, int index_dtype, int64_t n, const void* indices,
                            void* out);

/* Replaces cnnlEmbeddingBackward (NNKernels.cpp:283-286): out dense
 * [num_weights, dim] = sum over i with indices[i] == r of grad[i, :]
 * (divided by the number of such i when scale_grad_by_freq).  Indices equal
 * to padding_idx, or outside [0, num_weights), add nothing, so the
 * padding row is zero.  Accumulated in float32 with atomics (the order of
 * the additions is not fixed). */
int tp_amd_launch_embedding_backward(int device, int dtype, int64_t n, int64_t dim,
                                     const void* grad, int index_dtype, const void* indices,
                                     int64_t num_weights, int64_t padding_idx,
                                     int scale_grad_by_freq, void* out);

/* Replaces cnnlNlllossForward (NNKernels.cpp:350-353): x dense [n, classes],
 * per sample loss_i = -weight[t_i] * x[i, t_i] and weight w_i = weight[t_i]
 * (weight NULL: 1); a target equal to ignore_index gives 0 and 0, one
 * outside [0, classes) NaN and NaN.  reduction 0 writes y[i] = loss_i (and
 * leaves total_weight alone); 1 (mean) writes y = sum loss / sum w; 2 (sum)
 * y = sum loss; both write total_weight = sum w.  Sums in a fixed order. */
int tp_amd_launch_nll_loss(int device, int dtype, int64_t n, int64_t classes, const void* x,
                           int index_dtype, const void* target, const void* weight,
                           int reduction, int64_t ignore_index, void* y, void* total_weight);

/* Replaces cnnlNlllossBackward (NNKernels.cpp:385-388): dx dense [n, classes]
 * is zero except dx[i, t_i] = -weight[t_i] * g_i, with g_i = grad[i]
 * (reduction 0), grad[0] / total_weight[0] (1) or grad[0] (2); rows whose
 * target is ignore_index stay zero, rows whose target is outside
 * [0, classes) are NaN. */
int tp_amd_launch_nll_loss_backward(int device, int dtype, int64_t n, int64_t classes,
                                    const void* grad, int index_dtype, const void* target,
                                    const void* weight, int reduction, int64_t ignore_index,
                                    const void* total_weight, void* dx);

#ifdef __cplusplus
}
#endif

#endif /* TP_AMD_KERNELS_H */
