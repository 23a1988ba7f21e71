/* Operator-level C-ABI of libtp_amd.so: one entry per TensorPlay operator
 * the reference registers for the PrivateUse1 hot path (64 registrations:
 * CopyKernels.cpp:349-364, BinaryKernels.cpp:252-269,
 * UnaryKernels.cpp:291-310, BlasKernels.cpp:416-422,
 * ReduceKernels.cpp:267-282).  Each keeps the reference operator's argument
 * meaning, dtype rules and decline conditions; the TensorPlay adapter
 * (csrc/tensorplay/ in the package) turns TensorPlay tensors into tp_amd_tensor views,
 * calls these, and runs the host fallback on TP_AMD_DECLINED.
 *
 * Results: an entry that returns a new tensor writes it to ``*result`` --
 * device memory from the caching allocator, dense row-major, with
 * ``result->ctx`` set; the caller owns it and releases it with tp_amd_free.
 * ``result->ctx == NULL`` on success means the result is a view of an input
 * (contiguous() of a contiguous tensor).  In-place entries (trailing ``_``)
 * write into ``self``.  A host 0-d tensor (device -1, ndim 0) is accepted
 * where the reference accepts one (binary operands, BinaryKernels.cpp:20-22).
 */
#ifndef TP_AMD_OPS_H
#define TP_AMD_OPS_H

#include "tp_amd_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- factories, copies, casts, fills (CopyKernels.cpp:231-345) ---------- */

/* empty / empty.memory_format (:231-246): dtype TP_AMD_UNDEFINED means
 * float32; device < 0 means current; pin_memory != 0 is an error (:233). */
int tp_amd_empty(const int64_t* sizes, int ndim, int dtype, int device, int pin_memory,
                 tp_amd_tensor* result);
/* empty_like / zeros_like / ones_like / full_like (:322-345): dtype
 * TP_AMD_UNDEFINED keeps self's; device < 0 keeps self's. */
int tp_amd_empty_like(const tp_amd_tensor* self, int dtype, int device, tp_amd_tensor* result);
int tp_amd_zeros_like(const tp_amd_tensor* self, int dtype, int device, tp_amd_tensor* result);
int tp_amd_ones_like(const tp_amd_tensor* self, int dtype, int device, tp_amd_tensor* result);
int tp_amd_full_like(const tp_amd_tensor* self, tp_amd_scalar value, int dtype, int device,
                     tp_amd_tensor* result);
/* item / _local_scalar_dense (:340-345): the single element, read back. */
int tp_amd_item(const tp_amd_tensor* self, tp_amd_scalar* value);
/* copy_ (:248-264): either side may be host memory (device -1); src is
 * broadcast to self's shape and converted to self's dtype. */
int tp_amd_copy_(tp_amd_tensor* self, const tp_amd_tensor* src, int non_blocking);
/* fill_.Scalar / zero_ (:266-301): value encoded per dtype. */
int tp_amd_fill_(tp_amd_tensor* self, tp_amd_scalar value);
int tp_amd_zero_(tp_amd_tensor* self);
/* clone / contiguous (:303-320). */
int tp_amd_clone(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_contiguous(const tp_amd_tensor* self, tp_amd_tensor* result);
/* to_dtype (Cnnl.h:71-73, CopyKernels.cpp:222-227): a converted copy. */
int tp_amd_to_dtype(const tp_amd_tensor* self, int dtype, tp_amd_tensor* result);

/* ---- binary arithmetic (BinaryKernels.cpp:92-248) ----------------------- */

/* add.Tensor / sub.Tensor: self +/- alpha * other; mul.Tensor; div.Tensor
 * (:148-166).  Broadcasting, dtype promotion where a 0-d operand does not
 * widen a dimensioned one (Cnnl.cpp:178-192), a host 0-d operand folded into
 * an affine transform (:113-140).  Declined unless the result dtype is
 * float32, float16 or bfloat16. */
int tp_amd_add(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha,
               tp_amd_tensor* result);
int tp_amd_sub(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha,
               tp_amd_tensor* result);
int tp_amd_mul(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result);
int tp_amd_div(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result);
/* add_ / sub_ / mul_ / div_ .Tensor (:168-186): declined unless the result
 * has self's shape and dtype. */
int tp_amd_add_(tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha);
int tp_amd_sub_(tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_scalar alpha);
int tp_amd_mul_(tp_amd_tensor* self, const tp_amd_tensor* other);
int tp_amd_div_(tp_amd_tensor* self, const tp_amd_tensor* other);
/* Scalar forms (:189-248): one affine y = a * x + b with a, b computed in
 * double then rounded to float; division multiplies by 1/s. */
int tp_amd_add_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                      tp_amd_tensor* result);
int tp_amd_sub_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                      tp_amd_tensor* result);
int tp_amd_rsub_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha,
                       tp_amd_tensor* result);
int tp_amd_mul_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_tensor* result);
int tp_amd_div_scalar(const tp_amd_tensor* self, tp_amd_scalar other, tp_amd_tensor* result);
int tp_amd_add__scalar(tp_amd_tensor* self, tp_amd_scalar other, tp_amd_scalar alpha);
int tp_amd_mul__scalar(tp_amd_tensor* self, tp_amd_scalar other);
int tp_amd_div__scalar(tp_amd_tensor* self, tp_amd_scalar other);

/* ---- unary and activations (UnaryKernels.cpp:106-287) ------------------- */

/* Result dense in self's dtype; declined for non-float dtypes. */
int tp_amd_exp(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_log(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_sqrt(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_rsqrt(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_neg(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_abs(const tp_amd_tensor* self, tp_amd_tensor* result);
/* pow.Tensor_Scalar (:140-186): exponent 1 clones, 0 gives ones, 2 squares,
 * 0.5 and -0.5 take sqrt / rsqrt, any other value the general power. */
int tp_amd_pow_scalar(const tp_amd_tensor* self, tp_amd_scalar exponent, tp_amd_tensor* result);
int tp_amd_relu(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_relu_(tp_amd_tensor* self);
int tp_amd_sigmoid(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_tanh(const tp_amd_tensor* self, tp_amd_tensor* result);
int tp_amd_silu(const tp_amd_tensor* self, tp_amd_tensor* result);
/* gelu (:203-210): approximate 0 = "none" (erf form), 1 = "tanh". */
int tp_amd_gelu(const tp_amd_tensor* self, int approximate, tp_amd_tensor* result);
/* Backward kernels (:222-287): both operands must agree in dtype and shape
 * (:217-220). */
int tp_amd_threshold_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                              tp_amd_scalar threshold, tp_amd_tensor* result);
int tp_amd_sigmoid_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* output,
                            tp_amd_tensor* result);
int tp_amd_tanh_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* output,
                         tp_amd_tensor* result);
int tp_amd_gelu_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                         int approximate, tp_amd_tensor* result);
int tp_amd_silu_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                         tp_amd_tensor* result);

/* ---- matrix products (BlasKernels.cpp:261-412) -------------------------- */

/* mm [M,K] x [K,N] and bmm [B,M,K] x [B,K,N] (:261-304); K == 0 gives zeros.
 * Transposed views of row-major matrices are read in place. */
int tp_amd_mm(const tp_amd_tensor* self, const tp_amd_tensor* mat2, tp_amd_tensor* result);
int tp_amd_bmm(const tp_amd_tensor* self, const tp_amd_tensor* mat2, tp_amd_tensor* result);
/* addmm (:306-334): beta * self (broadcast to [M,N]) + alpha * mat1 @ mat2. */
int tp_amd_addmm(const tp_amd_tensor* self, const tp_amd_tensor* mat1, const tp_amd_tensor* mat2,
                 tp_amd_scalar beta, tp_amd_scalar alpha, tp_amd_tensor* result);
/* linear (:338-356): input [..., K] @ weight[N, K]^T (+ bias[N]); bias may
 * be NULL. */
int tp_amd_linear(const tp_amd_tensor* input, const tp_amd_tensor* weight,
                  const tp_amd_tensor* bias, tp_amd_tensor* result);
/* matmul (:360-412): 1-d/2-d to mm, [...,M,K] @ [K,N] folded into rows,
 * otherwise the batch dimensions broadcast into one bmm. */
int tp_amd_matmul(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result);

/* ---- reductions and softmax (ReduceKernels.cpp:47-263) ------------------ */

/* sum / mean over all dims (:97-103, 130-136); dtype TP_AMD_UNDEFINED keeps
 * self's; the input is converted to the result dtype first (:51). */
int tp_amd_sum(const tp_amd_tensor* self, int dtype, tp_amd_tensor* result);
int tp_amd_mean(const tp_amd_tensor* self, int dtype, tp_amd_tensor* result);
/* sum.dim_IntList / mean.dim / amax / amin (:105-144): ``dims`` (ndims
 * entries, negative counts from the end; none = all) reduced, kept as size 1
 * when keepdim. */
int tp_amd_sum_dim(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                   int dtype, tp_amd_tensor* result);
int tp_amd_mean_dim(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                    int dtype, tp_amd_tensor* result);
int tp_amd_amax(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                tp_amd_tensor* result);
int tp_amd_amin(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                tp_amd_tensor* result);
/* softmax / log_softmax with an optional result dtype (:201-222). */
int tp_amd_softmax(const tp_amd_tensor* self, int64_t dim, int dtype, tp_amd_tensor* result);
int tp_amd_log_softmax(const tp_amd_tensor* self, int64_t dim, int dtype,
                       tp_amd_tensor* result);
/* _softmax / _log_softmax (:224-240): half_to_float is declined (:202). */
int tp_amd__softmax(const tp_amd_tensor* self, int64_t dim, int half_to_float,
                    tp_amd_tensor* result);
int tp_amd__log_softmax(const tp_amd_tensor* self, int64_t dim, int half_to_float,
                        tp_amd_tensor* result);
/* _softmax_backward_data / _log_softmax_backward_data (:244-263): declined
 * unless grad, output and input_dtype agree (:246-247). */
int tp_amd__softmax_backward_data(const tp_amd_tensor* grad_output, const tp_amd_tensor* output,
                                  int64_t dim, int input_dtype, tp_amd_tensor* result);
int tp_amd__log_softmax_backward_data(const tp_amd_tensor* grad_output,
                                      const tp_amd_tensor* output, int64_t dim,
                                      int input_dtype, tp_amd_tensor* result);

/* ---- neural-network layers (NNKernels.cpp:57-395) ---------------------- */
/* An output the caller masks off comes back with data == NULL and dtype
 * TP_AMD_UNDEFINED.  Each entry declines where the reference falls back to
 * the host. */

/* native_layer_norm (:57-104): normalizes over the trailing dims
 * ``normalized_shape`` (nnorm entries); weight / bias may be NULL.  Results
 * y (input's shape and dtype) and float32 mean / rstd of shape [outer].
 * Declined unless the input is a native float on the device, at least one
 * leading dim remains, and weight / bias match its device and dtype. */
int tp_amd_native_layer_norm(const tp_amd_tensor* input, const int64_t* normalized_shape, int nnorm,
                             const tp_amd_tensor* weight, const tp_amd_tensor* bias, double eps,
                             tp_amd_tensor* y, tp_amd_tensor* mean, tp_amd_tensor* rstd);
/* native_layer_norm_backward (:106-159): output_mask (3 ints; NULL = all)
 * selects dx, dweight, dbias. */
int tp_amd_native_layer_norm_backward(const tp_amd_tensor* grad_out, const tp_amd_tensor* input,
                                      const int64_t* normalized_shape, int nnorm,
                                      const tp_amd_tensor* mean, const tp_amd_tensor* rstd,
                                      const tp_amd_tensor* weight, const tp_amd_tensor* bias,
                                      const int* output_mask, tp_amd_tensor* dx,
                                      tp_amd_tensor* dweight, tp_amd_tensor* dbias);
/* native_dropout (:163-191): train -1 (unset, i.e. training), 0 or 1; the
 * random stream is keyed by ``seed`` (the reference draws it from the host
 * generator, :181-183).  Results out (input's dtype) and a bool mask.  Not
 * training: a copy and an all-true mask; p == 1: zeros and an all-false
 * mask. */
int tp_amd_native_dropout(const tp_amd_tensor* input, double p, int train, uint64_t seed,
                          tp_amd_tensor* out, tp_amd_tensor* mask);
/* native_dropout_backward (:222-234): grad_output * mask * scale; the mask
 * bool or uint8. */
int tp_amd_native_dropout_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* mask,
                                   double scale, tp_amd_tensor* result);
/* embedding (:242-263): weight [V, D], int32 / int64 indices of any shape;
 * result [indices..., D].  sparse is declined. */
int tp_amd_embedding(const tp_amd_tensor* weight, const tp_amd_tensor* indices, int64_t padding_idx,
                     int scale_grad_by_freq, int sparse, tp_amd_tensor* result);
/* embedding_dense_backward (:265-296): result [num_weights, D]. */
int tp_amd_embedding_dense_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* indices,
                                    int64_t num_weights, int64_t padding_idx, int scale_grad_by_freq,
                                    tp_amd_tensor* result);
/* nll_loss (:327-364): self [N, C], target [N] int32 / int64, weight [C] or
 * NULL, reduction 0 none / 1 mean / 2 sum.  Results output ([N] or 0-d) and
 * a 0-d total_weight (0 for reduction none). */
int tp_amd_nll_loss(const tp_amd_tensor* self, const tp_amd_tensor* target, const tp_amd_tensor* weight,
                    int64_t reduction, int64_t ignore_index, tp_amd_tensor* output,
                    tp_amd_tensor* total_weight);
/* nll_loss_backward (:366-395): result [N, C]. */
int tp_amd_nll_loss_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                             const tp_amd_tensor* target, const tp_amd_tensor* weight, int64_t reduction,
                             int64_t ignore_index, const tp_amd_tensor* total_weight,
                             tp_amd_tensor* result);

/* ---- host-only helpers (Cnnl.cpp:107-205); no device work --------------- */

/* binary_result_dtype (Cnnl.cpp:178-192) for two tensors' dtypes and
 * dimensionality; returns the dtype code. */
int tp_amd_binary_result_dtype(int a_dtype, int a_ndim, int b_dtype, int b_ndim);
/* broadcast_shape (Cnnl.cpp:194-205): writes the broadcast sizes to ``out``
 * (capacity TP_AMD_MAX_DIMS) and their count to ``out_ndim``; TP_AMD_ERROR
 * when the shapes cannot be broadcast. */
int tp_amd_broadcast_shape(const int64_t* a, int a_ndim, const int64_t* b, int b_ndim,
                           int64_t* out, int* out_ndim);
/* is_dense (Cnnl.cpp:107-121): 1 when the view's elements are packed
 * without gaps in some order of its dimensions. */
int tp_amd_is_dense(const tp_amd_tensor* t);
/* is_native_float (Cnnl.h:24-27): 1 for float32, float16, bfloat16. */
int tp_amd_is_native_float(int dtype);
/* Size in bytes of one element of ``dtype`` (0 for an unknown code). */
int tp_amd_element_size(int dtype);

#ifdef __cplusplus
}
#endif

#endif /* TP_AMD_OPS_H */
