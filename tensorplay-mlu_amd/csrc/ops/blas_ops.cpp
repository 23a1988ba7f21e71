// Matrix products: the C entry points for the reference's 5 BLAS
// registrations (tensorplay_mlu/csrc/BlasKernels.cpp:32-422): mm, bmm,
// addmm, linear, matmul, over the gfx950 GEMM kernels.  A transposed view of
// a row-major matrix is read in place (as_operand, :38-54); addmm's bias is
// read by the GEMM epilogue directly instead of being copied into the output
// first (:318-324) -- the same beta * bias + alpha * product.

#include <numeric>

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

// A matrix operand as the GEMM reads it: the stored row-major matrix, its
// leading dimension, batch stride, and whether the product reads it
// transposed (Operand / as_operand, :32-54).
struct Operand {
    MaybeOwned storage;
    bool transposed = false;
    int64_t ld = 0;
    int64_t batch_stride = 0;
};

Operand as_operand(const TensorRef& t) {
    const int nd = t.ndim;
    const int64_t r = t.sizes[nd - 2], c = t.sizes[nd - 1];
    const int64_t s_r = t.strides[nd - 2], s_c = t.strides[nd - 1];
    const bool batch_ok = nd == 2 || t.strides[0] == r * c || t.sizes[0] == 1;
    const int64_t bstride = nd == 3 && t.sizes[0] > 1 ? r * c : 0;
    Operand op;
    if (batch_ok && (s_c == 1 || c == 1) && (s_r == c || r == 1)) {
        op.storage.ref = t;
        op.storage.ref.ctx = nullptr;
        op.transposed = false;
        op.ld = c;
        op.batch_stride = bstride;
        return op;
    }
    if (batch_ok && (s_r == 1 || r == 1) && (s_c == r || c == 1)) {
        op.storage.ref = t;
        op.storage.ref.ctx = nullptr;
        op.transposed = true;
        op.ld = r;
        op.batch_stride = bstride;
        return op;
    }
    op.storage = contiguous_on_device(t);
    op.transposed = false;
    op.ld = c;
    op.batch_stride = bstride;
    return op;
}

// out (dense [.., M, N]) = alpha * a @ b + beta * cin (gemm, :202-242).
// ``cin`` null means beta is 0.
void gemm(const TensorRef& a, const TensorRef& b, const TensorRef& out, float alpha, float beta,
          const TensorRef* cin) {
    Operand oa = as_operand(a), ob = as_operand(b);
    const bool batched = out.ndim == 3;
    const int64_t B = batched ? out.sizes[0] : 1;
    const int64_t M = out.sizes[out.ndim - 2], N = out.sizes[out.ndim - 1];
    const int64_t K = a.sizes[a.ndim - 1];
    const void* cptr = nullptr;
    int64_t crs = 0, ccs = 0, csb = 0;
    if (cin != nullptr && beta != 0.0f) {
        cptr = cin->data;
        crs = cin->strides[cin->ndim - 2];
        ccs = cin->strides[cin->ndim - 1];
        csb = cin->ndim == 3 ? cin->strides[0] : 0;
    } else {
        beta = 0.0f;
    }
    const int st = tp_amd_launch_gemm(out.device, out.dtype, B, M, N, K, alpha,
                                      oa.storage.ref.data, oa.ld, oa.batch_stride,
                                      oa.transposed ? 1 : 0, ob.storage.ref.data, ob.ld,
                                      ob.batch_stride, ob.transposed ? 1 : 0, beta, cptr, crs, ccs,
                                      csb, out.data, N, batched ? M * N : 0);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
}

bool native_pair(const TensorRef& a, const TensorRef& b) {
    return on_device(a) && on_device(b) && is_native_float(a.dtype) && a.dtype == b.dtype &&
           a.device == b.device;
}

// A dense tensor's memory under a new contiguous shape (reshape_dense,
// :251-259): a contiguous copy first when needed.
MaybeOwned reshape_dense(const TensorRef& t, const Sizes& sizes) {
    MaybeOwned c = contiguous_on_device(t);
    c.ref = make_view(c.ref, sizes, contiguous_strides(sizes));
    if (c.hold.ref().ctx != nullptr) c.ref.ctx = nullptr;
    return c;
}

void zero(const TensorRef& t) { fill(t, scalar_of(0.0)); }

Owned mm_native(const TensorRef& a, const TensorRef& b) {
    const int64_t M = a.sizes[0], N = b.sizes[1];
    Owned out = empty_on({M, N}, a.dtype, a.device);
    if (numel(out.ref()) == 0) return out;
    if (a.sizes[1] == 0) {
        zero(out.ref());
        return out;
    }
    gemm(a, b, out.ref(), 1.0f, 0.0f, nullptr);
    return out;
}

Owned bmm_native(const TensorRef& a, const TensorRef& b) {
    const int64_t B = a.sizes[0], M = a.sizes[1], N = b.sizes[2];
    Owned out = empty_on({B, M, N}, a.dtype, a.device);
    if (numel(out.ref()) == 0) return out;
    if (a.sizes[2] == 0) {
        zero(out.ref());
        return out;
    }
    gemm(a, b, out.ref(), 1.0f, 0.0f, nullptr);
    return out;
}

Owned mm_op(const TensorRef& self, const TensorRef& mat2) {
    check_view(self, "self");
    check_view(mat2, "mat2");
    if (!native_pair(self, mat2) || self.ndim != 2 || mat2.ndim != 2) {
        TP_AMD_DECLINE("mm operands have no device kernel");
    }
    TP_AMD_CHECK(self.sizes[1] == mat2.sizes[0], "mm: shapes ", self.sizes[0], "x",
                 self.sizes[1], " and ", mat2.sizes[0], "x", mat2.sizes[1],
                 " cannot be multiplied");
    return mm_native(self, mat2);
}

Owned bmm_op(const TensorRef& self, const TensorRef& mat2) {
    check_view(self, "self");
    check_view(mat2, "mat2");
    if (!native_pair(self, mat2) || self.ndim != 3 || mat2.ndim != 3) {
        TP_AMD_DECLINE("bmm operands have no device kernel");
    }
    TP_AMD_CHECK(self.sizes[0] == mat2.sizes[0] && self.sizes[2] == mat2.sizes[1],
                 "bmm: batch or inner dimensions do not match");
    return bmm_native(self, mat2);
}

// beta * self + alpha * mat1 @ mat2 (addmm_kernel, :306-334).
Owned addmm_op(const TensorRef& self, const TensorRef& mat1, const TensorRef& mat2, double beta,
               double alpha) {
    check_view(self, "self");
    check_view(mat1, "mat1");
    check_view(mat2, "mat2");
    if (!native_pair(mat1, mat2) || mat1.ndim != 2 || mat2.ndim != 2 || !on_device(self) ||
        self.dtype != mat1.dtype || self.device != mat1.device) {
        TP_AMD_DECLINE("addmm operands have no device kernel");
    }
    TP_AMD_CHECK(mat1.sizes[1] == mat2.sizes[0], "addmm: shapes cannot be multiplied");
    const int64_t M = mat1.sizes[0], N = mat2.sizes[1];
    Owned out = empty_on({M, N}, mat1.dtype, mat1.device);
    if (numel(out.ref()) == 0) return out;
    const float b = static_cast<float>(beta), a = static_cast<float>(alpha);
    const TensorRef bias = expand_to(self, {M, N});
    if (mat1.sizes[1] == 0) {
        if (b == 0.0f) {
            zero(out.ref());
        } else {
            strided_copy(out.ref(), bias);
            if (b != 1.0f) {
                const int st = tp_amd_launch_affine(out.ref().device, out.ref().dtype,
                                                    numel(out.ref()), out.ref().data, b, 0.0f,
                                                    out.ref().data);
                TP_AMD_CHECK(st == TP_AMD_OK, last_error());
            }
        }
        return out;
    }
    gemm(mat1, mat2, out.ref(), a, b, b != 0.0f ? &bias : nullptr);
    return out;
}

TensorRef transpose2d(const TensorRef& t) {
    return make_view(t, {t.sizes[1], t.sizes[0]}, {t.strides[1], t.strides[0]});
}

// input [..., K] @ weight [N, K].t() (+ bias [N]) (linear_kernel, :338-356).
Owned linear_op(const TensorRef& input, const TensorRef& weight, const TensorRef* bias) {
    check_view(input, "input");
    check_view(weight, "weight");
    const bool has_bias = bias != nullptr;
    if (has_bias) check_view(*bias, "bias");
    if (!native_pair(input, weight) || input.ndim == 0 || weight.ndim != 2 ||
        (has_bias && (!on_device(*bias) || bias->dtype != input.dtype))) {
        TP_AMD_DECLINE("linear operands have no device kernel");
    }
    const int64_t K = weight.sizes[1], N = weight.sizes[0];
    TP_AMD_CHECK(input.sizes[input.ndim - 1] == K, "linear: mat1 and mat2 shapes cannot be "
                 "multiplied (", input.sizes[input.ndim - 1], " and ", K, ")");
    const int64_t rows = numel(input) / std::max<int64_t>(K, 1);
    MaybeOwned in2 = reshape_dense(input, {rows, K});
    const TensorRef wt = transpose2d(weight);
    Owned out = has_bias ? addmm_op(*bias, in2.ref, wt, 1.0, 1.0) : mm_op(in2.ref, wt);
    Sizes shape = sizes_of(input);
    shape.back() = N;
    TensorRef view = make_view(out.ref(), shape, contiguous_strides(shape));
    view.ctx = out.ref().ctx;
    out.release();
    return Owned(view);
}

Owned with_shape(Owned t, const Sizes& shape) {
    TensorRef view = make_view(t.ref(), shape, contiguous_strides(shape));
    view.ctx = t.ref().ctx;
    t.release();
    return Owned(view);
}

// matmul over broadcast batch dimensions (matmul_kernel, :360-412).
Owned matmul_op(const TensorRef& self, const TensorRef& other) {
    check_view(self, "self");
    check_view(other, "other");
    if (!native_pair(self, other) || self.ndim == 0 || other.ndim == 0) {
        TP_AMD_DECLINE("matmul operands have no device kernel");
    }
    const int da = self.ndim, db = other.ndim;
    if (da <= 2 && db <= 2) {
        MaybeOwned a = da == 1 ? reshape_dense(self, {1, self.sizes[0]}) : MaybeOwned{self, Owned()};
        MaybeOwned b = db == 1 ? reshape_dense(other, {other.sizes[0], 1}) : MaybeOwned{other, Owned()};
        if (da != 1) a.ref.ctx = nullptr;
        if (db != 1) b.ref.ctx = nullptr;
        TP_AMD_CHECK(a.ref.sizes[1] == b.ref.sizes[0], "matmul: inner dimensions do not match");
        Owned out = mm_native(a.ref, b.ref);
        Sizes shape;
        if (da == 2) shape.push_back(a.ref.sizes[0]);
        if (db == 2) shape.push_back(b.ref.sizes[1]);
        return with_shape(std::move(out), shape);
    }
    if (db <= 2 && da >= 3) {
        // [..., M, K] @ [K, N]: fold the batch into the rows.
        const int64_t K = self.sizes[da - 1];
        const int64_t rows = numel(self) / std::max<int64_t>(K, 1);
        MaybeOwned b = db == 1 ? reshape_dense(other, {other.sizes[0], 1}) : MaybeOwned{other, Owned()};
        if (db != 1) b.ref.ctx = nullptr;
        TP_AMD_CHECK(b.ref.sizes[0] == K, "matmul: inner dimensions do not match");
        MaybeOwned a = reshape_dense(self, {rows, K});
        Owned out = mm_native(a.ref, b.ref);
        Sizes shape(self.sizes, self.sizes + da - 1);
        if (db == 2) shape.push_back(b.ref.sizes[1]);
        return with_shape(std::move(out), shape);
    }
    // General case: broadcast the batch dimensions, then one bmm.
    MaybeOwned a = da == 1 ? reshape_dense(self, {1, self.sizes[0]}) : MaybeOwned{self, Owned()};
    MaybeOwned b = db == 1 ? reshape_dense(other, {other.sizes[0], 1}) : MaybeOwned{other, Owned()};
    if (da != 1) a.ref.ctx = nullptr;
    if (db != 1) b.ref.ctx = nullptr;
    const Sizes sa = sizes_of(a.ref), sb = sizes_of(b.ref);
    const int64_t M = sa[sa.size() - 2], K = sa.back(), N = sb.back();
    TP_AMD_CHECK(sb[sb.size() - 2] == K, "matmul: inner dimensions do not match");
    const Sizes batch = broadcast_shape(Sizes(sa.begin(), sa.end() - 2), Sizes(sb.begin(), sb.end() - 2));
    const int64_t B = std::accumulate(batch.begin(), batch.end(), int64_t(1),
                                      std::multiplies<int64_t>());
    auto expanded = [&](const TensorRef& t, int64_t r, int64_t c) {
        Sizes shape = batch;
        shape.push_back(r);
        shape.push_back(c);
        const TensorRef e = sizes_of(t) == shape ? t : expand_to(t, shape);
        return reshape_dense(e, {B, r, c});
    };
    MaybeOwned ea = expanded(a.ref, M, K), eb = expanded(b.ref, K, N);
    Owned out = bmm_native(ea.ref, eb.ref);
    Sizes shape = batch;
    if (da > 1) shape.push_back(M);
    if (db > 1) shape.push_back(N);
    return with_shape(std::move(out), shape);
}

}  // namespace

extern "C" {

int tp_amd_mm(const tp_amd_tensor* self, const tp_amd_tensor* mat2, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return mm_op(deref(self, "self"), deref(mat2, "mat2")); });
}

int tp_amd_bmm(const tp_amd_tensor* self, const tp_amd_tensor* mat2, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return bmm_op(deref(self, "self"), deref(mat2, "mat2")); });
}

int tp_amd_addmm(const tp_amd_tensor* self, const tp_amd_tensor* mat1, const tp_amd_tensor* mat2,
                 tp_amd_scalar beta, tp_amd_scalar alpha, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return addmm_op(deref(self, "self"), deref(mat1, "mat1"), deref(mat2, "mat2"), beta.f,
                        alpha.f);
    });
}

int tp_amd_linear(const tp_amd_tensor* input, const tp_amd_tensor* weight,
                  const tp_amd_tensor* bias, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return linear_op(deref(input, "input"), deref(weight, "weight"), bias);
    });
}

int tp_amd_matmul(const tp_amd_tensor* self, const tp_amd_tensor* other, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return matmul_op(deref(self, "self"), deref(other, "other")); });
}

}  // extern "C"
