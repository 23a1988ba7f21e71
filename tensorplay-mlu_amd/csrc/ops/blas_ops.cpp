// Matrix products: mm, bmm, addmm, linear and matmul (the five BLAS
// registrations of tensorplay_mlu/csrc/BlasKernels.cpp:416-422).
//
// Every entry point only validates its operands and states its product as
//
//     out[b] (m x n) = alpha * L[b] (m x k) . R[b] (k x n) + beta * addend
//
// over a batch shape (empty for a plain product).  One planner (Product)
// then decides how the gfx950 GEMM kernels address each side:
//   * a side whose matrix is row-major, or the transpose of a row-major
//     matrix, with any leading dimension, is read where it lies; its batch
//     dimensions must collapse to one stride (0 for a broadcast side);
//   * anything else -- stride-0 matrix axes, unmergeable batch strides --
//     is first copied into a dense stack;
//   * a left side whose batch continues its rows, against a broadcast right
//     side, folds the batch into the rows: one product of B*m rows (the
//     [..., M, K] @ [K, N] matmul case, and linear on a 3-D input);
// and launches one GEMM.  The result is allocated directly in the shape the
// caller sees (vector operands drop their unit axis, linear keeps the
// input's leading dimensions), which is the dense [B, m, n] stack the GEMM
// writes.
//
// Semantics kept from the reference: which operands decline to the host
// (:244-248 and each kernel's first test), the shape errors, an inner size
// of 0 giving zeros or beta * bias (:265-268, :277-280, :326-329), addmm's
// beta * bias + alpha * product with the bias ignored when beta is 0
// (:318-324), linear as a product over the flattened rows with W read
// transposed (:338-356), and matmul's 1-D promotion and batch broadcasting
// (:360-412).  Where the reference densifies (reshape_dense, the expanded
// batch of the general matmul case) this planner reads in place whenever
// the kernels can; the values are the same dot products either way.

#include <utility>
#include <vector>

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

// How the kernels address one side: matrix b starts at data + b *
// batch_stride elements; element (i, j) sits at i * ld + j, or at j * ld + i
// when the side is stored as the transpose of a row-major matrix.
struct MatrixRead {
    const void* data = nullptr;
    int64_t ld = 1;
    int64_t batch_stride = 0;
    bool transposed = false;
};

// The matrix axes (the last two) of ``t`` as a MatrixRead, or false when
// neither axis is unit-stride with the other spanning at least a full line.
bool matrix_axes_in_place(const TensorRef& t, MatrixRead& read) {
    const int64_t rows = t.sizes[t.ndim - 2], cols = t.sizes[t.ndim - 1];
    const int64_t row_step = t.strides[t.ndim - 2], col_step = t.strides[t.ndim - 1];
    read.data = t.data;
    if ((cols == 1 || col_step == 1) && (rows == 1 || row_step >= cols)) {
        read.transposed = false;
        read.ld = rows == 1 ? cols : row_step;
        return true;
    }
    if ((rows == 1 || row_step == 1) && (cols == 1 || col_step >= rows)) {
        read.transposed = true;
        read.ld = cols == 1 ? rows : col_step;
        return true;
    }
    return false;
}

// The first ``nbatch`` axes of ``t`` walked as one flattened index: true with
// the single element stride that index steps by, or false when the axes do
// not merge (a broadcast axis next to a stored one, or a gap).
bool batch_axes_merge(const TensorRef& t, int nbatch, int64_t& step) {
    bool seen = false;
    int64_t next = 0;  // the stride the next outer non-unit axis must have
    step = 0;
    for (int d = nbatch - 1; d >= 0; --d) {
        if (t.sizes[d] == 1) continue;
        if (!seen) {
            step = t.strides[d];
            next = step * t.sizes[d];
            seen = true;
        } else if (t.strides[d] != next) {
            return false;
        } else {
            next *= t.sizes[d];
        }
    }
    return true;
}

Sizes with_matrix(Sizes shape, int64_t rows, int64_t cols) {
    shape.push_back(rows);
    shape.push_back(cols);
    return shape;
}

class Product {
public:
    // lhs [..., m, k] and rhs [..., k, n], both with at least two axes, inner
    // sizes already checked equal; ``batch`` is their broadcast batch shape
    // and ``result_shape`` the shape handed back (numel batch * m * n).
    Product(const TensorRef& lhs, const TensorRef& rhs, Sizes batch, Sizes result_shape)
        : lhs_(lhs), rhs_(rhs), batch_shape_(std::move(batch)), result_shape_(std::move(result_shape)) {
        m_ = lhs.sizes[lhs.ndim - 2];
        k_ = lhs.sizes[lhs.ndim - 1];
        n_ = rhs.sizes[rhs.ndim - 1];
        batch_ = 1;
        for (int64_t d : batch_shape_) batch_ *= d;
    }

    // ``addend`` (beta != 0 only) is a 2-D view over all batch * m output
    // rows: row r of it is added to output row r.
    Owned run(float alpha, float beta, const TensorRef* addend) {
        Owned out = empty_on(result_shape_, lhs_.dtype, lhs_.device);
        if (numel(out.ref()) == 0) return out;
        const TensorRef rows = make_view(out.ref(), {batch_ * m_, n_}, {n_, 1});
        if (k_ == 0) {
            no_terms(rows, beta, addend);
            return out;
        }
        std::vector<Owned> copies;
        const MatrixRead l = address(lhs_, m_, k_, copies);
        const MatrixRead r = address(rhs_, k_, n_, copies);
        // Fold the batch into the rows when the left stack's rows run on
        // from one matrix to the next and the right side is shared.
        const bool fold = batch_ > 1 && r.batch_stride == 0 && !l.transposed &&
                          l.batch_stride == m_ * l.ld;
        const int64_t nb = fold ? 1 : batch_, m = fold ? batch_ * m_ : m_;
        const void* cin = nullptr;
        int64_t cin_rs = 0, cin_cs = 0;
        if (addend != nullptr && beta != 0.0f) {
            cin = addend->data;
            cin_rs = addend->strides[0];
            cin_cs = addend->strides[1];
        } else {
            beta = 0.0f;
        }
        const int st = tp_amd_launch_gemm(
            rows.device, rows.dtype, nb, m, n_, k_, alpha, l.data, l.ld, fold ? 0 : l.batch_stride,
            l.transposed ? 1 : 0, r.data, r.ld, r.batch_stride, r.transposed ? 1 : 0, beta, cin, cin_rs,
            cin_cs, m * cin_rs, rows.data, n_, m * n_);
        TP_AMD_CHECK(st == TP_AMD_OK, last_error());
        return out;
    }

private:
    // An empty sum: every output element is 0, or beta * addend.
    static void no_terms(const TensorRef& rows, float beta, const TensorRef* addend) {
        if (addend == nullptr || beta == 0.0f) {
            fill(rows, scalar_of(0.0));
            return;
        }
        strided_copy(rows, *addend);
        if (beta != 1.0f) {
            const int st = tp_amd_launch_affine(rows.device, rows.dtype, numel(rows), rows.data, beta,
                                                0.0f, rows.data);
            TP_AMD_CHECK(st == TP_AMD_OK, last_error());
        }
    }

    // One side as the kernels read it, copying it into ``copies`` when its
    // layout cannot be addressed.  A side whose own batch axes are all 1 is
    // shared by every matrix of the batch (stride 0), and only its one
    // matrix is ever copied.
    MatrixRead address(const TensorRef& side, int64_t rows, int64_t cols, std::vector<Owned>& copies) const {
        const int own = side.ndim - 2;
        bool shared = true;
        for (int d = 0; d < own; ++d) shared = shared && side.sizes[d] == 1;
        MatrixRead read;
        if (shared) {
            const TensorRef matrix = make_view(side, {rows, cols}, {side.strides[own], side.strides[own + 1]});
            if (matrix_axes_in_place(matrix, read)) return read;
            return dense_copy(matrix, {rows, cols}, copies);
        }
        const Sizes full = with_matrix(batch_shape_, rows, cols);
        const TensorRef stack = expand_to(side, full);
        const int nbatch = static_cast<int>(batch_shape_.size());
        if (matrix_axes_in_place(stack, read) && batch_axes_merge(stack, nbatch, read.batch_stride)) {
            return read;
        }
        MatrixRead packed = dense_copy(stack, full, copies);
        packed.batch_stride = rows * cols;
        return packed;
    }

    static MatrixRead dense_copy(const TensorRef& view, const Sizes& shape, std::vector<Owned>& copies) {
        copies.push_back(empty_on(shape, view.dtype, view.device));
        strided_copy(copies.back().ref(), view);
        MatrixRead read;
        read.data = copies.back().ref().data;
        read.ld = shape.back();
        return read;
    }

    TensorRef lhs_, rhs_;
    Sizes batch_shape_, result_shape_;
    int64_t batch_ = 1, m_ = 0, n_ = 0, k_ = 0;
};

// Both sides on one device in one of the three float dtypes the kernels
// take; any other pairing runs on the host.
bool device_float_pair(const TensorRef& a, const TensorRef& b) {
    return on_device(a) && on_device(b) && a.device == b.device && a.dtype == b.dtype &&
           is_native_float(a.dtype);
}

// A 1-D operand as a one-row ([1, k]) or one-column ([k, 1]) matrix view.
TensorRef as_row(const TensorRef& v) {
    return make_view(v, {1, v.sizes[0]}, {v.sizes[0] * v.strides[0], v.strides[0]});
}
TensorRef as_column(const TensorRef& v) { return make_view(v, {v.sizes[0], 1}, {v.strides[0], 1}); }

TensorRef swap_last_two(const TensorRef& t) {
    Sizes sizes = sizes_of(t), strides = strides_of(t);
    std::swap(sizes[t.ndim - 2], sizes[t.ndim - 1]);
    std::swap(strides[t.ndim - 2], strides[t.ndim - 1]);
    return make_view(t, sizes, strides);
}

Owned mm_op(const TensorRef& self, const TensorRef& mat2) {
    check_view(self, "self");
    check_view(mat2, "mat2");
    if (!device_float_pair(self, mat2) || self.ndim != 2 || mat2.ndim != 2) {
        TP_AMD_DECLINE("mm runs on the device for two 2-D float tensors of one dtype");
    }
    TP_AMD_CHECK(self.sizes[1] == mat2.sizes[0], "mm: [", self.sizes[0], ", ", self.sizes[1],
                 "] times [", mat2.sizes[0], ", ", mat2.sizes[1], "]: the inner sizes differ");
    return Product(self, mat2, {}, {self.sizes[0], mat2.sizes[1]}).run(1.0f, 0.0f, nullptr);
}

Owned bmm_op(const TensorRef& self, const TensorRef& mat2) {
    check_view(self, "self");
    check_view(mat2, "mat2");
    if (!device_float_pair(self, mat2) || self.ndim != 3 || mat2.ndim != 3) {
        TP_AMD_DECLINE("bmm runs on the device for two 3-D float tensors of one dtype");
    }
    TP_AMD_CHECK(self.sizes[0] == mat2.sizes[0], "bmm: ", self.sizes[0], " and ", mat2.sizes[0],
                 " matrices in the two stacks");
    TP_AMD_CHECK(self.sizes[2] == mat2.sizes[1], "bmm: inner sizes ", self.sizes[2], " and ",
                 mat2.sizes[1], " differ");
    const int64_t b = self.sizes[0];
    return Product(self, mat2, {b}, {b, self.sizes[1], mat2.sizes[2]}).run(1.0f, 0.0f, nullptr);
}

Owned addmm_op(const TensorRef& self, const TensorRef& mat1, const TensorRef& mat2, double beta,
               double alpha) {
    check_view(self, "self");
    check_view(mat1, "mat1");
    check_view(mat2, "mat2");
    if (!device_float_pair(mat1, mat2) || mat1.ndim != 2 || mat2.ndim != 2 ||
        !device_float_pair(self, mat1)) {
        TP_AMD_DECLINE("addmm runs on the device when bias and both matrices share a float dtype and device");
    }
    TP_AMD_CHECK(mat1.sizes[1] == mat2.sizes[0], "addmm: mat1 has ", mat1.sizes[1],
                 " columns but mat2 has ", mat2.sizes[0], " rows");
    const int64_t m = mat1.sizes[0], n = mat2.sizes[1];
    Product product(mat1, mat2, {}, {m, n});
    // beta is applied in float32; a beta that rounds to 0 leaves the bias
    // unread (its shape is not even checked), as the reference's does.
    const float a = static_cast<float>(alpha), b = static_cast<float>(beta);
    if (b == 0.0f) return product.run(a, 0.0f, nullptr);
    const TensorRef bias = expand_to(self, {m, n});
    return product.run(a, b, &bias);
}

Owned linear_op(const TensorRef& input, const TensorRef& weight, const TensorRef* bias) {
    check_view(input, "input");
    check_view(weight, "weight");
    if (bias != nullptr) check_view(*bias, "bias");
    if (!device_float_pair(input, weight) || input.ndim == 0 || weight.ndim != 2 ||
        (bias != nullptr && !device_float_pair(*bias, input))) {
        TP_AMD_DECLINE("linear runs on the device when input, weight and bias share a float dtype and device");
    }
    const int64_t n = weight.sizes[0], k = weight.sizes[1];
    TP_AMD_CHECK(input.sizes[input.ndim - 1] == k, "linear: input rows have ",
                 input.sizes[input.ndim - 1], " features, the weight expects ", k);
    // The rows of the product are every index of the input's leading axes.
    Sizes result = sizes_of(input);
    result.back() = n;
    int64_t rows = 1;
    for (int d = 0; d + 1 < input.ndim; ++d) rows *= input.sizes[d];
    const TensorRef lhs = input.ndim == 1 ? as_row(input) : input;
    const Sizes batch(lhs.sizes, lhs.sizes + lhs.ndim - 2);
    Product product(lhs, swap_last_two(weight), batch, result);
    if (bias == nullptr) return product.run(1.0f, 0.0f, nullptr);
    const TensorRef addend = expand_to(*bias, {rows, n});
    return product.run(1.0f, 1.0f, &addend);
}

Owned matmul_op(const TensorRef& self, const TensorRef& other) {
    check_view(self, "self");
    check_view(other, "other");
    if (!device_float_pair(self, other) || self.ndim == 0 || other.ndim == 0) {
        TP_AMD_DECLINE("matmul runs on the device for float tensors of one dtype with at least one axis");
    }
    // A vector on the left is one row, on the right one column; that unit
    // axis is dropped from the result.
    const TensorRef lhs = self.ndim == 1 ? as_row(self) : self;
    const TensorRef rhs = other.ndim == 1 ? as_column(other) : other;
    const int64_t m = lhs.sizes[lhs.ndim - 2], k = lhs.sizes[lhs.ndim - 1];
    const int64_t n = rhs.sizes[rhs.ndim - 1];
    TP_AMD_CHECK(rhs.sizes[rhs.ndim - 2] == k, "matmul: the left operand's last axis has ", k,
                 " entries, the right operand's contracted axis ", rhs.sizes[rhs.ndim - 2]);
    const Sizes batch = broadcast_shape(Sizes(lhs.sizes, lhs.sizes + lhs.ndim - 2),
                                        Sizes(rhs.sizes, rhs.sizes + rhs.ndim - 2));
    Sizes result = batch;
    if (self.ndim > 1) result.push_back(m);
    if (other.ndim > 1) result.push_back(n);
    return Product(lhs, rhs, batch, result).run(1.0f, 0.0f, nullptr);
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
