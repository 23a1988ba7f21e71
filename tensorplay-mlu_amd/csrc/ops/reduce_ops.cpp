// Reductions and softmax: the C entry points for the reference's 12 reduce
// registrations (tensorplay_mlu/csrc/ReduceKernels.cpp:47-282), over the
// gfx950 reduction and fused softmax kernels.

#include <algorithm>

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

// One reduction of a dense tensor over a single run of adjacent dims
// [first, last]: the kernel's [outer, r, inner] view.
void reduce_run(const TensorRef& x, const Sizes& shape, int first, int last, int op,
                const TensorRef& out) {
    int64_t outer = 1, r = 1, inner = 1;
    for (int d = 0; d < first; ++d) outer *= shape[d];
    for (int d = first; d <= last; ++d) r *= shape[d];
    for (int d = last + 1; d < static_cast<int>(shape.size()); ++d) inner *= shape[d];
    const int st = tp_amd_launch_reduce(x.device, op, x.dtype, outer, r, inner, x.data, out.data);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
}

// When ``t`` is a permutation of a dense tensor (its strides, largest
// first, are the row-major strides of its sizes in that order), the dims in
// memory order, outermost first; otherwise empty.
std::vector<int> dense_order(const TensorRef& t) {
    const int nd = t.ndim;
    std::vector<int> order(nd);
    for (int i = 0; i < nd; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        // size-1 dims last, they hold no layout
        if ((t.sizes[a] == 1) != (t.sizes[b] == 1)) return t.sizes[b] == 1;
        return t.strides[a] > t.strides[b];
    });
    int64_t expected = 1;
    for (int i = nd - 1; i >= 0; --i) {
        const int d = order[i];
        if (t.sizes[d] == 1) continue;
        if (t.strides[d] != expected) return {};
        expected *= t.sizes[d];
    }
    return order;
}

Owned reduce_dense(const TensorRef& x, Sizes dims, bool keepdim, int op, int out_dtype, int device);

// Reduce ``self`` over ``dims`` (all when empty) into a keepdim-shaped
// tensor, then view it without the reduced dimensions unless keepdim
// (reduce(), :47-84).  The input is converted to the result dtype first.
// Reduced dims that are not adjacent take one pass per run of adjacent
// reduced dims, innermost run first, with float32 intermediates.  A
// non-contiguous input that is a permutation of a dense tensor (a
// transpose) is reduced where it lies, its dims taken in memory order, and
// only the (smaller) result is reordered if its kept dims come out of
// order; other strided inputs are copied dense first.
Owned reduce(const TensorRef& self, Sizes dims, bool keepdim, int op, int out_dtype) {
    const int nd = self.ndim;
    if (nd > 1 && self.dtype == out_dtype && !is_contiguous(self) && numel(self) > 0) {
        const std::vector<int> order = dense_order(self);
        if (!order.empty()) {
            std::vector<bool> reduced(nd, dims.empty());
            for (int64_t d : dims) {
                const int64_t k = d < 0 ? d + nd : d;
                TP_AMD_CHECK(k >= 0 && k < nd, "dimension ", d, " out of range for a ", nd, "-d tensor");
                reduced[k] = true;
            }
            // The same bytes viewed in memory order, and the dims to reduce there.
            Sizes psizes(nd), pstrides(nd), pdims;
            for (int i = 0; i < nd; ++i) {
                psizes[i] = self.sizes[order[i]];
                pstrides[i] = self.strides[order[i]];
                if (reduced[order[i]]) pdims.push_back(i);
            }
            TensorRef dense = make_view(self, psizes, pstrides);
            dense.ctx = self.ctx;
            Owned pout = reduce_dense(dense, pdims, true, op, out_dtype, self.device);
            // pout: keepdim result in memory order; view it in logical order.
            Sizes keep(nd), kstrides(nd);
            for (int i = 0; i < nd; ++i) keep[i] = reduced[i] ? 1 : self.sizes[i];
            const Sizes pstr = contiguous_strides(sizes_of(pout.ref()));
            for (int i = 0; i < nd; ++i) kstrides[order[i]] = pstr[i];
            TensorRef logical = make_view(pout.ref(), keep, kstrides);
            Owned out = empty_on(keep, out_dtype, self.device);
            strided_copy(out.ref(), logical);  // one memcpy when the order already matches
            if (keepdim) return out;
            Sizes final_shape;
            for (int i = 0; i < nd; ++i)
                if (!reduced[i]) final_shape.push_back(self.sizes[i]);
            TensorRef view = make_view(out.ref(), final_shape, contiguous_strides(final_shape));
            view.ctx = out.ref().ctx;
            out.release();
            return Owned(view);
        }
    }
    return reduce_dense(self, std::move(dims), keepdim, op, out_dtype, self.device);
}

Owned reduce_dense(const TensorRef& self, Sizes dims, bool keepdim, int op, int out_dtype, int) {
    const int nd = self.ndim;
    MaybeOwned converted = to_dtype(self, out_dtype);
    MaybeOwned x = contiguous_on_device(converted.ref);
    if (nd == 0) {
        Owned out = empty_on({}, out_dtype, self.device);
        strided_copy(out.ref(), x.ref);
        return out;
    }
    if (dims.empty()) {
        dims.resize(nd);
        for (int i = 0; i < nd; ++i) dims[i] = i;
    }
    std::vector<bool> reduced(nd, false);
    for (int64_t d : dims) {
        const int64_t k = d < 0 ? d + nd : d;
        TP_AMD_CHECK(k >= 0 && k < nd, "dimension ", d, " out of range for a ", nd, "-d tensor");
        reduced[k] = true;
    }
    Sizes keep_shape = sizes_of(x.ref), final_shape;
    for (int i = 0; i < nd; ++i) {
        if (reduced[i]) {
            keep_shape[i] = 1;
            if (keepdim) final_shape.push_back(1);
        } else {
            final_shape.push_back(x.ref.sizes[i]);
        }
    }
    Owned out = empty_on(keep_shape, out_dtype, self.device);
    if (numel(x.ref) == 0) {
        fill(out.ref(), scalar_of(0.0));
    } else {
        // Runs of adjacent reduced dims, ignoring size-1 dims in between.
        std::vector<std::pair<int, int>> runs;
        for (int i = 0; i < nd; ++i) {
            if (!reduced[i]) continue;
            if (!runs.empty()) {
                bool adjacent = true;
                for (int k = runs.back().second + 1; k < i; ++k)
                    if (x.ref.sizes[k] != 1) adjacent = false;
                if (adjacent) {
                    runs.back().second = i;
                    continue;
                }
            }
            runs.emplace_back(i, i);
        }
        if (runs.size() == 1) {
            reduce_run(x.ref, sizes_of(x.ref), runs[0].first, runs[0].second, op, out.ref());
        } else {
            // Several runs: float32 passes, innermost run first.
            MaybeOwned cur = to_dtype(x.ref, TP_AMD_FLOAT32);
            Sizes shape = sizes_of(x.ref);
            Owned stage;
            for (int k = static_cast<int>(runs.size()) - 1; k >= 0; --k) {
                Sizes next = shape;
                for (int d = runs[k].first; d <= runs[k].second; ++d) next[d] = 1;
                Owned dst = empty_on(next, TP_AMD_FLOAT32, self.device);
                reduce_run(cur.ref, shape, runs[k].first, runs[k].second, op, dst.ref());
                shape = next;
                stage = std::move(dst);
                cur.ref = stage.ref();
            }
            cast_dense(out.ref(), stage.ref());
        }
    }
    if (keepdim) return out;
    TensorRef view = make_view(out.ref(), final_shape, contiguous_strides(final_shape));
    view.ctx = out.ref().ctx;
    out.release();
    return Owned(view);
}

int reduce_dtype(const TensorRef& self, int requested) {
    return requested == TP_AMD_UNDEFINED ? self.dtype : requested;
}

void require_native_reduce(const TensorRef& self, int out_dtype) {
    check_view(self, "self");
    const bool ok = on_device(self) && is_native_float(out_dtype) &&
                    (is_native_float(self.dtype) || self.dtype == out_dtype);
    if (!ok) TP_AMD_DECLINE("reduction dtype has no device kernel");
}

Owned reduce_entry(const tp_amd_tensor* self, const int64_t* dims, int ndims, bool keepdim,
                   int op, int dtype, bool use_requested) {
    const TensorRef& s = deref(self, "self");
    const int out = use_requested ? reduce_dtype(s, dtype) : s.dtype;
    require_native_reduce(s, out);
    Sizes d;
    if (dims != nullptr && ndims > 0) d.assign(dims, dims + ndims);
    return reduce(s, d, keepdim, op, out);
}

// softmax over ``dim`` of a dense tensor seen as [outer, dim, inner]
// (softmax_shape, :147-161).
struct SoftmaxShape {
    int64_t outer, dim, inner;
};

SoftmaxShape softmax_shape(const TensorRef& t, int64_t dim) {
    const int64_t nd = std::max<int64_t>(t.ndim, 1);
    if (dim < 0) dim += nd;
    TP_AMD_CHECK(dim >= 0 && dim < nd, "softmax dimension out of range");
    const Sizes s = t.ndim == 0 ? Sizes{1} : sizes_of(t);
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < dim; ++i) outer *= s[i];
    for (int64_t i = dim + 1; i < nd; ++i) inner *= s[i];
    return {outer, s[dim], inner};
}

Owned softmax_forward(const TensorRef& self, int64_t dim, bool log) {
    MaybeOwned x = contiguous_on_device(self);
    Owned y = empty_on(sizes_of(x.ref), x.ref.dtype, x.ref.device);
    if (numel(y.ref()) == 0) return y;
    const SoftmaxShape sh = softmax_shape(x.ref, dim);
    const int st = tp_amd_launch_softmax(x.ref.device, log ? 1 : 0, x.ref.dtype, sh.outer, sh.dim,
                                         sh.inner, x.ref.data, y.ref().data);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    return y;
}

Owned softmax_backward(const TensorRef& grad, const TensorRef& output, int64_t dim, bool log) {
    MaybeOwned dy = contiguous_on_device(grad);
    MaybeOwned y = contiguous_on_device(output);
    Owned dx = empty_on(sizes_of(dy.ref), dy.ref.dtype, dy.ref.device);
    if (numel(dx.ref()) == 0) return dx;
    const SoftmaxShape sh = softmax_shape(dy.ref, dim);
    const int st = tp_amd_launch_softmax_backward(dy.ref.device, log ? 1 : 0, dy.ref.dtype,
                                                  sh.outer, sh.dim, sh.inner, y.ref.data,
                                                  dy.ref.data, dx.ref().data);
    TP_AMD_CHECK(st == TP_AMD_OK, last_error());
    return dx;
}

bool native_softmax(const TensorRef& self, bool half_to_float) {
    return on_device(self) && !half_to_float && is_native_float(self.dtype);
}

// softmax / log_softmax with a result dtype (softmax_dtype_kernel, :201-222).
Owned softmax_dtype(const TensorRef& self, int64_t dim, int dtype, bool log) {
    check_view(self, "self");
    const int out = dtype == TP_AMD_UNDEFINED ? self.dtype : dtype;
    if (!(on_device(self) && is_native_float(out) && is_native_float(self.dtype))) {
        TP_AMD_DECLINE("softmax dtype has no device kernel");
    }
    MaybeOwned x = to_dtype(self, out);
    return softmax_forward(x.ref, dim, log);
}

Owned softmax_plain(const TensorRef& self, int64_t dim, bool half_to_float, bool log) {
    check_view(self, "self");
    if (!native_softmax(self, half_to_float)) TP_AMD_DECLINE("softmax has no device kernel here");
    return softmax_forward(self, dim, log);
}

Owned softmax_backward_entry(const TensorRef& grad, const TensorRef& output, int64_t dim,
                             int input_dtype, bool log) {
    check_view(grad, "grad_output");
    check_view(output, "output");
    if (!(native_softmax(grad, false) && output.dtype == grad.dtype &&
          input_dtype == grad.dtype && on_device(output) && output.device == grad.device &&
          sizes_of(output) == sizes_of(grad))) {
        TP_AMD_DECLINE("softmax backward operands do not agree");
    }
    return softmax_backward(grad, output, dim, log);
}

}  // namespace

extern "C" {

int tp_amd_sum(const tp_amd_tensor* self, int dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return reduce_entry(self, nullptr, 0, false, TP_AMD_REDUCE_SUM, dtype, true);
    });
}

int tp_amd_mean(const tp_amd_tensor* self, int dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return reduce_entry(self, nullptr, 0, false, TP_AMD_REDUCE_MEAN, dtype, true);
    });
}

int tp_amd_sum_dim(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                   int dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return reduce_entry(self, dims, ndims, keepdim != 0, TP_AMD_REDUCE_SUM, dtype, true);
    });
}

int tp_amd_mean_dim(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                    int dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return reduce_entry(self, dims, ndims, keepdim != 0, TP_AMD_REDUCE_MEAN, dtype, true);
    });
}

int tp_amd_amax(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return reduce_entry(self, dims, ndims, keepdim != 0, TP_AMD_REDUCE_AMAX,
                            TP_AMD_UNDEFINED, false);
    });
}

int tp_amd_amin(const tp_amd_tensor* self, const int64_t* dims, int ndims, int keepdim,
                tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return reduce_entry(self, dims, ndims, keepdim != 0, TP_AMD_REDUCE_AMIN,
                            TP_AMD_UNDEFINED, false);
    });
}

int tp_amd_softmax(const tp_amd_tensor* self, int64_t dim, int dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] { return softmax_dtype(deref(self, "self"), dim, dtype, false); });
}

int tp_amd_log_softmax(const tp_amd_tensor* self, int64_t dim, int dtype,
                       tp_amd_tensor* result) {
    return guarded_result(result, [&] { return softmax_dtype(deref(self, "self"), dim, dtype, true); });
}

int tp_amd__softmax(const tp_amd_tensor* self, int64_t dim, int half_to_float,
                    tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return softmax_plain(deref(self, "self"), dim, half_to_float != 0, false);
    });
}

int tp_amd__log_softmax(const tp_amd_tensor* self, int64_t dim, int half_to_float,
                        tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return softmax_plain(deref(self, "self"), dim, half_to_float != 0, true);
    });
}

int tp_amd__softmax_backward_data(const tp_amd_tensor* grad_output, const tp_amd_tensor* output,
                                  int64_t dim, int input_dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return softmax_backward_entry(deref(grad_output, "grad_output"), deref(output, "output"),
                                      dim, input_dtype, false);
    });
}

int tp_amd__log_softmax_backward_data(const tp_amd_tensor* grad_output,
                                      const tp_amd_tensor* output, int64_t dim,
                                      int input_dtype, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        return softmax_backward_entry(deref(grad_output, "grad_output"), deref(output, "output"),
                                      dim, input_dtype, true);
    });
}

}  // extern "C"
