// Neural-network layers: the C entry points for the reference's 8 NN
// registrations (tensorplay_mlu/csrc/NNKernels.cpp:57-395) -- layer norm,
// dropout, embedding and the negative log-likelihood loss, forward and
// backward -- over the gfx950 kernels of kernels/nn.hip.  Each entry
// declines (TP_AMD_DECLINED) exactly where the reference hands the call to
// the host kernel.

#include <cmath>
#include <initializer_list>

#include "tensor.h"
#include "tp_amd_kernels.h"
#include "tp_amd_ops.h"

using namespace tp_amd;

namespace {

bool native_float_dtype(int dtype) {
    return dtype == TP_AMD_FLOAT32 || dtype == TP_AMD_FLOAT16 || dtype == TP_AMD_BFLOAT16;
}

bool native_float(const TensorRef& t) { return on_device(t) && native_float_dtype(t.dtype); }

// An optional affine parameter usable next to ``x``: absent, or on x's
// device with x's dtype (usable_param, :33-36).
bool usable_param(const tp_amd_tensor* p, const TensorRef& x) {
    return p == nullptr || (on_device(*p) && p->dtype == x.dtype && p->device == x.device);
}

bool index_tensor(const TensorRef& t) {
    return on_device(t) && (t.dtype == TP_AMD_INT64 || t.dtype == TP_AMD_INT32);
}

void check_status(int st) { TP_AMD_CHECK(st == TP_AMD_OK, last_error()); }

// The result slot of an output the caller did not ask for: no data, no
// dtype.
void set_undefined(tp_amd_tensor* r) {
    *r = tp_amd_tensor{};
    r->dtype = TP_AMD_UNDEFINED;
    r->device = -1;
}

// Several results: every slot is written only once all of them exist.
template <typename Body>
int guarded_results(std::initializer_list<tp_amd_tensor*> slots, Body&& body) noexcept {
    return guarded([&] {
        for (tp_amd_tensor* s : slots) TP_AMD_CHECK(s != nullptr, "null result pointer");
        body();
    });
}

// Filled with ``value`` (dtype per the fill encoding).
Owned filled(const Sizes& sizes, int dtype, int device, double value) {
    Owned t = empty_on(sizes, dtype, device);
    if (numel(t.ref()) > 0) fill(t.ref(), scalar_of(value));
    return t;
}

// ---- layer norm ---------------------------------------------------------------

// [outer, D] split of ``input`` for normalized_shape; -1 when the reference
// would decline (:61-68).
int64_t layer_norm_axis(const TensorRef& input, const int64_t* shape, int nnorm) {
    const int64_t axis = input.ndim - nnorm;
    if (nnorm <= 0 || axis <= 0) return -1;
    for (int i = 0; i < nnorm; ++i) {
        if (input.sizes[axis + i] != shape[i]) return -1;
    }
    return axis;
}

}  // namespace

extern "C" {

int tp_amd_native_layer_norm(const tp_amd_tensor* input, const int64_t* normalized_shape, int nnorm,
                             const tp_amd_tensor* weight, const tp_amd_tensor* bias, double eps,
                             tp_amd_tensor* y, tp_amd_tensor* mean, tp_amd_tensor* rstd) {
    return guarded_results({y, mean, rstd}, [&] {
        const TensorRef& in = deref(input, "input");
        const int64_t axis = layer_norm_axis(in, normalized_shape, nnorm);
        if (!native_float(in) || axis < 0 || !usable_param(weight, in) || !usable_param(bias, in)) {
            TP_AMD_DECLINE("layer_norm: not native for these operands");
        }
        if (numel(in) == 0) TP_AMD_DECLINE("layer_norm: empty input");
        MaybeOwned x = contiguous_on_device(in);
        int64_t outer = 1, D = 1;
        for (int64_t i = 0; i < axis; ++i) outer *= in.sizes[i];
        for (int i = 0; i < nnorm; ++i) D *= normalized_shape[i];
        MaybeOwned w, b;
        if (weight != nullptr) w = contiguous_on_device(*weight);
        if (bias != nullptr) b = contiguous_on_device(*bias);
        TP_AMD_CHECK(weight == nullptr || numel(w.ref) == D, "layer_norm: weight size");
        TP_AMD_CHECK(bias == nullptr || numel(b.ref) == D, "layer_norm: bias size");
        Owned out = empty_on(sizes_of(x.ref), x.ref.dtype, in.device);
        // The statistics are float32 for every native dtype (stats_dtype,
        // :52-54), shaped [outer] (:80).
        Owned m = empty_on({outer}, TP_AMD_FLOAT32, in.device);
        Owned r = empty_on({outer}, TP_AMD_FLOAT32, in.device);
        check_status(tp_amd_launch_layer_norm(in.device, in.dtype, outer, D, x.ref.data,
                                              weight ? w.ref.data : nullptr, bias ? b.ref.data : nullptr,
                                              eps, out.ref().data, static_cast<float*>(m.ref().data),
                                              static_cast<float*>(r.ref().data)));
        *y = out.release();
        *mean = m.release();
        *rstd = r.release();
    });
}

int tp_amd_native_layer_norm_backward(const tp_amd_tensor* grad_out, const tp_amd_tensor* input,
                                      const int64_t* normalized_shape, int nnorm,
                                      const tp_amd_tensor* mean, const tp_amd_tensor* rstd,
                                      const tp_amd_tensor* weight, const tp_amd_tensor* bias,
                                      const int* output_mask, tp_amd_tensor* dx, tp_amd_tensor* dweight,
                                      tp_amd_tensor* dbias) {
    (void)bias;  // not needed for the gradients (:150-159 passes it through)
    return guarded_results({dx, dweight, dbias}, [&] {
        const TensorRef& in = deref(input, "input");
        const TensorRef& dz = deref(grad_out, "grad_out");
        const TensorRef& mu = deref(mean, "mean");
        const TensorRef& rs = deref(rstd, "rstd");
        const int64_t axis = layer_norm_axis(in, normalized_shape, nnorm);
        if (!native_float(in) || !on_device(dz) || dz.dtype != in.dtype || !on_device(mu) ||
            !on_device(rs) || axis < 0 || !usable_param(weight, in) || sizes_of(dz) != sizes_of(in)) {
            TP_AMD_DECLINE("layer_norm_backward: not native for these operands");
        }
        if (numel(in) == 0) TP_AMD_DECLINE("layer_norm_backward: empty input");
        auto want = [&](int i) { return output_mask == nullptr || output_mask[i] != 0; };
        MaybeOwned x = contiguous_on_device(in);
        MaybeOwned g = contiguous_on_device(dz);
        int64_t outer = 1, D = 1;
        for (int64_t i = 0; i < axis; ++i) outer *= in.sizes[i];
        for (int i = 0; i < nnorm; ++i) D *= normalized_shape[i];
        // The statistics in float32 (:130-131).
        MaybeOwned m32 = to_dtype(mu, TP_AMD_FLOAT32);
        MaybeOwned r32 = to_dtype(rs, TP_AMD_FLOAT32);
        MaybeOwned m = contiguous_on_device(m32.ref);
        MaybeOwned r = contiguous_on_device(r32.ref);
        TP_AMD_CHECK(numel(m.ref) == outer && numel(r.ref) == outer, "layer_norm_backward: ", outer,
                     " rows but statistics of ", numel(m.ref), " and ", numel(r.ref));
        MaybeOwned w;
        if (weight != nullptr) w = contiguous_on_device(*weight);
        TP_AMD_CHECK(weight == nullptr || numel(w.ref) == D, "layer_norm_backward: weight size");
        Sizes norm(normalized_shape, normalized_shape + nnorm);
        Owned odx, odw, odb;
        if (want(0)) odx = empty_on(sizes_of(x.ref), in.dtype, in.device);
        if (want(1)) odw = empty_on(norm, in.dtype, in.device);
        if (want(2)) odb = empty_on(norm, in.dtype, in.device);
        if (want(0) || want(1) || want(2)) {
            check_status(tp_amd_launch_layer_norm_backward(
                in.device, in.dtype, outer, D, g.ref.data, x.ref.data, static_cast<const float*>(m.ref.data),
                static_cast<const float*>(r.ref.data), weight ? w.ref.data : nullptr,
                want(0) ? odx.ref().data : nullptr, want(1) ? odw.ref().data : nullptr,
                want(2) ? odb.ref().data : nullptr));
        }
        if (want(0)) *dx = odx.release(); else set_undefined(dx);
        if (want(1)) *dweight = odw.release(); else set_undefined(dweight);
        if (want(2)) *dbias = odb.release(); else set_undefined(dbias);
    });
}

int tp_amd_native_dropout(const tp_amd_tensor* input, double p, int train, uint64_t seed,
                          tp_amd_tensor* out, tp_amd_tensor* mask) {
    return guarded_results({out, mask}, [&] {
        const TensorRef& in = deref(input, "input");
        if (!native_float(in) || !(p >= 0.0 && p <= 1.0)) {
            TP_AMD_DECLINE("dropout: not native for these operands");
        }
        const Sizes sizes = sizes_of(in);
        // Not training keeps everything; p == 1 drops everything (:170-177).
        if (train == 0 || p == 1.0) {
            const bool keep = train == 0;
            Owned o;
            if (keep) {
                o = empty_on(sizes, in.dtype, in.device);
                copy_into(o.ref(), in);
            } else {
                o = filled(sizes, in.dtype, in.device, 0.0);
            }
            Owned mk = filled(sizes, TP_AMD_BOOL, in.device, keep ? 1.0 : 0.0);
            *out = o.release();
            *mask = mk.release();
            return;
        }
        MaybeOwned x = contiguous_on_device(in);
        Owned o = empty_on(sizes, in.dtype, in.device);
        Owned mk = empty_on(sizes, TP_AMD_BOOL, in.device);
        const int64_t n = numel(x.ref);
        if (n > 0) {
            check_status(tp_amd_launch_dropout(in.device, in.dtype, n, x.ref.data, p, seed, 0, o.ref().data,
                                               static_cast<uint8_t*>(mk.ref().data)));
        }
        *out = o.release();
        *mask = mk.release();
    });
}

int tp_amd_native_dropout_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* mask,
                                   double scale, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        const TensorRef& g = deref(grad_output, "grad_output");
        const TensorRef& mk = deref(mask, "mask");
        if (!native_float(g) || !on_device(mk) || sizes_of(g) != sizes_of(mk) ||
            !(mk.dtype == TP_AMD_BOOL || mk.dtype == TP_AMD_UINT8)) {
            TP_AMD_DECLINE("dropout_backward: not native for these operands");
        }
        MaybeOwned gc = contiguous_on_device(g);
        MaybeOwned mc = contiguous_on_device(mk);
        Owned out = empty_on(sizes_of(g), g.dtype, g.device);
        const int64_t n = numel(gc.ref);
        if (n > 0) {
            check_status(tp_amd_launch_dropout_backward(g.device, g.dtype, n, gc.ref.data,
                                                        static_cast<const uint8_t*>(mc.ref.data), scale,
                                                        out.ref().data));
        }
        return out;
    });
}

int tp_amd_embedding(const tp_amd_tensor* weight, const tp_amd_tensor* indices, int64_t padding_idx,
                     int scale_grad_by_freq, int sparse, tp_amd_tensor* result) {
    (void)padding_idx;          // only the gradient skips the padding row (:250-252)
    (void)scale_grad_by_freq;   // a gradient option
    return guarded_result(result, [&] {
        const TensorRef& w = deref(weight, "weight");
        const TensorRef& idx = deref(indices, "indices");
        if (!native_float(w) || w.ndim != 2 || !index_tensor(idx) || sparse != 0 || w.device != idx.device) {
            TP_AMD_DECLINE("embedding: not native for these operands");
        }
        MaybeOwned wc = contiguous_on_device(w);
        MaybeOwned ic = contiguous_on_device(idx);
        Sizes shape = sizes_of(idx);
        shape.push_back(w.sizes[1]);
        TP_AMD_CHECK(static_cast<int>(shape.size()) <= TP_AMD_MAX_DIMS, "embedding: too many dimensions");
        Owned out = empty_on(shape, w.dtype, w.device);
        if (numel(out.ref()) > 0) {
            check_status(tp_amd_launch_embedding(w.device, w.dtype, w.sizes[0], w.sizes[1], wc.ref.data,
                                                 idx.dtype, numel(ic.ref), ic.ref.data, out.ref().data));
        }
        return out;
    });
}

int tp_amd_embedding_dense_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* indices,
                                    int64_t num_weights, int64_t padding_idx, int scale_grad_by_freq,
                                    tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        const TensorRef& g = deref(grad_output, "grad_output");
        const TensorRef& idx = deref(indices, "indices");
        if (!native_float(g) || !index_tensor(idx) || g.ndim < 1 || g.device != idx.device) {
            TP_AMD_DECLINE("embedding_dense_backward: not native for these operands");
        }
        const int64_t dim = g.sizes[g.ndim - 1];
        MaybeOwned gc = contiguous_on_device(g);
        MaybeOwned ic = contiguous_on_device(idx);
        const int64_t n = numel(ic.ref);
        TP_AMD_CHECK(numel(gc.ref) == n * dim, "embedding_dense_backward: ", n, " indices but a gradient of ",
                     numel(gc.ref), " elements with rows of ", dim);
        TP_AMD_CHECK(num_weights >= 0, "embedding_dense_backward: negative num_weights");
        Owned out = empty_on({num_weights, dim}, g.dtype, g.device);
        if (numel(out.ref()) > 0) {
            check_status(tp_amd_launch_embedding_backward(g.device, g.dtype, n, dim, gc.ref.data, idx.dtype,
                                                          ic.ref.data, num_weights, padding_idx,
                                                          scale_grad_by_freq, out.ref().data));
        }
        return out;
    });
}

int tp_amd_nll_loss(const tp_amd_tensor* self, const tp_amd_tensor* target, const tp_amd_tensor* weight,
                    int64_t reduction, int64_t ignore_index, tp_amd_tensor* output,
                    tp_amd_tensor* total_weight) {
    return guarded_results({output, total_weight}, [&] {
        const TensorRef& x = deref(self, "self");
        const TensorRef& t = deref(target, "target");
        // (N, C) input with (N) targets on one device (nll_native, :327-333).
        const bool native = reduction >= 0 && reduction <= 2 && native_float(x) && x.ndim == 2 &&
                            index_tensor(t) && t.ndim == 1 && t.sizes[0] == x.sizes[0] && numel(x) > 0 &&
                            x.device == t.device && usable_param(weight, x) &&
                            (weight == nullptr || numel(*weight) == x.sizes[1]);
        if (!native) TP_AMD_DECLINE("nll_loss: not native for these operands");
        const int64_t n = x.sizes[0], c = x.sizes[1];
        MaybeOwned xc = contiguous_on_device(x);
        MaybeOwned tc = contiguous_on_device(t);
        MaybeOwned wc;
        if (weight != nullptr) wc = contiguous_on_device(*weight);
        Owned y = empty_on(reduction == 0 ? Sizes{n} : Sizes{}, x.dtype, x.device);
        // A per-sample result of a batch reports no total (:357-358).
        Owned total = filled({}, x.dtype, x.device, 0.0);
        check_status(tp_amd_launch_nll_loss(x.device, x.dtype, n, c, xc.ref.data, t.dtype, tc.ref.data,
                                            weight ? wc.ref.data : nullptr, static_cast<int>(reduction),
                                            ignore_index, y.ref().data, total.ref().data));
        *output = y.release();
        *total_weight = total.release();
    });
}

int tp_amd_nll_loss_backward(const tp_amd_tensor* grad_output, const tp_amd_tensor* self,
                             const tp_amd_tensor* target, const tp_amd_tensor* weight, int64_t reduction,
                             int64_t ignore_index, const tp_amd_tensor* total_weight, tp_amd_tensor* result) {
    return guarded_result(result, [&] {
        const TensorRef& g = deref(grad_output, "grad_output");
        const TensorRef& x = deref(self, "self");
        const TensorRef& t = deref(target, "target");
        const TensorRef& tw = deref(total_weight, "total_weight");
        const bool native = reduction >= 0 && reduction <= 2 && native_float(x) && x.ndim == 2 &&
                            index_tensor(t) && t.ndim == 1 && t.sizes[0] == x.sizes[0] && numel(x) > 0 &&
                            x.device == t.device && usable_param(weight, x) &&
                            (weight == nullptr || numel(*weight) == x.sizes[1]) && on_device(g) &&
                            g.dtype == x.dtype && on_device(tw) &&
                            numel(g) == (reduction == 0 ? x.sizes[0] : 1);
        if (!native) TP_AMD_DECLINE("nll_loss_backward: not native for these operands");
        const int64_t n = x.sizes[0], c = x.sizes[1];
        MaybeOwned gc = contiguous_on_device(g);
        MaybeOwned tc = contiguous_on_device(t);
        MaybeOwned wc;
        if (weight != nullptr) wc = contiguous_on_device(*weight);
        // The total in the input dtype (:377).
        MaybeOwned tot = to_dtype(tw, x.dtype);
        MaybeOwned totc = contiguous_on_device(tot.ref);
        Owned dx = empty_on({n, c}, x.dtype, x.device);
        check_status(tp_amd_launch_nll_loss_backward(x.device, x.dtype, n, c, gc.ref.data, t.dtype, tc.ref.data,
                                                     weight ? wc.ref.data : nullptr, static_cast<int>(reduction),
                                                     ignore_index, totc.ref.data, dx.ref().data));
        return dx;
    });
}

}  // extern "C"
