// Host-side index-space preparation for the elementwise and copy kernels:
// merging dimensions that are laid out back to back in every operand and
// dropping size-1 dimensions, so most launches see one or two dimensions.
// (The reference does the same to fit CNNL's descriptor limit,
// tensorplay_mlu/csrc/Cnnl.cpp:127-150.)
#pragma once

#include <cstdint>

#include "../common.h"
#include "device_common.h"

namespace tp_amd {

template <int NOPS>
struct Layout {
    int ndim = 0;
    int64_t sizes[TP_AMD_MAX_DIMS] = {};
    int64_t strides[NOPS][TP_AMD_MAX_DIMS] = {};

    int64_t numel() const {
        int64_t n = 1;
        for (int d = 0; d < ndim; ++d) n *= sizes[d];
        return n;
    }
};

// Build a layout over ``ndim`` dims with each operand's strides, then drop
// size-1 dims and merge dim d into d+1 when, for every operand,
// stride[d] == stride[d+1] * size[d+1].  Dims stay outermost-first.
template <int NOPS>
Layout<NOPS> coalesce(int ndim, const int64_t* sizes, const int64_t* const* strides) {
    TP_AMD_CHECK(ndim >= 0 && ndim <= TP_AMD_MAX_DIMS, "at most ", TP_AMD_MAX_DIMS,
                 " dimensions are supported, got ", ndim);
    Layout<NOPS> out;
    for (int d = 0; d < ndim; ++d) {
        TP_AMD_CHECK(sizes[d] >= 0, "negative size ", sizes[d]);
        if (sizes[d] == 1) continue;
        if (out.ndim > 0) {
            bool mergeable = true;
            const int last = out.ndim - 1;
            for (int k = 0; k < NOPS; ++k) {
                if (out.strides[k][last] != strides[k][d] * sizes[d]) {
                    mergeable = false;
                    break;
                }
            }
            if (mergeable) {
                out.sizes[last] *= sizes[d];
                for (int k = 0; k < NOPS; ++k) out.strides[k][last] = strides[k][d];
                continue;
            }
        }
        out.sizes[out.ndim] = sizes[d];
        for (int k = 0; k < NOPS; ++k) out.strides[k][out.ndim] = strides[k][d];
        ++out.ndim;
    }
    return out;
}

// Row-major contiguous strides for ``sizes``.
inline void contiguous_strides(int ndim, const int64_t* sizes, int64_t* strides) {
    int64_t s = 1;
    for (int d = ndim - 1; d >= 0; --d) {
        strides[d] = s;
        s *= sizes[d] > 1 ? sizes[d] : 1;
    }
}

// Kernel-side description of a general strided index space (up to 8 dims,
// innermost last), passed by value.
template <int NOPS>
struct NdParams {
    int32_t ndim;
    int64_t sizes[TP_AMD_MAX_DIMS];
    int64_t strides[NOPS][TP_AMD_MAX_DIMS];
};

template <int NOPS>
NdParams<NOPS> nd_params(const Layout<NOPS>& l) {
    NdParams<NOPS> p{};
    p.ndim = l.ndim;
    for (int d = 0; d < l.ndim; ++d) {
        p.sizes[d] = l.sizes[d];
        for (int k = 0; k < NOPS; ++k) p.strides[k][d] = l.strides[k][d];
    }
    return p;
}


}  // namespace tp_amd
