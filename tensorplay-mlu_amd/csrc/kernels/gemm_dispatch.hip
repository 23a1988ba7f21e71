// GEMM dispatch: dtype selection over the GEMM kernels.

#include "device_common.h"
#include "gemm.h"
#include "../common.h"

namespace tp_amd {

void launch_gemm(int dtype, const GemmArgs& p, hipStream_t stream) {
    switch (dtype) {
        case TP_AMD_FLOAT32: launch_gemm_general<float>(p, stream); break;
        case TP_AMD_BFLOAT16: launch_gemm_general<bf16_t>(p, stream); break;
        case TP_AMD_FLOAT16: launch_gemm_general<f16_t>(p, stream); break;
        default:
            TP_AMD_CHECK(false, "GEMM takes float32, float16 or bfloat16, got ", dtype_name(dtype));
    }
}

}  // namespace tp_amd
