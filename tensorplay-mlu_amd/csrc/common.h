// Internal error handling shared by the runtime, allocator, kernels and the
// operator layer.  Inside the library failures are C++ exceptions; the
// extern "C" entry points turn them into status codes (guarded()), so no
// exception crosses the C boundary (the reference's rule for its C entries,
// tensorplay_mlu/csrc/Cncl.cpp:4-9, GraphCapture.cpp:38-57).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <sstream>
#include <stdexcept>
#include <string>

#include "tp_amd_types.h"

namespace tp_amd {

// A real failure: bad arguments, a HIP error, out of memory.
struct Error : std::runtime_error {
    explicit Error(const std::string& what) : std::runtime_error(what) {}
};

// The device path does not handle these arguments; nothing has been written
// and the caller runs the operator on the host (the reference's
// TP_CNNL_TRY / std::nullopt convention, MLURuntime.h:34-51).
struct Declined {
    const char* reason;
};

template <typename... Args>
std::string concat(const Args&... args) {
    std::ostringstream os;
    (os << ... << args);
    return os.str();
}

#define TP_AMD_CHECK(cond, ...)                                                  \
    do {                                                                         \
        if (!(cond)) throw ::tp_amd::Error(::tp_amd::concat(__VA_ARGS__));      \
    } while (0)

#define TP_AMD_HIP_CHECK(expr)                                                   \
    do {                                                                         \
        const hipError_t tp_amd_status = (expr);                                 \
        if (tp_amd_status != hipSuccess)                                         \
            throw ::tp_amd::Error(::tp_amd::concat("HIP error: ",               \
                                                   hipGetErrorString(tp_amd_status), \
                                                   " (", #expr, ")"));           \
    } while (0)

#define TP_AMD_DECLINE(reason) throw ::tp_amd::Declined{reason}

// Thread-local last error message (tp_mlu_last_error).
void set_last_error(const std::string& message);
const char* last_error();

// Run ``body`` and map its outcome to a status code.
template <typename Body>
int guarded(Body&& body) noexcept {
    try {
        body();
        set_last_error("");
        return TP_AMD_OK;
    } catch (const Declined& d) {
        set_last_error(d.reason ? d.reason : "declined");
        return TP_AMD_DECLINED;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return TP_AMD_ERROR;
    } catch (...) {
        set_last_error("unknown error");
        return TP_AMD_ERROR;
    }
}

// Element size in bytes (0 for an unknown code).
inline int element_size(int dtype) {
    switch (dtype) {
        case TP_AMD_FLOAT32: return 4;
        case TP_AMD_FLOAT16: return 2;
        case TP_AMD_BFLOAT16: return 2;
        case TP_AMD_FLOAT64: return 8;
        case TP_AMD_INT8: return 1;
        case TP_AMD_INT16: return 2;
        case TP_AMD_INT32: return 4;
        case TP_AMD_INT64: return 8;
        case TP_AMD_UINT8: return 1;
        case TP_AMD_BOOL: return 1;
        default: return 0;
    }
}

inline bool is_native_float(int dtype) {
    return dtype == TP_AMD_FLOAT32 || dtype == TP_AMD_FLOAT16 || dtype == TP_AMD_BFLOAT16;
}

inline bool is_floating(int dtype) { return is_native_float(dtype) || dtype == TP_AMD_FLOAT64; }

const char* dtype_name(int dtype);

}  // namespace tp_amd
