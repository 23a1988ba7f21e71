// Device time for TensorPlay's profiler (the reference's MLUProfiler.cpp and
// MLUActivity.cpp), in two parts:
//
// * Per-operation device time: HIP events placed on the device's single
//   stream before and after an operation.  Events are pooled -- a session
//   records two per operation, and creating one is a runtime call the
//   dispatch path should not pay for each time.
//
// * Kernel-level records: the kernels and copies the GPU ran during a
//   session, from rocprofiler-sdk's buffer tracing, each carrying the
//   external correlation id the launching operation pushed.  rocprofiler-sdk
//   takes a tool only before the HIP runtime starts, so this part is set up
//   when the library loads, and only with TP_AMD_DEVICE_TRACE=1 in the
//   environment; the SDK is opened with dlopen, so the library loads and
//   runs without it.  Otherwise a session reports per-operation device time
//   only, as the reference does without its activity library.

#include <dlfcn.h>

#include <chrono>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>
#include <rocprofiler-sdk/buffer.h>
#include <rocprofiler-sdk/buffer_tracing.h>
#include <rocprofiler-sdk/callback_tracing.h>
#include <rocprofiler-sdk/context.h>
#include <rocprofiler-sdk/external_correlation.h>
#include <rocprofiler-sdk/internal_threading.h>
#include <rocprofiler-sdk/registration.h>
#include <rocprofiler-sdk/rocprofiler.h>

#include "common.h"
#include "runtime.h"
#include "tp_amd_runtime.h"

using namespace tp_amd;

namespace {

// ---- event pool -------------------------------------------------------------

std::mutex pool_mutex;
std::vector<hipEvent_t> event_pool;

hipEvent_t take_event() {
    {
        std::lock_guard<std::mutex> lock(pool_mutex);
        if (!event_pool.empty()) {
            hipEvent_t e = event_pool.back();
            event_pool.pop_back();
            return e;
        }
    }
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

void give_back(hipEvent_t e) {
    std::lock_guard<std::mutex> lock(pool_mutex);
    event_pool.push_back(e);
}

// ---- rocprofiler-sdk tracing ---------------------------------------------------

struct Sdk {
    decltype(&rocprofiler_force_configure) force_configure = nullptr;
    decltype(&rocprofiler_create_context) create_context = nullptr;
    decltype(&rocprofiler_configure_callback_tracing_service) callback_service = nullptr;
    decltype(&rocprofiler_create_buffer) create_buffer = nullptr;
    decltype(&rocprofiler_configure_buffer_tracing_service) buffer_service = nullptr;
    decltype(&rocprofiler_create_callback_thread) create_thread = nullptr;
    decltype(&rocprofiler_assign_callback_thread) assign_thread = nullptr;
    decltype(&rocprofiler_start_context) start_context = nullptr;
    decltype(&rocprofiler_stop_context) stop_context = nullptr;
    decltype(&rocprofiler_flush_buffer) flush_buffer = nullptr;
    decltype(&rocprofiler_push_external_correlation_id) push = nullptr;
    decltype(&rocprofiler_pop_external_correlation_id) pop = nullptr;
    decltype(&rocprofiler_get_thread_id) thread_id = nullptr;
    decltype(&rocprofiler_get_timestamp) timestamp = nullptr;
    decltype(&rocprofiler_query_available_agents) query_agents = nullptr;
};

struct Tracer {
    std::mutex mutex;            // records, names, queues
    Sdk sdk;
    bool configured = false;     // the tool was accepted and its contexts exist
    bool active = false;         // a session is running
    std::string error;           // why tracing is unavailable
    rocprofiler_context_id_t symbols{};  // code-object context, always on
    rocprofiler_context_id_t trace{};    // kernels and copies, on during sessions
    rocprofiler_buffer_id_t buffer{};
    std::unordered_map<uint64_t, std::string> kernel_names;   // kernel id -> symbol
    std::unordered_map<uint64_t, int32_t> gpu_of_agent;       // agent handle -> GPU index
    std::unordered_map<uint64_t, int32_t> queue_index;        // queue handle -> small index
    std::vector<tp_amd_activity> records;
    std::deque<std::string> names;   // names the records point at, until the next start
    int64_t offset_ns = 0;           // steady clock minus the SDK's clock
};

Tracer& tracer() {
    static Tracer* t = new Tracer;  // leaked: the SDK may call back during exit
    return *t;
}

uint64_t steady_ns() {
    return static_cast<uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                     std::chrono::steady_clock::now().time_since_epoch())
                                     .count());
}

const char* copy_name(int kind) {
    switch (kind) {
        case TP_AMD_COPY_HTOD: return "Memcpy HtoD";
        case TP_AMD_COPY_DTOH: return "Memcpy DtoH";
        case TP_AMD_COPY_DTOD: return "Memcpy DtoD";
        default: return "Memcpy";
    }
}

// Called with the tracer's mutex held.
int32_t queue_of(Tracer& t, uint64_t handle) {
    auto it = t.queue_index.find(handle);
    if (it != t.queue_index.end()) return it->second;
    const int32_t q = static_cast<int32_t>(t.queue_index.size());
    t.queue_index.emplace(handle, q);
    return q;
}

int32_t gpu_of(Tracer& t, uint64_t agent) {
    auto it = t.gpu_of_agent.find(agent);
    return it == t.gpu_of_agent.end() ? -1 : it->second;
}

// The pushed id is stored plus one, so 0 means "none pushed".
uint64_t external_of(const rocprofiler_user_data_t& ext) {
    return ext.value == 0 ? TP_AMD_NO_EXTERNAL : ext.value - 1;
}

void on_code_object(rocprofiler_callback_tracing_record_t record, rocprofiler_user_data_t*, void*) {
    if (record.kind != ROCPROFILER_CALLBACK_TRACING_CODE_OBJECT ||
        record.operation != ROCPROFILER_CODE_OBJECT_DEVICE_KERNEL_SYMBOL_REGISTER ||
        record.phase != ROCPROFILER_CALLBACK_PHASE_LOAD) {
        return;
    }
    auto* data = static_cast<rocprofiler_callback_tracing_code_object_kernel_symbol_register_data_t*>(
        record.payload);
    Tracer& t = tracer();
    std::lock_guard<std::mutex> lock(t.mutex);
    t.kernel_names[data->kernel_id] = data->kernel_name ? data->kernel_name : "kernel";
}

void on_records(rocprofiler_context_id_t, rocprofiler_buffer_id_t, rocprofiler_record_header_t** headers,
                size_t count, void*, uint64_t) {
    Tracer& t = tracer();
    std::lock_guard<std::mutex> lock(t.mutex);
    for (size_t i = 0; i < count; ++i) {
        const rocprofiler_record_header_t* h = headers[i];
        if (h->category != ROCPROFILER_BUFFER_CATEGORY_TRACING) continue;
        tp_amd_activity a{};
        if (h->kind == ROCPROFILER_BUFFER_TRACING_KERNEL_DISPATCH) {
            auto* r = static_cast<const rocprofiler_buffer_tracing_kernel_dispatch_record_t*>(h->payload);
            auto name = t.kernel_names.find(r->dispatch_info.kernel_id);
            t.names.emplace_back(name != t.kernel_names.end() ? name->second : std::string("kernel"));
            a.name = t.names.back().c_str();
            a.kind = 'k';
            a.start_ns = static_cast<uint64_t>(static_cast<int64_t>(r->start_timestamp) + t.offset_ns);
            a.end_ns = static_cast<uint64_t>(static_cast<int64_t>(r->end_timestamp) + t.offset_ns);
            a.external_id = external_of(r->correlation_id.external);
            a.correlation = static_cast<uint32_t>(r->correlation_id.internal);
            a.device = gpu_of(t, r->dispatch_info.agent_id.handle);
            a.stream = queue_of(t, r->dispatch_info.queue_id.handle);
        } else if (h->kind == ROCPROFILER_BUFFER_TRACING_MEMORY_COPY) {
            auto* r = static_cast<const rocprofiler_buffer_tracing_memory_copy_record_t*>(h->payload);
            int kind = TP_AMD_COPY_OTHER;
            switch (r->operation) {
                case ROCPROFILER_MEMORY_COPY_HOST_TO_DEVICE: kind = TP_AMD_COPY_HTOD; break;
                case ROCPROFILER_MEMORY_COPY_DEVICE_TO_HOST: kind = TP_AMD_COPY_DTOH; break;
                case ROCPROFILER_MEMORY_COPY_DEVICE_TO_DEVICE: kind = TP_AMD_COPY_DTOD; break;
                default: break;
            }
            a.name = copy_name(kind);
            a.kind = 'm';
            a.copy_kind = static_cast<uint8_t>(kind);
            a.start_ns = static_cast<uint64_t>(static_cast<int64_t>(r->start_timestamp) + t.offset_ns);
            a.end_ns = static_cast<uint64_t>(static_cast<int64_t>(r->end_timestamp) + t.offset_ns);
            a.external_id = external_of(r->correlation_id.external);
            a.correlation = static_cast<uint32_t>(r->correlation_id.internal);
            const int32_t dst = gpu_of(t, r->dst_agent_id.handle);
            a.device = dst >= 0 ? dst : gpu_of(t, r->src_agent_id.handle);
            a.stream = -1;
            a.bytes = r->bytes;
        } else {
            continue;
        }
        t.records.push_back(a);
    }
}

rocprofiler_status_t on_agents(rocprofiler_agent_version_t, const void** agents, size_t count, void*) {
    Tracer& t = tracer();
    std::lock_guard<std::mutex> lock(t.mutex);
    for (size_t i = 0; i < count; ++i) {
        const auto* a = static_cast<const rocprofiler_agent_t*>(agents[i]);
        if (a->type == ROCPROFILER_AGENT_TYPE_GPU) t.gpu_of_agent[a->id.handle] = a->logical_node_type_id;
    }
    return ROCPROFILER_STATUS_SUCCESS;
}

int tool_init(rocprofiler_client_finalize_t, void*) {
    Tracer& t = tracer();
    const Sdk& s = t.sdk;
    auto ok = [&](rocprofiler_status_t status, const char* what) {
        if (status == ROCPROFILER_STATUS_SUCCESS) return true;
        t.error = std::string("rocprofiler-sdk: ") + what + " failed (status " + std::to_string(status) + ")";
        return false;
    };
    rocprofiler_tracing_operation_t symbol_ops[] = {ROCPROFILER_CODE_OBJECT_DEVICE_KERNEL_SYMBOL_REGISTER};
    rocprofiler_callback_thread_t thread{};
    constexpr size_t kBufferBytes = size_t(8) << 20;
    const bool built =
        ok(s.query_agents(ROCPROFILER_AGENT_INFO_VERSION_0, on_agents, sizeof(rocprofiler_agent_t), nullptr),
           "agent query") &&
        ok(s.create_context(&t.symbols), "context creation") &&
        ok(s.callback_service(t.symbols, ROCPROFILER_CALLBACK_TRACING_CODE_OBJECT, symbol_ops, 1, on_code_object,
                              nullptr),
           "code-object tracing") &&
        ok(s.create_context(&t.trace), "context creation") &&
        ok(s.create_buffer(t.trace, kBufferBytes, kBufferBytes - kBufferBytes / 8, ROCPROFILER_BUFFER_POLICY_LOSSLESS,
                           on_records, nullptr, &t.buffer),
           "buffer creation") &&
        ok(s.buffer_service(t.trace, ROCPROFILER_BUFFER_TRACING_KERNEL_DISPATCH, nullptr, 0, t.buffer),
           "kernel-dispatch tracing") &&
        ok(s.buffer_service(t.trace, ROCPROFILER_BUFFER_TRACING_MEMORY_COPY, nullptr, 0, t.buffer),
           "memory-copy tracing") &&
        ok(s.create_thread(&thread), "callback thread") && ok(s.assign_thread(t.buffer, thread), "callback thread") &&
        ok(s.start_context(t.symbols), "code-object context start");
    t.configured = built;
    return built ? 0 : -1;
}

void tool_fini(void*) {}

rocprofiler_tool_configure_result_t* configure(uint32_t, const char*, uint32_t, rocprofiler_client_id_t* id) {
    id->name = "tensorplay-mlu_amd";
    static rocprofiler_tool_configure_result_t result{sizeof(rocprofiler_tool_configure_result_t), tool_init,
                                                     tool_fini, nullptr};
    return &result;
}

// Opens the SDK and hands it the tool, before the HIP runtime starts.
void set_up_tracing() {
    Tracer& t = tracer();
    const char* want = std::getenv("TP_AMD_DEVICE_TRACE");
    if (want == nullptr || std::strcmp(want, "1") != 0) {
        t.error = "kernel-level tracing is off (set TP_AMD_DEVICE_TRACE=1 before the process starts)";
        return;
    }
    // Global, so the runtimes' registration finds the SDK.
    void* lib = dlopen("librocprofiler-sdk.so.1", RTLD_NOW | RTLD_GLOBAL);
    if (lib == nullptr) lib = dlopen("librocprofiler-sdk.so", RTLD_NOW | RTLD_GLOBAL);
    if (lib == nullptr) {
        const char* e = dlerror();
        t.error = std::string("librocprofiler-sdk.so not loadable: ") + (e ? e : "unknown");
        return;
    }
    Sdk& s = t.sdk;
    bool found = true;
    auto bind = [&](auto& fn, const char* name) {
        fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(lib, name));
        if (fn == nullptr) {
            found = false;
            t.error = std::string("librocprofiler-sdk.so lacks ") + name;
        }
    };
    bind(s.force_configure, "rocprofiler_force_configure");
    bind(s.create_context, "rocprofiler_create_context");
    bind(s.callback_service, "rocprofiler_configure_callback_tracing_service");
    bind(s.create_buffer, "rocprofiler_create_buffer");
    bind(s.buffer_service, "rocprofiler_configure_buffer_tracing_service");
    bind(s.create_thread, "rocprofiler_create_callback_thread");
    bind(s.assign_thread, "rocprofiler_assign_callback_thread");
    bind(s.start_context, "rocprofiler_start_context");
    bind(s.stop_context, "rocprofiler_stop_context");
    bind(s.flush_buffer, "rocprofiler_flush_buffer");
    bind(s.push, "rocprofiler_push_external_correlation_id");
    bind(s.pop, "rocprofiler_pop_external_correlation_id");
    bind(s.thread_id, "rocprofiler_get_thread_id");
    bind(s.timestamp, "rocprofiler_get_timestamp");
    bind(s.query_agents, "rocprofiler_query_available_agents");
    if (!found) return;
    const rocprofiler_status_t status = s.force_configure(configure);
    if (status != ROCPROFILER_STATUS_SUCCESS) {
        t.error = "rocprofiler-sdk refused the tool (status " + std::to_string(status) +
                  "); the HIP runtime had probably started before this library loaded";
    }
}

// Runs when the library loads, ahead of any HIP call this library makes.
[[maybe_unused]] const bool tracing_set_up = [] {
    set_up_tracing();
    return true;
}();

}  // namespace

extern "C" {

int tp_amd_timer_record(int device, void** marker) {
    return guarded([&] {
        TP_AMD_CHECK(marker != nullptr, "null marker pointer");
        *marker = nullptr;
        if (device < 0 || device >= device_count()) return;
        hipEvent_t e = take_event();
        if (e == nullptr) return;
        const OnDevice scope(device);
        if (hipEventRecord(e, stream(device)) == hipSuccess) {
            *marker = e;
        } else {
            give_back(e);
        }
    });
}

int tp_amd_timer_elapsed_ms(void* start, void* end, float* ms) {
    return guarded([&] {
        TP_AMD_CHECK(start != nullptr && end != nullptr && ms != nullptr, "null timer argument");
        TP_AMD_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(end)));
        TP_AMD_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
    });
}

void tp_amd_timer_release(void* marker) {
    if (marker != nullptr) give_back(static_cast<hipEvent_t>(marker));
}

int tp_amd_activity_start(void) {
    Tracer& t = tracer();
    return guarded([&] {
        TP_AMD_CHECK(t.configured, t.error);
        std::lock_guard<std::mutex> lock(t.mutex);
        TP_AMD_CHECK(!t.active, "a tracing session is already running");
        t.records.clear();
        t.names.clear();
        // The SDK's clock mapped onto the steady clock operation events use.
        rocprofiler_timestamp_t now = 0;
        const uint64_t before = steady_ns();
        TP_AMD_CHECK(t.sdk.timestamp(&now) == ROCPROFILER_STATUS_SUCCESS, "rocprofiler-sdk timestamp failed");
        const uint64_t after = steady_ns();
        t.offset_ns = static_cast<int64_t>(before + (after - before) / 2) - static_cast<int64_t>(now);
        TP_AMD_CHECK(t.sdk.start_context(t.trace) == ROCPROFILER_STATUS_SUCCESS,
                     "rocprofiler-sdk context start failed");
        t.active = true;
    });
}

int tp_amd_activity_stop(const tp_amd_activity** records, size_t* count) {
    Tracer& t = tracer();
    return guarded([&] {
        TP_AMD_CHECK(records != nullptr && count != nullptr, "null result pointer");
        *records = nullptr;
        *count = 0;
        TP_AMD_CHECK(t.configured, t.error);
        {
            std::lock_guard<std::mutex> lock(t.mutex);
            TP_AMD_CHECK(t.active, "no tracing session is running");
        }
        // Everything launched in the session completes, its records reach
        // the buffer, and the buffer is handed to on_records (which takes
        // the mutex, so it is not held here).
        for (int d = 0; d < device_count(); ++d) TP_AMD_HIP_CHECK(hipStreamSynchronize(stream(d)));
        t.sdk.flush_buffer(t.buffer);
        t.sdk.stop_context(t.trace);
        t.sdk.flush_buffer(t.buffer);
        std::lock_guard<std::mutex> lock(t.mutex);
        t.active = false;
        *records = t.records.data();
        *count = t.records.size();
    });
}

int tp_amd_activity_push_external(uint64_t id) {
    Tracer& t = tracer();
    if (!t.configured) return TP_AMD_OK;
    rocprofiler_thread_id_t tid = 0;
    if (t.sdk.thread_id(&tid) != ROCPROFILER_STATUS_SUCCESS) return TP_AMD_ERROR;
    rocprofiler_user_data_t value{};
    value.value = id + 1;
    return t.sdk.push(t.trace, tid, value) == ROCPROFILER_STATUS_SUCCESS ? TP_AMD_OK : TP_AMD_ERROR;
}

int tp_amd_activity_pop_external(void) {
    Tracer& t = tracer();
    if (!t.configured) return TP_AMD_OK;
    rocprofiler_thread_id_t tid = 0;
    if (t.sdk.thread_id(&tid) != ROCPROFILER_STATUS_SUCCESS) return TP_AMD_ERROR;
    rocprofiler_user_data_t last{};
    return t.sdk.pop(t.trace, tid, &last) == ROCPROFILER_STATUS_SUCCESS ? TP_AMD_OK : TP_AMD_ERROR;
}

const char* tp_amd_activity_error(void) {
    Tracer& t = tracer();
    return t.configured ? "" : t.error.c_str();
}

}  // extern "C"
