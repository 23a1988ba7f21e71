/* Runtime, device hooks and caching allocator of libtp_amd.so.
 *
 * Each entry states the reference interface it replaces.  The five
 * ``tp_mlu_*`` entries keep the reference's exact names and signatures
 * (tensorplay_mlu/csrc/Module.cpp:15-37, bound by ctypes in
 * tensorplay_mlu/__init__.py:73-76) so the reference's Python loader binds
 * this library unchanged; everything else is ``tp_amd_*``.
 *
 * Ordering: every device has exactly one HIP stream (default priority,
 * non-blocking) and every kernel, device-to-device copy and allocator reuse
 * is ordered on it, as the reference orders everything on one CNRT queue per
 * device (MLURuntime.cpp:81-93, MLUAllocator.cpp:1-6).
 */
#ifndef TP_AMD_RUNTIME_H
#define TP_AMD_RUNTIME_H

#include "tp_amd_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- C entry points with the reference's names (Module.cpp:15-37) ------ */

/* Replaces tp_mlu_init (Module.cpp:15-22).  Initialises the runtime and
 * allocator; returns 0 on success, 1 on failure (the reference's codes).
 * Registering TensorPlay's host fallbacks is done by the TensorPlay adapter
 * (csrc/tensorplay/Module.cpp), which wraps this call. */
int tp_mlu_init(void);

/* Replaces tp_mlu_device_count (Module.cpp:24, MLURuntime.cpp:34-41):
 * visible devices, 0 when no driver or GPU is present. */
int tp_mlu_device_count(void);

/* Replaces tp_mlu_memory_stats (Module.cpp:27-33): out[0..3] = allocated,
 * reserved, peak allocated, peak reserved bytes of device ``index``. */
void tp_mlu_memory_stats(int index, int64_t* out);

/* Replaces tp_mlu_reset_peak_memory_stats (Module.cpp:35). */
void tp_mlu_reset_peak_memory_stats(int index);

/* Replaces tp_mlu_empty_cache (Module.cpp:37, MLUAllocator.cpp:208-219):
 * synchronizes each device's stream, then returns cached unused blocks. */
void tp_mlu_empty_cache(void);

/* Replaces tp_mlu_last_error (bound at tensorplay_mlu/__init__.py:77):
 * the calling thread's last error message ("" when none). */
const char* tp_mlu_last_error(void);

/* ---- recording and replay (GraphCapture.cpp:38-130) --------------------- */

/* Replace tp_mlu_capture_* (GraphCapture.cpp:59-129, bound at
 * tensorplay_mlu/__init__.py:81-92), one recording per process, on a
 * device's stream as a HIP graph.  begin drains the stream and starts
 * recording; end stops it, sets aside the blocks handed out meanwhile and
 * instantiates the graph (an error when the recorded step did host work);
 * invoke queues one replay; reset drops the recording and returns its
 * blocks.  Return 0, or -1 with the message in tp_mlu_last_error. */
int tp_mlu_capture_begin(int index);
int tp_mlu_capture_end(int index);
int tp_mlu_capture_invoke(int index);
int tp_mlu_capture_reset(void);
/* 1 when a recording is held and can be invoked (GraphCapture.cpp:62). */
int tp_mlu_capture_ready(void);
/* out[0]: blocks handed out while the last recording ran; out[1]: blocks
 * set aside for recordings (GraphCapture.cpp:65-68). */
void tp_mlu_capture_stats(int64_t* out);
/* No counterpart in the reference: how the held recording is replayed.  The
 * number of kernels tp_mlu_capture_invoke launches one by one (a chain of at
 * most 16 kernel nodes), or 0 when it launches the HIP graph (longer
 * recordings, or ones holding copies, events or branches; also when none is
 * held). */
int tp_amd_capture_direct_kernels(void);

/* ---- device hooks (MLUHooks.cpp:14-52, MLURuntime.cpp:43-136) ---------- */

/* PrivateUse1HooksInterface::is_available (MLUHooks.cpp:15). */
int tp_amd_is_available(void);
/* current_device / set_device (MLUHooks.cpp:17-18, MLURuntime.cpp:43-54). */
int tp_amd_current_device(int* index);
int tp_amd_set_device(int index);
/* synchronize (MLUHooks.cpp:19-21, MLURuntime.cpp:107-110): waits for the
 * device's stream; index < 0 means the current device. */
int tp_amd_synchronize(int index);
/* memory_info (MLUHooks.cpp:46-51): free and total bytes from the driver. */
int tp_amd_mem_get_info(int index, size_t* free_bytes, size_t* total_bytes);
/* The device's compute units (the figure the kernels size their grids by;
 * stands where the reference's capability() query does,
 * MLURuntime.cpp:54-67); index < 0 means the current device. */
int tp_amd_compute_units(int index, int* units);
/* copy_bytes (MLUHooks.cpp:23-44): device -1 is host memory.  Host copies
 * return once the bytes have landed (MLURuntime.cpp:112-129); a copy on one
 * device is ordered on its stream; between two devices it bounces through
 * the host. */
int tp_amd_copy_bytes(void* dst, int dst_device, const void* src, int src_device,
                      size_t nbytes);
/* The device's single stream as an opaque handle (hipStream_t), for callers
 * that need to order their own work with this library's
 * (MLURuntime.cpp:81-93 queue()). */
int tp_amd_stream(int index, void** stream);

/* ---- caching allocator (MLUAllocator.cpp:61-236) ------------------------ */

/* Allocator::allocate (MLUAllocator.cpp:63-73, take :98-128): a block of at
 * least ``nbytes`` on ``device`` (< 0: current).  ``*ptr`` is its address,
 * ``*ctx`` the handle tp_amd_free takes (both NULL for nbytes == 0).  Sizes
 * round up to 512 B below 1 MiB and to 2 MiB above; a cached block is reused
 * when it is no more than a quarter larger than the rounded request; on
 * out-of-memory the cache is released and the allocation retried once. */
int tp_amd_malloc(size_t nbytes, int device, void** ptr, void** ctx);
/* The DataPtr deleter (MLUAllocator.cpp:93-96, give_back :130-141): the
 * block returns to its device's pool for reuse by later work on the same
 * stream.  NULL is ignored. */
void tp_amd_free(void* ctx);
/* Size in bytes of the block behind ``ctx`` (after rounding). */
size_t tp_amd_block_size(void* ctx);

/* ---- timing on the device's stream (hipEvent pairs) --------------------- */

/* Events recorded on the device's single stream, so a measurement brackets
 * exactly this library's kernels (reference counterpart: the notifier pair
 * of MLUProfiler.cpp:20-51). */
int tp_amd_event_create(void** event);
int tp_amd_event_record(void* event, int device);
int tp_amd_event_elapsed_ms(void* start, void* stop, float* ms);
int tp_amd_event_destroy(void* event);

/* ---- profiler hooks (MLUProfiler.cpp:20-80, MLUActivity.cpp:87-258) ----- */

/* Per-operation device time; replaces the notifier timer of
 * MLUProfiler.cpp:20-51 (TensorPlay's prof::DeviceTimerHooks).  record
 * places a pooled event on the device's stream; *marker is NULL when the
 * device is out of range or the event cannot be placed (the hook then
 * reports no time).  elapsed_ms waits for `end` and gives the milliseconds
 * between two markers.  release returns a marker to the pool (NULL is
 * ignored). */
int tp_amd_timer_record(int device, void** marker);
int tp_amd_timer_elapsed_ms(void* start, void* end, float* ms);
void tp_amd_timer_release(void* marker);

/* Copy directions of tp_amd_activity.copy_kind. */
enum { TP_AMD_COPY_OTHER = 0, TP_AMD_COPY_HTOD = 1, TP_AMD_COPY_DTOH = 2, TP_AMD_COPY_DTOD = 3 };
/* tp_amd_activity.external_id when the launching thread had none pushed. */
#define TP_AMD_NO_EXTERNAL UINT64_MAX

/* One kernel ('k') or copy ('m') the GPU ran during a tracing session,
 * with the fields of TensorPlay's prof::GpuActivity that the reference's
 * CNPAPI collector fills (MLUActivity.cpp:126-176, 233-247).  Times are on
 * std::chrono::steady_clock, in nanoseconds. */
typedef struct tp_amd_activity {
    const char* name;       /* kernel symbol, or "Memcpy HtoD" / "DtoH" / "DtoD" */
    char kind;              /* 'k' kernel, 'm' copy */
    uint8_t copy_kind;      /* TP_AMD_COPY_* for copies */
    uint64_t start_ns, end_ns;
    uint64_t external_id;   /* the id pushed around the launch, or TP_AMD_NO_EXTERNAL */
    uint32_t correlation;   /* the runtime's correlation id */
    int32_t device;         /* GPU index (-1 unknown) */
    int32_t stream;         /* queue index in order of first appearance (-1 for copies) */
    uint64_t bytes;         /* bytes copied (copies) */
} tp_amd_activity;

/* Kernel-level tracing; replaces the CNPAPI collector of
 * MLUActivity.cpp:87-258 (TensorPlay's prof::DeviceActivityHooks) with
 * rocprofiler-sdk buffer tracing.  Available when the process starts with
 * TP_AMD_DEVICE_TRACE=1 (the SDK takes a tool only before the HIP runtime
 * starts; it is opened with dlopen); otherwise start fails and
 * tp_amd_activity_error says why, and a session reports per-operation
 * time only.  stop waits for the session's work, then hands out the
 * records, valid until the next start.  push/pop bracket the launches of
 * one operation with its id (a no-op while tracing is unavailable). */
int tp_amd_activity_start(void);
int tp_amd_activity_stop(const tp_amd_activity** records, size_t* count);
int tp_amd_activity_push_external(uint64_t id);
int tp_amd_activity_pop_external(void);
const char* tp_amd_activity_error(void);

#ifdef __cplusplus
}
#endif

#endif /* TP_AMD_RUNTIME_H */
