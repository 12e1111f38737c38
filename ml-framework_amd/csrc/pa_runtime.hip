// pa_runtime.hip -- device, memory, stream, event and error entry points of the C-ABI.
//
// These back the reference HAL interfaces (src/MLFramework/HAL/IDevice.cs, IMemoryAllocator.cs,
// IStream.cs, IEvent.cs) for a ROCm device, replacing the P/Invoke surface the CUDA HAL declares
// against nvcuda.dll (src/MLFramework/HAL/CUDA/CudaApi.cs:18-128).
#include <cstdio>
#include <cstring>
#include <new>

#include "pa_internal.h"

namespace {
thread_local std::string g_last_error;

// RAII guard that makes `ordinal` the current device and restores the previous one.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int ordinal) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != ordinal) err = hipSetDevice(ordinal);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};
}  // namespace

namespace pa {

pa_status set_error(pa_status st, const std::string& msg) {
    g_last_error = msg;
    return st;
}

pa_status set_hip_error(hipError_t err, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
    return err == hipErrorOutOfMemory ? PA_ERROR_OUT_OF_MEMORY : PA_ERROR_HIP;
}

pa_status clear_error() {
    g_last_error.clear();
    return PA_SUCCESS;
}

pa_status check_config(const pa_config* cfg, const char* fn) {
    std::string f(fn);
    if (!cfg) return set_error(PA_ERROR_INVALID_ARGUMENT, f + ": cfg is null");
    if (cfg->block_size != kBlockSize)
        return set_error(PA_ERROR_UNSUPPORTED, f + ": block_size must be 16");
    if (cfg->num_q_heads <= 0 || cfg->num_kv_heads <= 0 || cfg->num_q_heads % cfg->num_kv_heads != 0)
        return set_error(PA_ERROR_INVALID_CONFIG,
                         f + ": num_q_heads must be a positive multiple of num_kv_heads");
    if (cfg->head_dim != 32 && cfg->head_dim != 64 && cfg->head_dim != 128 && cfg->head_dim != 256)
        return set_error(PA_ERROR_UNSUPPORTED, f + ": head_dim must be 32, 64, 128 or 256");
    if (cfg->kv_dtype != PA_DTYPE_FP32 && cfg->kv_dtype != PA_DTYPE_BF16 && cfg->kv_dtype != PA_DTYPE_INT8)
        return set_error(PA_ERROR_UNSUPPORTED, f + ": kv_dtype must be FP32, BF16 or INT8");
    // int8 codes meet the int8 MFMA (64 dims per instruction) and 64-lane quantiser rows.
    if (cfg->kv_dtype == PA_DTYPE_INT8 && cfg->head_dim < 64)
        return set_error(PA_ERROR_UNSUPPORTED, f + ": int8 caches take head_dim 64, 128 or 256");
    if (cfg->q_dtype != PA_DTYPE_FP32 && cfg->q_dtype != PA_DTYPE_BF16)
        return set_error(PA_ERROR_UNSUPPORTED, f + ": q_dtype must be FP32 or BF16");
    if (cfg->num_blocks < 0) return set_error(PA_ERROR_INVALID_CONFIG, f + ": num_blocks < 0");
    if (!(cfg->scale == cfg->scale)) return set_error(PA_ERROR_INVALID_CONFIG, f + ": scale is NaN");
    return PA_SUCCESS;
}

}  // namespace pa

using pa::set_error;

extern "C" {

pa_status pa_get_version(int32_t* major, int32_t* minor) {
    if (!major || !minor) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_get_version: null argument");
    *major = PA_API_VERSION_MAJOR;
    *minor = PA_API_VERSION_MINOR;
    return PA_SUCCESS;
}

const char* pa_status_string(pa_status status) {
    switch (status) {
        case PA_SUCCESS: return "PA_SUCCESS";
        case PA_ERROR_INVALID_ARGUMENT: return "PA_ERROR_INVALID_ARGUMENT";
        case PA_ERROR_INVALID_CONFIG: return "PA_ERROR_INVALID_CONFIG";
        case PA_ERROR_OUT_OF_MEMORY: return "PA_ERROR_OUT_OF_MEMORY";
        case PA_ERROR_HIP: return "PA_ERROR_HIP";
        case PA_ERROR_UNSUPPORTED: return "PA_ERROR_UNSUPPORTED";
        case PA_ERROR_WORKSPACE_TOO_SMALL: return "PA_ERROR_WORKSPACE_TOO_SMALL";
        case PA_ERROR_NO_DEVICE: return "PA_ERROR_NO_DEVICE";
    }
    return "PA_ERROR_UNKNOWN";
}

pa_status pa_get_last_error(char* buf, size_t buf_len) {
    if (!buf || buf_len == 0) return PA_ERROR_INVALID_ARGUMENT;
    size_t n = g_last_error.size() < buf_len - 1 ? g_last_error.size() : buf_len - 1;
    memcpy(buf, g_last_error.data(), n);
    buf[n] = '\0';
    return PA_SUCCESS;
}

// ---- device ------------------------------------------------------------------------------------
pa_status pa_device_count(int32_t* count) {
    if (!count) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_device_count: count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) n = 0;
    else if (e != hipSuccess) return pa::set_hip_error(e, "hipGetDeviceCount");
    *count = n;
    return PA_SUCCESS;
}

pa_status pa_device_open(int32_t ordinal, pa_device** out_device) {
    if (!out_device) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_device_open: out_device is null");
    *out_device = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || ordinal < 0 || ordinal >= n)
        return set_error(PA_ERROR_NO_DEVICE, "pa_device_open: no HIP device with ordinal " + std::to_string(ordinal));
    // CudaDevice's constructor makes its device current (HAL/CUDA/CudaDevice.cs:15-21).
    PA_HIP_CHECK(hipSetDevice(ordinal));
    // Per-device set-up: the scratch address of pa_paged_decode_noalloc.
    pa_status st = pa::init_decode_scratch(ordinal);
    if (st != PA_SUCCESS) return st;
    auto* d = new (std::nothrow) pa_device{ordinal};
    if (!d) return set_error(PA_ERROR_OUT_OF_MEMORY, "pa_device_open: host allocation failed");
    *out_device = d;
    return PA_SUCCESS;
}

pa_status pa_device_close(pa_device* device) {
    if (!device) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_device_close: device is null");
    delete device;
    return PA_SUCCESS;
}

pa_status pa_device_get_props(const pa_device* device, pa_device_props* props) {
    if (!device || !props) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_device_get_props: null argument");
    hipDeviceProp_t p;
    PA_HIP_CHECK(hipGetDeviceProperties(&p, device->ordinal));
    memset(props, 0, sizeof(*props));
    snprintf(props->name, sizeof(props->name), "%s", p.name);
    snprintf(props->arch, sizeof(props->arch), "%s", p.gcnArchName);
    props->total_memory = p.totalGlobalMem;
    props->compute_units = p.multiProcessorCount;
    props->ordinal = device->ordinal;
    return PA_SUCCESS;
}

pa_status pa_device_synchronize(pa_device* device) {
    if (!device) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_device_synchronize: device is null");
    DeviceGuard g(device->ordinal);
    if (g.err != hipSuccess) return pa::set_hip_error(g.err, "hipSetDevice");
    PA_HIP_CHECK(hipDeviceSynchronize());
    return PA_SUCCESS;
}

// ---- memory ------------------------------------------------------------------------------------
pa_status pa_alloc(pa_device* device, size_t bytes, void** dptr) {
    if (!device || !dptr) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_alloc: null argument");
    *dptr = nullptr;
    if (bytes == 0) return PA_SUCCESS;
    DeviceGuard g(device->ordinal);
    if (g.err != hipSuccess) return pa::set_hip_error(g.err, "hipSetDevice");
    PA_HIP_CHECK(hipMalloc(dptr, bytes));
    return PA_SUCCESS;
}

pa_status pa_free(pa_device* device, void* dptr) {
    if (!device) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_free: device is null");
    if (!dptr) return PA_SUCCESS;
    DeviceGuard g(device->ordinal);
    if (g.err != hipSuccess) return pa::set_hip_error(g.err, "hipSetDevice");
    PA_HIP_CHECK(hipFree(dptr));
    return PA_SUCCESS;
}

pa_status pa_memcpy(void* dst, const void* src, size_t bytes, int32_t kind, pa_stream* stream) {
    if (bytes == 0) return PA_SUCCESS;
    if (!dst || !src) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_memcpy: null pointer");
    if (kind < PA_MEMCPY_HOST_TO_HOST || kind > PA_MEMCPY_DEFAULT)
        return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_memcpy: bad kind");
    hipMemcpyKind k = static_cast<hipMemcpyKind>(kind);  // enumerators coincide with hipMemcpyKind
    if (stream) PA_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, k, stream->stream));
    else PA_HIP_CHECK(hipMemcpy(dst, src, bytes, k));
    return PA_SUCCESS;
}

pa_status pa_memset(void* dst, int32_t value, size_t bytes, pa_stream* stream) {
    if (bytes == 0) return PA_SUCCESS;
    if (!dst) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_memset: null pointer");
    if (stream) {
        // Memset nodes in a captured graph have given wrong results on replays after the first
        // on this platform, so a capturing stream is refused (clear memory with a kernel instead).
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        PA_HIP_CHECK(hipStreamIsCapturing(stream->stream, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_memset: the stream is capturing a graph; "
                                                        "memset nodes are not recorded");
        PA_HIP_CHECK(hipMemsetAsync(dst, value, bytes, stream->stream));
    }
    else PA_HIP_CHECK(hipMemset(dst, value, bytes));
    return PA_SUCCESS;
}

// ---- streams -----------------------------------------------------------------------------------
pa_status pa_stream_create(pa_device* device, pa_stream** out_stream) {
    if (!device || !out_stream) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_stream_create: null argument");
    *out_stream = nullptr;
    DeviceGuard g(device->ordinal);
    if (g.err != hipSuccess) return pa::set_hip_error(g.err, "hipSetDevice");
    hipStream_t s = nullptr;
    // Default priority only: streams of other priorities are not used by this library.
    PA_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    auto* ps = new (std::nothrow) pa_stream{device->ordinal, s, true};
    if (!ps) {
        (void)hipStreamDestroy(s);
        return set_error(PA_ERROR_OUT_OF_MEMORY, "pa_stream_create: host allocation failed");
    }
    *out_stream = ps;
    return PA_SUCCESS;
}

pa_status pa_stream_wrap(pa_device* device, void* hip_stream, pa_stream** out_stream) {
    if (!device || !out_stream) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_stream_wrap: null argument");
    auto* ps = new (std::nothrow) pa_stream{device->ordinal, static_cast<hipStream_t>(hip_stream), false};
    if (!ps) return set_error(PA_ERROR_OUT_OF_MEMORY, "pa_stream_wrap: host allocation failed");
    *out_stream = ps;
    return PA_SUCCESS;
}

pa_status pa_stream_native(const pa_stream* stream, void** hip_stream) {
    if (!stream || !hip_stream) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_stream_native: null argument");
    *hip_stream = stream->stream;
    return PA_SUCCESS;
}

pa_status pa_stream_destroy(pa_stream* stream) {
    if (!stream) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_stream_destroy: stream is null");
    hipError_t e = hipSuccess;
    if (stream->owned && stream->stream) e = hipStreamDestroy(stream->stream);
    delete stream;
    if (e != hipSuccess) return pa::set_hip_error(e, "hipStreamDestroy");
    return PA_SUCCESS;
}

pa_status pa_stream_synchronize(pa_stream* stream) {
    if (!stream) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_stream_synchronize: stream is null");
    PA_HIP_CHECK(hipStreamSynchronize(stream->stream));
    return PA_SUCCESS;
}

pa_status pa_stream_wait_event(pa_stream* stream, pa_event* event) {
    if (!stream || !event) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_stream_wait_event: null argument");
    PA_HIP_CHECK(hipStreamWaitEvent(stream->stream, event->event, 0));
    return PA_SUCCESS;
}

// ---- events ------------------------------------------------------------------------------------
pa_status pa_event_create(pa_device* device, pa_event** out_event) {
    if (!device || !out_event) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_event_create: null argument");
    *out_event = nullptr;
    DeviceGuard g(device->ordinal);
    if (g.err != hipSuccess) return pa::set_hip_error(g.err, "hipSetDevice");
    hipEvent_t e = nullptr;
    PA_HIP_CHECK(hipEventCreate(&e));
    auto* pe = new (std::nothrow) pa_event{device->ordinal, e};
    if (!pe) {
        (void)hipEventDestroy(e);
        return set_error(PA_ERROR_OUT_OF_MEMORY, "pa_event_create: host allocation failed");
    }
    *out_event = pe;
    return PA_SUCCESS;
}

pa_status pa_event_destroy(pa_event* event) {
    if (!event) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_event_destroy: event is null");
    hipError_t e = hipEventDestroy(event->event);
    delete event;
    if (e != hipSuccess) return pa::set_hip_error(e, "hipEventDestroy");
    return PA_SUCCESS;
}

pa_status pa_event_record(pa_event* event, pa_stream* stream) {
    if (!event) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_event_record: event is null");
    PA_HIP_CHECK(hipEventRecord(event->event, pa::native(stream)));
    return PA_SUCCESS;
}

pa_status pa_event_query(pa_event* event, int32_t* completed) {
    if (!event || !completed) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_event_query: null argument");
    hipError_t e = hipEventQuery(event->event);
    if (e == hipSuccess) *completed = 1;
    else if (e == hipErrorNotReady) *completed = 0;
    else return pa::set_hip_error(e, "hipEventQuery");
    return PA_SUCCESS;
}

pa_status pa_event_synchronize(pa_event* event) {
    if (!event) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_event_synchronize: event is null");
    PA_HIP_CHECK(hipEventSynchronize(event->event));
    return PA_SUCCESS;
}

pa_status pa_event_elapsed_ms(pa_event* start, pa_event* end, float* ms) {
    if (!start || !end || !ms) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_event_elapsed_ms: null argument");
    PA_HIP_CHECK(hipEventElapsedTime(ms, start->event, end->event));
    return PA_SUCCESS;
}

// ---- graphs ------------------------------------------------------------------------------------
pa_status pa_graph_capture_begin(pa_stream* stream) {
    if (!stream) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_graph_capture_begin: stream is null");
    PA_HIP_CHECK(hipStreamBeginCapture(stream->stream, hipStreamCaptureModeThreadLocal));
    return PA_SUCCESS;
}

pa_status pa_graph_capture_end(pa_stream* stream, pa_graph** out_graph) {
    if (!stream || !out_graph) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_graph_capture_end: null argument");
    *out_graph = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(stream->stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return pa::set_hip_error(e, "hipStreamEndCapture");
    }
    if (!g) return set_error(PA_ERROR_HIP, "pa_graph_capture_end: the capture produced no graph");
    size_t nodes = 0;
    e = hipGraphGetNodes(g, nullptr, &nodes);
    hipGraphExec_t x = nullptr;
    if (e == hipSuccess) e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return pa::set_hip_error(e, "hipGraphInstantiate");
    }
    auto* pg = new (std::nothrow) pa_graph{stream->ordinal, g, x, nodes};
    if (!pg) {
        (void)hipGraphExecDestroy(x);
        (void)hipGraphDestroy(g);
        return set_error(PA_ERROR_OUT_OF_MEMORY, "pa_graph_capture_end: host allocation failed");
    }
    *out_graph = pg;
    return PA_SUCCESS;
}

pa_status pa_graph_launch(pa_graph* graph, pa_stream* stream) {
    if (!graph) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_graph_launch: graph is null");
    PA_HIP_CHECK(hipGraphLaunch(graph->exec, pa::native(stream)));
    return PA_SUCCESS;
}

pa_status pa_graph_node_count(const pa_graph* graph, size_t* count) {
    if (!graph || !count) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_graph_node_count: null argument");
    *count = graph->nodes;
    return PA_SUCCESS;
}

pa_status pa_graph_destroy(pa_graph* graph) {
    if (!graph) return set_error(PA_ERROR_INVALID_ARGUMENT, "pa_graph_destroy: graph is null");
    hipError_t e = hipGraphExecDestroy(graph->exec);
    const hipError_t e2 = hipGraphDestroy(graph->graph);
    delete graph;
    if (e == hipSuccess) e = e2;
    if (e != hipSuccess) return pa::set_hip_error(e, "hipGraphDestroy");
    return PA_SUCCESS;
}

}  // extern "C"
