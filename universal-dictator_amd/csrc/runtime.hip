// Device-memory, stream and event helpers (include/ud_runtime.h).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/ud_encoder.h"
#include "../../include/ud_runtime.h"

// Defined in encoder.hip: records the message returned by ud_last_error().
int ud_set_error(int code, const char* msg);

static int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return UD_OK;
    char buf[256];
    snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
    return ud_set_error(UD_ERR_HIP, buf);
}

extern "C" UD_API int ud_device_count(int32_t* count) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (count) *count = e == hipSuccess ? n : 0;
    return hip_status(e, "hipGetDeviceCount");
}

extern "C" UD_API int ud_device_arch(char* buf, int32_t len) {
    if (!buf || len < 1) return ud_set_error(UD_ERR_INVALID, "ud_device_arch: bad buffer");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDeviceProperties");
    snprintf(buf, (size_t)len, "%s", p.gcnArchName);
    return UD_OK;
}

extern "C" UD_API int ud_malloc(void** dev, size_t bytes) {
    if (!dev) return ud_set_error(UD_ERR_INVALID, "ud_malloc: null out pointer");
    hipError_t e = hipMalloc(dev, bytes ? bytes : 16);
    if (e != hipSuccess) return ud_set_error(UD_ERR_NOMEM, "ud_malloc: hipMalloc failed");
    return UD_OK;
}
extern "C" UD_API int ud_free(void* dev) { return hip_status(hipFree(dev), "hipFree"); }

extern "C" UD_API int ud_memcpy_htod(void* dst, const void* src, size_t bytes) {
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
    return hip_status(e, "ud_memcpy_htod");
}
extern "C" UD_API int ud_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    return hip_status(e, "ud_memcpy_dtoh");
}
extern "C" UD_API int ud_memcpy_dtod(void* dst, const void* src, size_t bytes) {
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
    return hip_status(e, "ud_memcpy_dtod");
}
extern "C" UD_API int ud_memset(void* dev, int32_t byte, size_t bytes) {
    hipError_t e = hipMemset(dev, byte, bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return hip_status(e, "ud_memset");
}
extern "C" UD_API int ud_device_synchronize(void) { return hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

extern "C" UD_API int ud_hip_stream_create(void** stream) {
    if (!stream) return ud_set_error(UD_ERR_INVALID, "ud_hip_stream_create: null out pointer");
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = s;
    return hip_status(e, "hipStreamCreate");
}
extern "C" UD_API int ud_hip_stream_destroy(void* stream) {
    return hip_status(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
}
extern "C" UD_API int ud_hip_stream_synchronize(void* stream) {
    return hip_status(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
}
extern "C" UD_API int ud_event_create(void** event) {
    if (!event) return ud_set_error(UD_ERR_INVALID, "ud_event_create: null out pointer");
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    *event = ev;
    return hip_status(e, "hipEventCreate");
}
extern "C" UD_API int ud_event_destroy(void* event) {
    return hip_status(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}
extern "C" UD_API int ud_event_record(void* event, void* stream) {
    return hip_status(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)),
                      "hipEventRecord");
}
extern "C" UD_API int ud_event_synchronize(void* event) {
    return hip_status(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
}
extern "C" UD_API int ud_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms) return ud_set_error(UD_ERR_INVALID, "ud_event_elapsed_ms: null out pointer");
    return hip_status(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                      "hipEventElapsedTime");
}

extern "C" UD_API int ud_mem_get_info(size_t* free_bytes, size_t* total_bytes) {
    size_t f = 0, t = 0;
    hipError_t e = hipMemGetInfo(&f, &t);
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return hip_status(e, "hipMemGetInfo");
}

// A captured and instantiated graph (ud_graph_capture_end), owned by the caller.
struct ud_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

extern "C" UD_API int ud_graph_capture_begin(void* stream) {
    if (!stream) return ud_set_error(UD_ERR_INVALID, "ud_graph_capture_begin: the null stream cannot be captured");
    return hip_status(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal),
                      "hipStreamBeginCapture");
}

extern "C" UD_API int ud_graph_capture_end(void* stream, void** graph) {
    if (!stream || !graph) return ud_set_error(UD_ERR_INVALID, "ud_graph_capture_end: null argument");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
    if (e != hipSuccess) return hip_status(e, "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_status(e, "hipGraphInstantiate");
    }
    *graph = new ud_graph{g, x};
    return UD_OK;
}

extern "C" UD_API int ud_graph_launch(void* graph, void* stream) {
    if (!graph) return ud_set_error(UD_ERR_INVALID, "ud_graph_launch: null graph");
    return hip_status(hipGraphLaunch(static_cast<ud_graph*>(graph)->exec, static_cast<hipStream_t>(stream)),
                      "hipGraphLaunch");
}

extern "C" UD_API int ud_graph_destroy(void* graph) {
    if (!graph) return UD_OK;
    ud_graph* g = static_cast<ud_graph*>(graph);
    hipError_t e = hipGraphExecDestroy(g->exec);
    if (e == hipSuccess) e = hipGraphDestroy(g->graph);
    delete g;
    return hip_status(e, "hipGraphDestroy");
}
