// Device memory, stream, event and graph services of the thin C-ABI layer.
// Every function returns 1 on success and 0 on failure (pointer-returning
// ones return NULL) and records the HIP error text for pgpu_last_error().
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include "phonon_gpu.h"

static thread_local char g_error[256];

// pgpu_attention.hip: the static attention partials' per-device address.
extern "C" float *pgpu_attention_static_setup(void);

static int check(hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    snprintf(g_error, sizeof(g_error), "%s: %s", what, hipGetErrorString(e));
    return 0;
}

extern "C" const char *pgpu_last_error(void) { return g_error; }

extern "C" void pgpu_record_error(const char *what) {
    snprintf(g_error, sizeof(g_error), "%s", what ? what : "");
}

extern "C" int pgpu_device_init(void) {
    static int initialized = 0;
    if (initialized) return 1;
    int count = 0;
    if (!check(hipGetDeviceCount(&count), "hipGetDeviceCount")) return 0;
    if (count < 1) {
        snprintf(g_error, sizeof(g_error), "no HIP device visible");
        return 0;
    }
    hipDeviceProp_t prop;
    int device = 0;
    if (!check(hipGetDevice(&device), "hipGetDevice") ||
        !check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"))
        return 0;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_error, sizeof(g_error), "device %s is not gfx950", prop.gcnArchName);
        return 0;
    }
    // The device address of pgpu_attention_static's partials, looked up here
    // once with the device current.
    if (!pgpu_attention_static_setup()) return 0;
    initialized = 1;
    return 1;
}

extern "C" int pgpu_device_name(char *buffer, size_t size) {
    hipDeviceProp_t prop;
    int device = 0;
    if (!buffer || !size || !check(hipGetDevice(&device), "hipGetDevice") ||
        !check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"))
        return 0;
    snprintf(buffer, size, "%s (%s, %d CUs)", prop.name, prop.gcnArchName,
             prop.multiProcessorCount);
    return 1;
}

extern "C" void *pgpu_malloc(size_t bytes) {
    void *p = NULL;
    if (!bytes) bytes = 1;
    if (!check(hipMalloc(&p, bytes), "hipMalloc")) return NULL;
    return p;
}

extern "C" void pgpu_free(void *ptr) {
    if (ptr) (void)hipFree(ptr);
}

extern "C" int pgpu_memset(void *stream, void *dst, int value, size_t bytes) {
    return check(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream), "hipMemsetAsync");
}

extern "C" int pgpu_copy_h2d(void *stream, void *dst, const void *src, size_t bytes) {
    if (!bytes) return 1;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream),
                 "hipMemcpyAsync H2D") &&
           check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

extern "C" void *pgpu_host_malloc(size_t bytes) {
    void *p = NULL;
    if (!bytes) bytes = 1;
    if (!check(hipHostMalloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc")) return NULL;
    return p;
}

extern "C" void pgpu_host_free(void *ptr) {
    if (ptr) (void)hipHostFree(ptr);
}

extern "C" int pgpu_copy_h2d_async(void *stream, void *dst, const void *src, size_t bytes) {
    if (!bytes) return 1;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream),
                 "hipMemcpyAsync H2D");
}

extern "C" int pgpu_copy_d2h(void *stream, void *dst, const void *src, size_t bytes) {
    if (!bytes) return 1;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream),
                 "hipMemcpyAsync D2H") &&
           check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

extern "C" int pgpu_copy_d2d(void *stream, void *dst, const void *src, size_t bytes) {
    if (!bytes) return 1;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
                 "hipMemcpyAsync D2D");
}

extern "C" int pgpu_stream_create(void **stream) {
    hipStream_t s = NULL;
    if (!check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return 0;
    *stream = s;
    return 1;
}

extern "C" void pgpu_stream_destroy(void *stream) {
    if (stream) (void)hipStreamDestroy((hipStream_t)stream);
}

extern "C" int pgpu_stream_sync(void *stream) {
    return check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

extern "C" int pgpu_event_create(void **event) {
    hipEvent_t e = NULL;
    if (!check(hipEventCreate(&e), "hipEventCreate")) return 0;
    *event = e;
    return 1;
}

extern "C" void pgpu_event_destroy(void *event) {
    if (event) (void)hipEventDestroy((hipEvent_t)event);
}

extern "C" int pgpu_event_record(void *event, void *stream) {
    return check(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
}

extern "C" int pgpu_event_elapsed_ms(void *start, void *stop, float *ms) {
    return check(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize") &&
           check(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop),
                 "hipEventElapsedTime");
}

extern "C" int pgpu_stream_wait_event(void *stream, void *event) {
    return check(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0),
                 "hipStreamWaitEvent");
}

extern "C" int pgpu_graph_begin(void *stream) {
    return check(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal),
                 "hipStreamBeginCapture");
}

extern "C" int pgpu_graph_begin_global(void *stream) {
    return check(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeGlobal),
                 "hipStreamBeginCapture");
}

extern "C" int pgpu_graph_end(void *stream, void **exec) {
    hipGraph_t graph = NULL;
    hipGraphExec_t instance = NULL;
    if (!check(hipStreamEndCapture((hipStream_t)stream, &graph), "hipStreamEndCapture"))
        return 0;
    const int ok = check(hipGraphInstantiate(&instance, graph, NULL, NULL, 0),
                         "hipGraphInstantiate");
    (void)hipGraphDestroy(graph);
    if (!ok) return 0;
    *exec = instance;
    return 1;
}

extern "C" int pgpu_graph_launch(void *exec, void *stream) {
    return check(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream), "hipGraphLaunch");
}

extern "C" void pgpu_graph_destroy(void *exec) {
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

extern "C" int pgpu_check_launch(void) {
    return check(hipGetLastError(), "kernel launch");
}
