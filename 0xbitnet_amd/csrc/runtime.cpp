// Host runtime plumbing for liboxbitnet: thread-local errors, device memory,
// streams, events and device information, exported over the plain C ABI in
// include/oxbitnet_ops.h.  The reference's equivalent layer is wgpu
// (gpu/device.rs:11-54, gpu/buffer_pool.rs:12-41); here it is the HIP
// runtime directly, one process per GPU.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "oxb_common.h"
#include "oxb_kernels.h"

namespace oxb {

static thread_local std::string g_error;
static thread_local bool g_has_error = false;

int allow_dynamic_lds(const void *kernel) {
    static std::mutex mu;
    static std::set<std::pair<int, const void *>> done;
    int dev = 0;
    OXB_CHECK_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({dev, kernel})) return 0;
    hipFuncAttributes a{};
    OXB_CHECK_HIP(hipFuncGetAttributes(&a, kernel));
    const int room = 160 * 1024 - (int)a.sharedSizeBytes;
    OXB_CHECK_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, room));
    done.insert({dev, kernel});
    return 0;
}

int device_cus() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return cus;
}

void set_error(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    g_has_error = true;
}

void clear_error() {
    g_error.clear();
    g_has_error = false;
}

const char *last_error() { return g_has_error ? g_error.c_str() : nullptr; }

}  // namespace oxb

using namespace oxb;

extern "C" const char *oxb_last_error(void) { return last_error(); }

extern "C" void *oxb_device_malloc(size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        set_error("hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

extern "C" int oxb_device_free(void *p) {
    if (!p) return 0;
    OXB_CHECK_HIP(hipFree(p));
    return 0;
}

extern "C" int oxb_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    OXB_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    OXB_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
    return 0;
}

extern "C" int oxb_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    OXB_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    OXB_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
    return 0;
}

extern "C" int oxb_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream) {
    OXB_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return 0;
}

extern "C" int oxb_memset_d(void *dst, int value, size_t bytes, void *stream) {
    OXB_CHECK_HIP(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
    return 0;
}

extern "C" void *oxb_stream_create(void) {
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) {
        set_error("hipStreamCreate: %s", hipGetErrorString(e));
        return nullptr;
    }
    return (void *)s;
}

extern "C" int oxb_stream_destroy(void *stream) {
    if (stream) OXB_CHECK_HIP(hipStreamDestroy((hipStream_t)stream));
    return 0;
}

extern "C" int oxb_stream_sync(void *stream) {
    OXB_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
    return 0;
}

extern "C" int oxb_device_sync(void) {
    OXB_CHECK_HIP(hipDeviceSynchronize());
    return 0;
}

extern "C" void *oxb_event_create(void) {
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) {
        set_error("hipEventCreate: %s", hipGetErrorString(e));
        return nullptr;
    }
    return (void *)ev;
}

extern "C" int oxb_event_destroy(void *ev) {
    if (ev) OXB_CHECK_HIP(hipEventDestroy((hipEvent_t)ev));
    return 0;
}

extern "C" int oxb_event_record(void *ev, void *stream) {
    OXB_CHECK_HIP(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
    return 0;
}

extern "C" int oxb_event_sync(void *ev) {
    OXB_CHECK_HIP(hipEventSynchronize((hipEvent_t)ev));
    return 0;
}

extern "C" int oxb_stream_begin_capture(void *stream) {
    OXB_REQUIRE(stream, "stream capture needs a created stream (not the null stream)");
    OXB_CHECK_HIP(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    return 0;
}

extern "C" void *oxb_stream_end_capture(void *stream) {
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (g) (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        set_error("stream capture: %s", hipGetErrorString(e));
        return nullptr;
    }
    return (void *)ge;
}

extern "C" int oxb_graph_launch(void *graph, void *stream) {
    OXB_REQUIRE(graph, "oxb_graph_launch: null graph");
    OXB_CHECK_HIP(hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)stream));
    return 0;
}

extern "C" int oxb_graph_destroy(void *graph) {
    if (graph) OXB_CHECK_HIP(hipGraphExecDestroy((hipGraphExec_t)graph));
    return 0;
}

extern "C" float oxb_event_elapsed_ms(void *start, void *stop) {
    float ms = -1.0f;
    hipError_t e = hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop);
    if (e != hipSuccess) {
        set_error("hipEventElapsedTime: %s", hipGetErrorString(e));
        return -1.0f;
    }
    return ms;
}

extern "C" int oxb_device_info(char *name, int len, int *cus, int *clock_khz, size_t *hbm_bytes) {
    int dev = 0;
    OXB_CHECK_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    OXB_CHECK_HIP(hipGetDeviceProperties(&prop, dev));
    if (name && len > 0) {
        // the marketing name can be empty (some drivers leave it blank): the
        // architecture and CU count identify the part then
        if (prop.name[0])
            snprintf(name, (size_t)len, "%s (%s)", prop.name, prop.gcnArchName);
        else
            snprintf(name, (size_t)len, "%s, %d CUs", prop.gcnArchName, prop.multiProcessorCount);
    }
    if (cus) *cus = prop.multiProcessorCount;
    if (clock_khz) *clock_khz = prop.clockRate;
    if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
    return 0;
}
