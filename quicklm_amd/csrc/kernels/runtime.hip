// Device, memory, stream, event and graph plumbing behind the C ABI, so that
// the C++17 host engine and the Python bindings need no HIP headers.

#include <stdio.h>

#include "common.hpp"

extern "C" const char* qlm_error_string(int status) {
    switch (status) {
        case QLM_OK: return "ok";
        case QLM_ERR_ARG: return "invalid argument (null pointer or non-positive size)";
        case QLM_ERR_SHAPE: return "unsupported shape";
        case QLM_ERR_NO_DEVICE: return "no HIP device";
        case QLM_ERR_SCRATCH:
            return "work exceeds the static device scratch of a no-allocation entry point";
        default: break;
    }
    if (status > 0) return hipGetErrorString((hipError_t)status);
    return "unknown error";
}

extern "C" int qlm_device_count(int* count) {
    if (!count) return QLM_ERR_ARG;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return e == hipErrorNoDevice ? QLM_ERR_NO_DEVICE : qlm_status(e);
    }
    *count = n;
    return QLM_OK;
}

// One kernel of each kernel file (defined there): asking for its attributes
// loads that file's code object.
hipError_t qlm_load_attention();
hipError_t qlm_load_deltanet();
hipError_t qlm_load_deltanet_chunk();
hipError_t qlm_load_elementwise();
hipError_t qlm_load_gemm();
hipError_t qlm_load_gemm_mx();
hipError_t qlm_load_gemm_t();
hipError_t qlm_load_gemm_w();
hipError_t qlm_load_gemv();
hipError_t qlm_load_quant();

// Selects the device and loads every kernel file's code object on it, so no
// first launch (of a prefill, a decode step, a graph capture) pays the load.
extern "C" int qlm_set_device(int device) {
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return qlm_status(e);
    for (hipError_t (*load)() : {qlm_load_attention, qlm_load_deltanet, qlm_load_deltanet_chunk, qlm_load_elementwise, qlm_load_gemm, qlm_load_gemm_mx, qlm_load_gemm_t, qlm_load_gemm_w, qlm_load_gemv, qlm_load_quant}) {
        e = load();
        if (e != hipSuccess) return qlm_status(e);
    }
    return QLM_OK;
}

extern "C" int qlm_device_name(char* buf, int len) {
    if (!buf || len <= 0) return QLM_ERR_ARG;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return qlm_status(e);
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return qlm_status(e);
    snprintf(buf, (size_t)len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return QLM_OK;
}

extern "C" int qlm_mem_info(size_t* free_bytes, size_t* total_bytes) {
    if (!free_bytes || !total_bytes) return QLM_ERR_ARG;
    return qlm_status(hipMemGetInfo(free_bytes, total_bytes));
}

extern "C" int qlm_malloc(void** ptr, size_t bytes) {
    if (!ptr) return QLM_ERR_ARG;
    *ptr = nullptr;
    if (bytes == 0) return QLM_OK;
    return qlm_status(hipMalloc(ptr, bytes));
}

extern "C" int qlm_free(void* ptr) { return ptr ? qlm_status(hipFree(ptr)) : QLM_OK; }

extern "C" int qlm_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QLM_OK;
    if (!dst || !src) return QLM_ERR_ARG;
    return qlm_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
}

extern "C" int qlm_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QLM_OK;
    if (!dst || !src) return QLM_ERR_ARG;
    return qlm_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
}

extern "C" int qlm_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QLM_OK;
    if (!dst || !src) return QLM_ERR_ARG;
    return qlm_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
}

extern "C" int qlm_stream_create(void** stream) {
    if (!stream) return QLM_ERR_ARG;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = s;
    return qlm_status(e);
}

extern "C" int qlm_stream_destroy(void* stream) {
    return stream ? qlm_status(hipStreamDestroy(as_stream(stream))) : QLM_OK;
}

extern "C" int qlm_stream_sync(void* stream) {
    return qlm_status(hipStreamSynchronize(as_stream(stream)));
}

extern "C" int qlm_device_sync(void) { return qlm_status(hipDeviceSynchronize()); }

extern "C" int qlm_event_create(void** event) {
    if (!event) return QLM_ERR_ARG;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    *event = ev;
    return qlm_status(e);
}

extern "C" int qlm_event_destroy(void* event) {
    return event ? qlm_status(hipEventDestroy(reinterpret_cast<hipEvent_t>(event))) : QLM_OK;
}

extern "C" int qlm_event_record(void* event, void* stream) {
    if (!event) return QLM_ERR_ARG;
    return qlm_status(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
}

extern "C" int qlm_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms || !start || !stop) return QLM_ERR_ARG;
    hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop));
    if (e != hipSuccess) return qlm_status(e);
    return qlm_status(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                          reinterpret_cast<hipEvent_t>(stop)));
}

extern "C" int qlm_graph_begin(void* stream) {
    if (!stream) return QLM_ERR_ARG;  // the null stream cannot be captured
    return qlm_status(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
}

extern "C" int qlm_graph_end(void* stream, void** graph_exec) {
    if (!stream || !graph_exec) return QLM_ERR_ARG;
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(as_stream(stream), &g);
    if (e != hipSuccess) return qlm_status(e);
    hipGraphExec_t ge = nullptr;
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return qlm_status(e);
    *graph_exec = ge;
    return QLM_OK;
}

extern "C" int qlm_graph_launch(void* graph_exec, void* stream) {
    if (!graph_exec) return QLM_ERR_ARG;
    return qlm_status(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
}

extern "C" int qlm_graph_destroy(void* graph_exec) {
    return graph_exec ? qlm_status(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)))
                      : QLM_OK;
}
