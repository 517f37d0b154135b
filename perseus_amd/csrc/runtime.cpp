// The HIP runtime FFI: the MI355X replacement of crates/pc-cuda's hand-written cudart bindings (ffi.rs:18-50,
// mem.rs:19-24). Thin wrappers so a C / Rust / Python caller needs no HIP headers; each returns 0 or the HIP error.
#include <hip/hip_runtime.h>
#include <string.h>

#include "pc_hip.h"

static inline int rc(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

namespace pch {
int fill_bytes(void* dst, int value, size_t bytes, pc_stream_t s);  // elem.hip: a fill kernel
}
static inline hipStream_t S(pc_stream_t s) { return (hipStream_t)s; }

extern "C" {
int pc_hip_device_count(int* n) { return rc(hipGetDeviceCount(n)); }
int pc_hip_set_device(int dev) { return rc(hipSetDevice(dev)); }
int pc_hip_device_name(int dev, char* out, int len) {
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return rc(e);
    strncpy(out, p.gcnArchName, len > 0 ? (size_t)len - 1 : 0);
    if (len > 0) out[len - 1] = 0;
    return 0;
}
int pc_hip_malloc(void** p, size_t bytes) { return rc(hipMalloc(p, bytes)); }
int pc_hip_free(void* p) { return rc(hipFree(p)); }
int pc_hip_malloc_host(void** p, size_t bytes) { return rc(hipHostMalloc(p, bytes, hipHostMallocDefault)); }
int pc_hip_free_host(void* p) { return rc(hipHostFree(p)); }
int pc_hip_memcpy_htod(void* dst, const void* src, size_t bytes, pc_stream_t s) {
    return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(s)));
}
int pc_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes, pc_stream_t s) {
    return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(s)));
}
int pc_hip_memcpy_dtod(void* dst, const void* src, size_t bytes, pc_stream_t s) {
    return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(s)));
}
// a fill kernel, not hipMemsetAsync: a replay captured into a graph then holds no memset node
int pc_hip_memset(void* dst, int value, size_t bytes, pc_stream_t s) { return pch::fill_bytes(dst, value, bytes, s); }
// non-blocking streams at the default priority (crates/pc-cuda/src/stream.rs:20-28)
int pc_hip_stream_create(pc_stream_t* s) {
    hipStream_t h;
    hipError_t e = hipStreamCreateWithFlags(&h, hipStreamNonBlocking);
    *s = (pc_stream_t)h;
    return rc(e);
}
int pc_hip_stream_destroy(pc_stream_t s) { return rc(hipStreamDestroy(S(s))); }
int pc_hip_stream_sync(pc_stream_t s) { return rc(hipStreamSynchronize(S(s))); }
int pc_hip_stream_wait_event(pc_stream_t s, void* ev) { return rc(hipStreamWaitEvent(S(s), (hipEvent_t)ev, 0)); }
int pc_hip_device_sync(void) { return rc(hipDeviceSynchronize()); }
int pc_hip_event_create(void** ev) {
    hipEvent_t e;
    hipError_t r = hipEventCreate(&e);
    *ev = (void*)e;
    return rc(r);
}
int pc_hip_event_destroy(void* ev) { return rc(hipEventDestroy((hipEvent_t)ev)); }
int pc_hip_event_record(void* ev, pc_stream_t s) { return rc(hipEventRecord((hipEvent_t)ev, S(s))); }
int pc_hip_event_sync(void* ev) { return rc(hipEventSynchronize((hipEvent_t)ev)); }
int pc_hip_event_elapsed_ms(float* ms, void* start, void* stop) {
    return rc(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}
int pc_hip_graph_begin_capture(pc_stream_t s) { return rc(hipStreamBeginCapture(S(s), hipStreamCaptureModeGlobal)); }
int pc_hip_graph_end_capture(pc_stream_t s, void** graph) {
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(S(s), &g);
    *graph = (void*)g;
    return rc(e);
}
int pc_hip_graph_instantiate(void** exec, void* graph) {
    hipGraphExec_t x = nullptr;
    hipError_t e = hipGraphInstantiate(&x, (hipGraph_t)graph, nullptr, nullptr, 0);
    *exec = (void*)x;
    return rc(e);
}
int pc_hip_graph_launch(void* exec, pc_stream_t s) { return rc(hipGraphLaunch((hipGraphExec_t)exec, S(s))); }
int pc_hip_graph_destroy(void* graph) { return rc(hipGraphDestroy((hipGraph_t)graph)); }
int pc_hip_graph_exec_destroy(void* exec) { return rc(hipGraphExecDestroy((hipGraphExec_t)exec)); }
const char* pc_hip_error_string(int code) {
    if (code == -1) return "launch argument outside the kernel's range (-1)";
    if (code == -2) return "launch argument outside the kernel's range (-2)";
    if (code == -3) return "launch mode not supported by this kernel (-3)";
    return hipGetErrorString((hipError_t)code);
}
int pc_hip_last_error(void) { return rc(hipGetLastError()); }
}
