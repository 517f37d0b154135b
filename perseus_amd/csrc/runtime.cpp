// The HIP runtime FFI: the MI355X replacement of crates/pc-cuda's hand-written cudart bindings (ffi.rs:18-50,
// mem.rs:19-24). Thin wrappers so a C / Rust / Python caller needs no HIP headers; each returns 0 or the HIP error.
#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>
#include <string.h>

#include "pc_hip.h"

// A failed call's error is returned here and then cleared from the thread's last-error slot, so that the next kernel
// launch's check (hipGetLastError after the launch) does not report it a second time as its own.
static inline int rc(hipError_t e) {
    if (e == hipSuccess) return 0;
    (void)hipGetLastError();
    return (int)e;
}

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
// cudaRuntimeGetVersion / cudaDriverGetVersion (crates/pc-cuda/src/device.rs:83-84): HIP's own version numbers
int pc_hip_runtime_version(int* v) { return rc(hipRuntimeGetVersion(v)); }
int pc_hip_driver_version(int* v) { return rc(hipDriverGetVersion(v)); }
// cudaDeviceGetAttribute (device.rs:115, :126) for the attribute numbers the reference passes, plus the gfx code
int pc_hip_device_attribute(int* v, int attr, int dev) {
    if (!v) return (int)hipErrorInvalidValue;
    switch (attr) {
    case PC_HIP_ATTR_CU_COUNT:
        return rc(hipDeviceGetAttribute(v, hipDeviceAttributeMultiprocessorCount, dev));
    case PC_HIP_ATTR_CC_MAJOR:
        return rc(hipDeviceGetAttribute(v, hipDeviceAttributeComputeCapabilityMajor, dev));
    case PC_HIP_ATTR_CC_MINOR:
        return rc(hipDeviceGetAttribute(v, hipDeviceAttributeComputeCapabilityMinor, dev));
    case PC_HIP_ATTR_CLOCK_KHZ:
        return rc(hipDeviceGetAttribute(v, hipDeviceAttributeClockRate, dev));
    case PC_HIP_ATTR_CLUSTERS: {
        // CDNA has no thread-block clusters: 0 for every valid device
        int cus = 0;
        if (int e = rc(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev))) return e;
        *v = 0;
        return 0;
    }
    case PC_HIP_ATTR_GFX_ARCH: {
        // "gfx950" -> 0x950: the hexadecimal digits after "gfx", up to the first ':'
        hipDeviceProp_t p;
        hipError_t e = hipGetDeviceProperties(&p, dev);
        if (e != hipSuccess) return rc(e);
        const char* a = p.gcnArchName;
        if (strncmp(a, "gfx", 3) != 0) return (int)hipErrorInvalidValue;
        int code = 0;
        for (a += 3; *a && *a != ':'; ++a) {
            const char ch = *a;
            const int d = ch >= '0' && ch <= '9' ? ch - '0' : ch >= 'a' && ch <= 'f' ? ch - 'a' + 10 : -1;
            if (d < 0) return (int)hipErrorInvalidValue;
            code = code * 16 + d;
        }
        *v = code;
        return 0;
    }
    default:
        return (int)hipErrorInvalidValue;
    }
}
// cudaMemGetInfo (device.rs:137, :188): free and total bytes of the current device
int pc_hip_mem_get_info(size_t* free_bytes, size_t* total_bytes) { return rc(hipMemGetInfo(free_bytes, total_bytes)); }
// cudaProfilerStart / cudaProfilerStop (device.rs:151-158): the device is synchronised first, as the reference does,
// then a running rocprofv3 is asked to resume or pause collection (its --selected-regions mode). With no profiling
// tool attached the request is a no-op, as cudaProfilerStart is without a profiler.
int pc_hip_profiler_start(void) {
    if (int e = rc(hipDeviceSynchronize())) return e;
    (void)roctxProfilerResume(0);
    return 0;
}
int pc_hip_profiler_stop(void) {
    if (int e = rc(hipDeviceSynchronize())) return e;
    (void)roctxProfilerPause(0);
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
// cudaDeviceGetStreamPriorityRange / cudaStreamCreateWithPriority (stream.rs:33-44, Stream::high_priority). Every
// stream of this library runs at the default priority: streams of different priorities sharing an MI355X have been
// seen to stop making progress. The range reads (0, 0), and the priority argument is accepted and not applied.
int pc_hip_stream_priority_range(int* least, int* greatest) {
    if (!least || !greatest) return (int)hipErrorInvalidValue;
    *least = 0;
    *greatest = 0;
    return 0;
}
int pc_hip_stream_create_with_priority(pc_stream_t* s, int priority) {
    (void)priority;
    return pc_hip_stream_create(s);
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
// cudaEventCreateWithFlags (stream.rs:146): PC_HIP_EVENT_DISABLE_TIMING (2, the value of both runtimes' flag) makes
// an ordering-only event (Event::new); 0 a timing event (Event::timing)
int pc_hip_event_create_flags(void** ev, unsigned flags) {
    if (!ev || (flags & ~(unsigned)PC_HIP_EVENT_DISABLE_TIMING)) return (int)hipErrorInvalidValue;
    hipEvent_t e;
    hipError_t r = hipEventCreateWithFlags(&e, flags ? hipEventDisableTiming : hipEventDefault);
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
// cudaGetErrorName (crates/pc-cuda/src/error.rs:29-32)
const char* pc_hip_error_name(int code) {
    if (code == -1 || code == -2) return "PC_LAUNCH_ARGS";
    if (code == -3) return "PC_LAUNCH_MODE";
    return hipGetErrorName((hipError_t)code);
}
int pc_hip_last_error(void) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}
}
