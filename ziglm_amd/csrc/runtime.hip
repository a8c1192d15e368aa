// hip_bridge runtime entry points: device info, memory, copies, streams, graphs
// (replacing cuda_bridge.cu:14-150), plus events, a kernel byte fill and error reporting.
// Same return convention as the reference: 0 on success, otherwise the hipError_t value;
// a NULL stream means a synchronous copy / device-wide sync, as in the reference.
#include <stdio.h>
#include <string.h>

#include "zl_common.h"
#include "zl_host.h"

namespace zl {

static thread_local int t_last_error = HIP_BRIDGE_OK;

void set_error(int code) {
    if (t_last_error == HIP_BRIDGE_OK) t_last_error = code;
}

__global__ void k_fill_u8(unsigned char* __restrict__ p, unsigned char v, size_t n) {
    // 16 bytes per thread where the pointer allows, bytes at the ends.
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const uintptr_t base = reinterpret_cast<uintptr_t>(p);
    const size_t head = (16 - (base & 15)) & 15;
    const size_t h = head < n ? head : n;
    for (size_t i = tid; i < h; i += stride) p[i] = v;
    const size_t nvec = (n - h) / 16;
    const uint32_t w = 0x01010101u * v;
    u32x4 word = {w, w, w, w};
    u32x4* pv = reinterpret_cast<u32x4*>(p + h);
    for (size_t i = tid; i < nvec; i += stride) pv[i] = word;
    for (size_t i = h + nvec * 16 + tid; i < n; i += stride) p[i] = v;
}

}  // namespace zl

using namespace zl;

extern "C" {

int hip_device_get_info(int device_id, char* name, size_t name_len, size_t* total_vram_bytes) {
    hipDeviceProp_t prop;
    hipError_t err = hipGetDeviceProperties(&prop, device_id);
    if (err != hipSuccess) return (int)err;
    if (name && name_len > 0) {
        strncpy(name, prop.name, name_len - 1);
        name[name_len - 1] = '\0';
    }
    if (total_vram_bytes) *total_vram_bytes = prop.totalGlobalMem;
    return 0;
}

int hip_malloc(void** ptr, size_t bytes) { return (int)hipMalloc(ptr, bytes); }

int hip_free(void* ptr) { return (int)hipFree(ptr); }

int hip_malloc_host(void** ptr, size_t bytes) { return (int)hipHostMalloc(ptr, bytes, hipHostMallocDefault); }

int hip_free_host(void* ptr) {
    if (!ptr) return 0;
    return (int)hipHostFree(ptr);
}

static int memcpy_kind(void* dst, const void* src, size_t bytes, HipStream_t stream,
                       hipMemcpyKind kind, const char* what) {
    if (bytes == 0) return 0;
    hipError_t err = stream ? hipMemcpyAsync(dst, src, bytes, kind, stream_of(stream))
                            : hipMemcpy(dst, src, bytes, kind);
    if (err != hipSuccess)
        fprintf(stderr, "[hip_bridge] %s failed (dst=%p, src=%p, bytes=%zu): %s (%d)\n", what, dst,
                src, bytes, hipGetErrorString(err), (int)err);
    return (int)err;
}

int hip_memcpy_h2d(void* dst, const void* src, size_t bytes, HipStream_t stream) {
    return memcpy_kind(dst, src, bytes, stream, hipMemcpyHostToDevice, "hip_memcpy_h2d");
}

int hip_memcpy_d2h(void* dst, const void* src, size_t bytes, HipStream_t stream) {
    return memcpy_kind(dst, src, bytes, stream, hipMemcpyDeviceToHost, "hip_memcpy_d2h");
}

int hip_memcpy_d2d(void* dst, const void* src, size_t bytes, HipStream_t stream) {
    return memcpy_kind(dst, src, bytes, stream, hipMemcpyDeviceToDevice, "hip_memcpy_d2d");
}

int hip_stream_create(HipStream_t* stream) {
    hipStream_t s;
    hipError_t err = hipStreamCreate(&s);
    if (err != hipSuccess) return (int)err;
    *stream = (HipStream_t)s;
    return 0;
}

int hip_stream_destroy(HipStream_t stream) {
    if (!stream) return 0;
    return (int)hipStreamDestroy(stream_of(stream));
}

int hip_stream_sync(HipStream_t stream) {
    if (!stream) return (int)hipDeviceSynchronize();
    return (int)hipStreamSynchronize(stream_of(stream));
}

int hip_graph_begin_capture(HipStream_t stream) {
    hipError_t err = hipStreamBeginCapture(stream_of(stream), hipStreamCaptureModeGlobal);
    if (err != hipSuccess)
        fprintf(stderr, "[hip_bridge] hipStreamBeginCapture failed: %s (%d)\n", hipGetErrorString(err), (int)err);
    return (int)err;
}

int hip_graph_end_capture(HipStream_t stream, HipGraph_t* graph_out) {
    hipGraph_t g = nullptr;
    hipError_t err = hipStreamEndCapture(stream_of(stream), &g);
    if (err != hipSuccess) {
        fprintf(stderr, "[hip_bridge] hipStreamEndCapture failed: %s (%d)\n", hipGetErrorString(err), (int)err);
        return (int)err;
    }
    *graph_out = (HipGraph_t)g;
    return 0;
}

int hip_graph_instantiate(HipGraphExec_t* exec_out, HipGraph_t graph) {
    hipGraphExec_t exec = nullptr;
    hipError_t err = hipGraphInstantiate(&exec, (hipGraph_t)graph, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        fprintf(stderr, "[hip_bridge] hipGraphInstantiate failed: %s (%d)\n", hipGetErrorString(err), (int)err);
        return (int)err;
    }
    *exec_out = (HipGraphExec_t)exec;
    return 0;
}

int hip_graph_launch(HipGraphExec_t exec, HipStream_t stream) {
    hipError_t err = hipGraphLaunch((hipGraphExec_t)exec, stream_of(stream));
    if (err != hipSuccess)
        fprintf(stderr, "[hip_bridge] hipGraphLaunch failed: %s (%d)\n", hipGetErrorString(err), (int)err);
    return (int)err;
}

int hip_graph_destroy(HipGraph_t graph) {
    if (!graph) return 0;
    return (int)hipGraphDestroy((hipGraph_t)graph);
}

int hip_graph_exec_destroy(HipGraphExec_t exec) {
    if (!exec) return 0;
    return (int)hipGraphExecDestroy((hipGraphExec_t)exec);
}

int hip_event_create(HipEvent_t* event) {
    hipEvent_t e;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) return (int)err;
    *event = (HipEvent_t)e;
    return 0;
}

int hip_event_destroy(HipEvent_t event) {
    if (!event) return 0;
    return (int)hipEventDestroy((hipEvent_t)event);
}

int hip_event_record(HipEvent_t event, HipStream_t stream) {
    return (int)hipEventRecord((hipEvent_t)event, stream_of(stream));
}

int hip_event_sync(HipEvent_t event) { return (int)hipEventSynchronize((hipEvent_t)event); }

int hip_event_elapsed_ms(float* ms, HipEvent_t start, HipEvent_t stop) {
    return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
}

int hip_fill_u8(void* ptr, unsigned char value, size_t bytes, HipStream_t stream) {
    if (bytes == 0) return 0;
    if (!ptr) return (int)hipErrorInvalidValue;
    int64_t blocks = cdiv((int64_t)(bytes / 16 + 1), 256);
    if (blocks > 4096) blocks = 4096;
    k_fill_u8<<<(unsigned)blocks, 256, 0, stream_of(stream)>>>((unsigned char*)ptr, value, bytes);
    return (int)hipGetLastError();
}

int hip_bridge_last_error(void) {
    int e = t_last_error;
    t_last_error = HIP_BRIDGE_OK;
    return e;
}

const char* hip_bridge_error_string(int code) {
    if (code == HIP_BRIDGE_OK) return "ok";
    if (code == HIP_BRIDGE_EINVAL) return "invalid argument (op not launched)";
    if (code == HIP_BRIDGE_EUNSUPPORTED) return "unsupported type or shape (op not launched)";
    if (code == HIP_BRIDGE_ESCRATCH)
        return "call needs more scratch than the no-allocation entry point's static maximum (op not launched)";
    return hipGetErrorString((hipError_t)code);
}

const char* hip_bridge_version(void) {
    return "hip_bridge 0.1 gfx950 -O3 -ffp-contract=off -packed-fp32-ops:off";
}

}  // extern "C"
