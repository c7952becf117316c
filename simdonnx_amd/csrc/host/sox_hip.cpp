// Thin C ABI over libamdhip64 (include/sox_hip.h). Every call maps one-to-one onto a HIP runtime
// call and returns its status; device-lost class errors latch the process-wide lost flag.
#include "../../../include/sox_hip.h"

#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace {

std::atomic<int> g_lost{0};

// A launch recorded into a graph: the `extra` array hipModuleLaunchKernel is given, the size it
// points at and a copy of the kernarg block, at addresses that stay valid for as long as the graph
// (and the executable instantiated from it) exists. A launch outside capture passes the same three
// from its own stack frame; a captured kernel node may keep the `extra` pointers it was given, so a
// captured launch never hands the runtime anything on the stack.
struct LaunchRecord {
    void* config[5];
    size_t size = 0;
    std::vector<uint8_t> args;
};
using RecordList = std::vector<std::unique_ptr<LaunchRecord>>;
std::mutex g_rec_mu;
std::map<void*, RecordList> g_capturing;  // stream -> records of the capture in progress
std::map<void*, RecordList> g_exec_recs;  // graph exec -> the records its kernel nodes point at

bool is_lost_error(hipError_t e) {
    return e == hipErrorLaunchFailure || e == hipErrorIllegalAddress || e == hipErrorECCNotCorrectable ||
           e == hipErrorLaunchTimeOut || e == hipErrorAssert;
}

int st(hipError_t e) {
    if (e == hipSuccess) return SOX_OK;
    if (is_lost_error(e)) g_lost.store(1);
    return (int)e;
}

}  // namespace

extern "C" {

int sox_init(int device, sox_device_info* info) {
    int n = 0;
    int rc = st(hipGetDeviceCount(&n));
    if (rc) return rc;
    if (device < 0 || device >= n) return SOX_E_INVALID;
    rc = st(hipSetDevice(device));
    if (rc || !info) return rc;
    hipDeviceProp_t p;
    rc = st(hipGetDeviceProperties(&p, device));
    if (rc) return rc;
    memset(info, 0, sizeof(*info));
    snprintf(info->name, sizeof(info->name), "%s", p.name);
    snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
    info->device = device;
    info->compute_units = p.multiProcessorCount;
    info->lds_per_cu = (int32_t)p.maxSharedMemoryPerMultiProcessor;
    info->clock_khz = p.clockRate;
    info->warp_size = p.warpSize;
    info->vendor_id = 0x1002;
    info->hbm_bytes = p.totalGlobalMem;
    int xcc = 1;
    // MI300/MI355-class parts spread CUs over 8 accelerator dies; the runtime does not expose the
    // count portably, so derive it from the arch (gfx942 / gfx950 multi-die parts report >= 256 CUs)
    if (strncmp(p.gcnArchName, "gfx9", 4) == 0 && p.multiProcessorCount >= 228) xcc = 8;
    info->xcds = xcc;
    return SOX_OK;
}

const char* sox_error_string(int status) {
    switch (status) {
        case SOX_OK: return "ok";
        case SOX_E_INVALID: return "invalid argument or unsupported shape";
        case SOX_E_NOT_FOUND: return "kernel or resource not found";
        case SOX_E_LOST: return "device lost";
        case SOX_E_UNSUPPORTED: return "not supported by the HIP backend";
        default: return hipGetErrorString((hipError_t)status);
    }
}

int sox_device_lost(void) { return g_lost.load(); }
void sox_device_reset_lost(void) { g_lost.store(0); }
void sox_device_mark_lost(void) { g_lost.store(1); }
int sox_device_sync(void) { return st(hipDeviceSynchronize()); }

std::atomic<uint64_t> g_allocs{0};
int sox_malloc(void** ptr, size_t bytes) {
    g_allocs++;
    return st(hipMalloc(ptr, bytes ? bytes : 256));
}
uint64_t sox_alloc_count(void) { return g_allocs.load(); }
int sox_free(void* ptr) { return ptr ? st(hipFree(ptr)) : SOX_OK; }
int sox_host_alloc(void** ptr, size_t bytes) {
    g_allocs++;
    return st(hipHostMalloc(ptr, bytes ? bytes : 64, hipHostMallocDefault));
}
int sox_host_free(void* ptr) { return ptr ? st(hipHostFree(ptr)) : SOX_OK; }

int sox_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return st(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
}
int sox_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return st(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
}
int sox_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return st(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
}

int sox_module_load(void** module, const void* image, size_t bytes) {
    (void)bytes;  // the code object is self-describing (ELF)
    if (!module || !image) return SOX_E_INVALID;
    return st(hipModuleLoadData((hipModule_t*)module, image));
}
int sox_module_unload(void* module) { return st(hipModuleUnload((hipModule_t)module)); }
int sox_module_function(void** fn, void* module, const char* name) {
    hipError_t e = hipModuleGetFunction((hipFunction_t*)fn, (hipModule_t)module, name);
    if (e == hipErrorNotFound) return SOX_E_NOT_FOUND;
    return st(e);
}

int sox_launch(void* fn, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes, void* stream,
               const void* kernarg, size_t kernarg_bytes) {
    if (g_lost.load()) return SOX_E_LOST;
    if (!fn || grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return SOX_E_INVALID;
    {
        std::lock_guard<std::mutex> lk(g_rec_mu);
        auto it = g_capturing.find(stream);
        if (it != g_capturing.end()) {
            auto rec = std::make_unique<LaunchRecord>();
            rec->size = kernarg_bytes;
            rec->args.assign((const uint8_t*)kernarg, (const uint8_t*)kernarg + kernarg_bytes);
            void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, rec->args.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE,
                              &rec->size, HIP_LAUNCH_PARAM_END};
            memcpy(rec->config, config, sizeof config);
            void** extra = rec->config;
            it->second.push_back(std::move(rec));
            return st(hipModuleLaunchKernel((hipFunction_t)fn, grid[0], grid[1], grid[2], block[0], block[1],
                                            block[2], lds_bytes, (hipStream_t)stream, nullptr, extra));
        }
    }
    size_t size = kernarg_bytes;
    void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(kernarg), HIP_LAUNCH_PARAM_BUFFER_SIZE,
                      &size, HIP_LAUNCH_PARAM_END};
    return st(hipModuleLaunchKernel((hipFunction_t)fn, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                    lds_bytes, (hipStream_t)stream, nullptr, config));
}

int sox_stream_create(void** stream) { return st(hipStreamCreateWithFlags((hipStream_t*)stream, hipStreamNonBlocking)); }
int sox_stream_destroy(void* stream) { return st(hipStreamDestroy((hipStream_t)stream)); }
int sox_stream_sync(void* stream) { return st(hipStreamSynchronize((hipStream_t)stream)); }
int sox_stream_wait_event(void* stream, void* ev) { return st(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)ev, 0)); }
int sox_stream_is_capturing(void* stream, int* capturing) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const int rc = st(hipStreamIsCapturing((hipStream_t)stream, &cs));
    *capturing = cs != hipStreamCaptureStatusNone;
    return rc;
}

int sox_event_create(void** ev) { return st(hipEventCreate((hipEvent_t*)ev)); }
int sox_event_destroy(void* ev) { return st(hipEventDestroy((hipEvent_t)ev)); }
int sox_event_record(void* ev, void* stream) { return st(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream)); }
int sox_event_sync(void* ev) { return st(hipEventSynchronize((hipEvent_t)ev)); }
int sox_event_elapsed_ms(float* ms, void* start, void* stop) {
    return st(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
}

int sox_graph_begin(void* stream) {
    if (!stream) return SOX_E_INVALID;  // the legacy default stream cannot be captured
    {
        std::lock_guard<std::mutex> lk(g_rec_mu);
        if (g_capturing.count(stream)) return SOX_E_INVALID;
        g_capturing[stream];
    }
    int rc = st(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    if (rc) {
        std::lock_guard<std::mutex> lk(g_rec_mu);
        g_capturing.erase(stream);
    }
    return rc;
}
int sox_graph_end(void* stream, void** graph_exec) {
    RecordList recs;
    {
        std::lock_guard<std::mutex> lk(g_rec_mu);
        auto it = g_capturing.find(stream);
        if (it != g_capturing.end()) {
            recs = std::move(it->second);
            g_capturing.erase(it);
        }
    }
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    int rc = st(hipStreamEndCapture((hipStream_t)stream, &g));
    if (rc) return rc;
    hipGraphExec_t ex = nullptr;
    rc = st(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *graph_exec = ex;
    std::lock_guard<std::mutex> lk(g_rec_mu);
    g_exec_recs[ex] = std::move(recs);
    return SOX_OK;
}
int sox_graph_launch(void* graph_exec, void* stream) {
    if (g_lost.load()) return SOX_E_LOST;
    return st(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream));
}
int sox_graph_destroy(void* graph_exec) {
    if (!graph_exec) return SOX_OK;
    int rc = st(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    std::lock_guard<std::mutex> lk(g_rec_mu);
    g_exec_recs.erase(graph_exec);
    return rc;
}

}  // extern "C"
