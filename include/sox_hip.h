/*
 * sox_hip.h - the thin C ABI over libamdhip64 that a managed host P/Invokes.
 *
 * It replaces the reference's Vulkan device API surface (Backends/Vulkan/Vk.cs:388-474, the 68
 * [LibraryImport] declarations, and the error mapping of Vk.Check, Vk.cs:44-49). Conventions:
 *   - every function returns int: 0 = success, otherwise the hipError_t value (or a negative
 *     SOX_E_* code below); sox_error_string() renders it. No exception or longjmp crosses the ABI.
 *   - handles are opaque pointers; sizes are size_t; no C++ or torch types appear.
 *   - a device-lost class error (launch failure, illegal address, ECC) latches a process-wide
 *     "lost" flag (the analogue of VkDevice.Lost, VkDevice.cs:18, 885-899); sox_device_lost()
 *     reports it, sox_device_reset_lost() clears it after the host has re-created its objects,
 *     and sox_device_mark_lost() sets it from the host (the settable VkDevice.Lost that
 *     tests/Sdcb.SimdOnnx.Tests/VkDeviceLossTests.cs:33 uses to exercise recovery without a fault).
 */
#ifndef SOX_HIP_H
#define SOX_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SOX_OK 0
#define SOX_E_INVALID -1     /* bad argument / unsupported shape */
#define SOX_E_NOT_FOUND -2   /* kernel or resource name not found */
#define SOX_E_LOST -3        /* device lost earlier in this process */
#define SOX_E_UNSUPPORTED -4 /* op / epilogue the backend does not implement (NotSupportedException) */

typedef struct sox_device_info {
    char name[256];
    char arch[64];        /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t device;
    int32_t compute_units;
    int32_t lds_per_cu;   /* bytes */
    int32_t clock_khz;
    int32_t warp_size;
    int32_t vendor_id;    /* 0x1002 (GpuDeviceInfo, Backends/GpuDeviceInfo.cs:12-20) */
    uint64_t hbm_bytes;
    int32_t xcds;         /* accelerator complex dies sharing the CUs (8 on MI355X) */
    int32_t pad_;
} sox_device_info;

/* Device (vkCreateInstance/EnumeratePhysicalDevices/CreateDevice/GetPhysicalDeviceProperties, Vk.cs:388-399). */
int sox_init(int device, sox_device_info* info);
const char* sox_error_string(int status);
int sox_device_lost(void);
void sox_device_reset_lost(void);
void sox_device_mark_lost(void); /* VkDevice.Lost = true (VkDevice.cs:18): every later launch returns SOX_E_LOST */
int sox_device_sync(void); /* vkDeviceWaitIdle, Vk.cs:474 */

/* Memory (vkCreateBuffer/AllocateMemory/MapMemory, Vk.cs:401-413): device slabs and pinned staging. */
int sox_malloc(void** ptr, size_t bytes);
/* Device (sox_malloc) and pinned host (sox_host_alloc) allocations made since the process started:
 * the check that an allocation-free entry point made none (no counterpart in the reference). */
uint64_t sox_alloc_count(void);
int sox_free(void* ptr);
int sox_host_alloc(void** ptr, size_t bytes); /* pinned, mapped: the "mapped staging" of VkSession */
int sox_host_free(void* ptr);
int sox_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int sox_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int sox_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);

/* Code objects (vkCreateShaderModule + vkCreateComputePipelines, Vk.cs:415-419):
 * hipModuleLoadData on an in-memory gfx950 code object, hipModuleGetFunction by name. */
int sox_module_load(void** module, const void* image, size_t bytes);
int sox_module_unload(void* module);
int sox_module_function(void** fn, void* module, const char* name);

/* Dispatch (vkCmdPushConstants + vkCmdDispatch, Vk.cs:440-441): hipModuleLaunchKernel with the
 * kernarg block passed as HIP_LAUNCH_PARAM_BUFFER_POINTER / _SIZE. */
int sox_launch(void* fn, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes, void* stream,
               const void* kernarg, size_t kernarg_bytes);

/* Streams: one per session (the compute queue, VkDevice.cs:92; vkQueueSubmit/WaitForFences, Vk.cs:467-473). */
int sox_stream_create(void** stream);
int sox_stream_destroy(void* stream);
int sox_stream_sync(void* stream);
/* hipStreamWaitEvent: later work on `stream` waits for the event's last record. */
int sox_stream_wait_event(void* stream, void* ev);
/* Whether `stream` is capturing into a graph (sox_graph_begin). */
int sox_stream_is_capturing(void* stream, int* capturing);

/* Events (vkCmdWriteTimestamp + vkGetQueryPoolResults, Vk.cs:449-453). */
int sox_event_create(void** ev);
int sox_event_destroy(void* ev);
int sox_event_record(void* ev, void* stream);
int sox_event_sync(void* ev);
int sox_event_elapsed_ms(float* ms, void* start, void* stop);

/* Replay: capture a stream's work into a graph and relaunch it (the analogue of the
 * pre-recorded command buffer, VkSession.cs:139-140). A sox_launch into a stream between
 * sox_graph_begin and sox_graph_end copies its kernarg block (and the launch's `extra` array) into
 * storage the graph owns until sox_graph_destroy, so the caller's kernarg memory may be reused at
 * once. Only streams created by sox_stream_create can be captured. */
int sox_graph_begin(void* stream);
int sox_graph_end(void* stream, void** graph_exec);
int sox_graph_launch(void* graph_exec, void* stream);
int sox_graph_destroy(void* graph_exec);

/* Device scratch of the allocation-free entry points (no counterpart in the reference: it serves
 * callers that cannot allocate, such as code under HIP graph capture or a serving loop). Every GPU
 * holds one static array of SOX_SCRATCH_BYTES bytes from its first use until the process ends;
 * sox_scratch returns this device's copy (device = the current device; call it once per device, e.g.
 * at initialisation) and its size. Kernels get the address as an argument; every user of a GPU shares
 * that GPU's array, so calls that use it concurrently on one GPU race. */
#define SOX_SCRATCH_BYTES (8u << 20)
int sox_scratch(int device, void** ptr, size_t* bytes);

#ifdef __cplusplus
}
#endif
#endif
