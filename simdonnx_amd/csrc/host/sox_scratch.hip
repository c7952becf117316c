// The device scratch of the allocation-free entry points (include/sox_hip.h: sox_scratch): one
// static array in every GPU's memory, laid down with the library's code object when the device first
// uses it and kept until the process ends. Host code never passes the array's name to a kernel or a
// copy (on the host it only names a registration stand-in): sox_scratch resolves this device's copy
// with hipGetSymbolAddress once, with that device current, and every caller uses that address.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../../include/sox_hip.h"

static __device__ __align__(256) unsigned char scratch[SOX_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // per device: the address hipGetSymbolAddress returned
}  // namespace

extern "C" int sox_scratch(int device, void** ptr, size_t* bytes) {
    if (!ptr || device < 0 || device >= kMaxDevices) return SOX_E_INVALID;
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return (int)e;
    if (cur != device) return SOX_E_INVALID;  // resolved with the device current, as its copy lives there
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return SOX_E_NOT_FOUND;
        g_scratch_ptr[device] = p;
    }
    *ptr = g_scratch_ptr[device];
    if (bytes) *bytes = SOX_SCRATCH_BYTES;
    return SOX_OK;
}
