// The fixed device scratch of the allocation-free entry points (slm_hip_attend_noalloc): one
// statically sized array in every GPU's copy of this file's code object, found once per
// device with hipGetSymbolAddress and handed to kernels as a plain pointer.
//
// In host code `scratch` names a host-side stand-in, not device memory: only the address
// slm_scratch_address returns may reach a kernel, a copy or a fill.
#include <hip/hip_runtime.h>

#include <mutex>

#include "scratch.h"

static __device__ __align__(256) float scratch[SLM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_addr[MAX_DEVICES];  // per device: its copy of `scratch` (null until looked up)
}  // namespace

// The device address of `scratch` on the current device (looked up on the first call for
// that device, with the device current, then kept). Returns hipSuccess or the error of
// hipGetDevice / hipGetSymbolAddress.
__attribute__((visibility("hidden"))) hipError_t slm_scratch_address(void** out) {
    *out = nullptr;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_addr[dev] = p;
    }
    *out = g_addr[dev];
    return hipSuccess;
}
