// Library-owned scratch of mxfa_run_bwd_noalloc: the fp32 partial dK/dV sums
// of the split GQA dK/dV pass (what mxfa_run_bwd_ws keeps in the caller's
// workspace), in a file-scope device array, so that entry point allocates
// nothing. This translation unit is the only device code compiled into
// libmxfa.so: the array, no kernels (those are in the code object, and take
// the array's address as an argument).
#include <hip/hip_runtime.h>

#include <mutex>

#include "fa_launch.h"

namespace mxfa {

namespace {

// 65 MiB per device (64 MiB of partial planes and up to 1 MiB of share
// flags), held from the library's first use on the device until the process
// ends.
constexpr size_t kScratchBytes = 65ull << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices];  // the array's device address, per device

}  // namespace

size_t noalloc_scratch_bytes() { return kScratchBytes; }

// The array's address on `device` (current on the calling thread), looked up
// once per device with hipGetSymbolAddress: the host-side name `scratch` is a
// stand-in, not a device address, so only this pointer is passed to kernels.
hipError_t noalloc_scratch(int device, void **ptr) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    return hipSuccess;
}

}  // namespace mxfa
