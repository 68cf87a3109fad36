// static_scratch.hip -- the fixed device scratch of the no-allocation projection entry
// point (prism_hip_project_device_noalloc): one file-scope device array per GPU,
// allocated with the code object and held until the process ends, so that call needs no
// hipMalloc.  Host code never passes the array's name to a kernel (on the host it names
// a stand-in, not device memory): static_scratch_address looks the device address up
// once per device, with that device current, and every user takes that address.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "prism_hip.h"

namespace prism {

namespace {

static __device__ __align__(256) unsigned char scratch[PRISM_NOALLOC_SCRATCH_BYTES];

std::mutex g_mu;
std::map<int, void *> g_addr;  // device ordinal -> its copy of `scratch`

}  // namespace

// Device address of `scratch` on `device`, which must be the current device.  Returns
// hipSuccess, or the error hipGetSymbolAddress reported (nothing is cached then).
hipError_t static_scratch_address(int device, void **ptr, size_t *bytes) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_addr.find(device);
    if (it == g_addr.end()) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return e != hipSuccess ? e : hipErrorInvalidSymbol;
        it = g_addr.emplace(device, p).first;
    }
    *ptr = it->second;
    *bytes = sizeof(scratch);
    return hipSuccess;
}

}  // namespace prism
