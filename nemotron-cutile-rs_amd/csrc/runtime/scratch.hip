// Static device scratch of the allocation-free linear entry point
// (nh_linear_w8a8_noalloc): a file-scope device array that the HIP runtime
// places on every GPU the library runs on, held until the process ends.  Its
// name is only a host-side stand-in: host code uses the device address that
// hipGetSymbolAddress returns, resolved once per device (with that device
// current) when a context is created, and passes that address to the kernels
// like any caller workspace.  Built by hipcc (host and device code) so that
// the runtime registers the array; the kernels themselves live in the
// separately loaded gfx950 code object.
#include <hip/hip_runtime.h>

#include "nh_runtime.h"

static __device__ __align__(256) unsigned char scratch[nh::kScratchBytes];

namespace nh {

nh_status scratch_address(void** out, nh_error* err) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
        *out = nullptr;
        return device_error(err, e, "hipGetSymbolAddress(scratch)");
    }
    *out = p;
    return NH_OK;
}

}  // namespace nh
