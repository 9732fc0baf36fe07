// The fixed device scratch of zt_attn_decode_noalloc: the decode's per-chunk
// partials live here instead of in a caller workspace, so that entry point
// allocates nothing (for callers that cannot: code under graph capture, tight
// serving loops, harnesses that forbid allocation).
//
// One array per device, part of this library's image: each GPU the library
// runs on holds its own copy at its own address until the process ends.  In
// host code `scratch` names a host-side stand-in, not device memory; the
// library asks the runtime for the device address once per device
// (zt_noalloc_scratch_address, called while that device is current) and passes
// that address to the kernels, never the array's name.
#include <hip/hip_runtime.h>

#include "kernels/args.h"

static __device__ __align__(256) float scratch[ZT_NOALLOC_SCRATCH_BYTES / sizeof(float)];

// The current device's address of `scratch` into *ptr; 0, or 1 if the runtime
// refuses (then *ptr is untouched).  Internal to the library.
extern "C" __attribute__((visibility("hidden"))) int zt_noalloc_scratch_address(void **ptr) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
        (void)hipGetLastError();
        return 1;
    }
    *ptr = p;
    return 0;
}
