// The fixed device scratch of rq_matmul_many_noalloc (include/rq.h): a
// file-scope device array whose address is resolved once per device, so
// that entry point allocates nothing (callers under graph capture, serving
// loops and harnesses that cannot call hipMalloc).
//
// Compiled by hipcc into librq.so next to the g++ host code: this
// translation unit's code object carries the array, and the HIP runtime
// places one copy of it on every device the library runs on (held until
// the process ends). Host code must not use the array's name as a device
// address (in host code it names a host-side stand-in); it uses the pointer
// hipGetSymbolAddress returns for the current device.

#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/rq.h"

// Layout: codes [RQ_NOALLOC_MAX_VALUES] int8, then f16 d and f16 s
// [RQ_NOALLOC_MAX_VALUES / 32] each, every plane 256-byte aligned.
#define RQ_NOALLOC_BYTES ((size_t)RQ_NOALLOC_MAX_VALUES + 2 * ((size_t)RQ_NOALLOC_MAX_VALUES / 32 * 2))

static __device__ __align__(256) unsigned char scratch[RQ_NOALLOC_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];
}  // namespace

// The device address of `scratch` on `device`, which must be the current
// device (rq_open calls this right after hipSetDevice). Resolved once per
// device; later calls return the kept pointer.
extern "C" __attribute__((visibility("hidden"))) hipError_t rq_noalloc_scratch(int device, void** ptr, size_t* bytes) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_mu);
    if (!g_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    *bytes = RQ_NOALLOC_BYTES;
    return hipSuccess;
}
