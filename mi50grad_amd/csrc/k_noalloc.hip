// Scratch for the allocation-free decode entry point (kva_legacy_decode_noalloc).
//
// The split-K decode keeps per-workgroup partials (m, l, acc) for the
// sequences a workgroup range cuts; kva_legacy_decode takes them from a
// kva_cache's workspace, allocated by kva_create.  Callers that cannot
// allocate (code under graph capture, tight serving loops, harnesses that
// forbid hipMalloc) get them from this file-scope device array instead: it is
// part of the code object, so each GPU the library runs on holds its own copy
// from module load until the process ends, and no call allocates.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// the device address is fetched once per device with hipGetSymbolAddress
// (with that device current) and kept; only that pointer reaches kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kva_internal.h"

namespace kva {
namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};
int g_cus[kMaxDevices] = {};

}  // namespace

hipError_t noalloc_scratch(void **ptr, int *n_cu) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        g_cus[dev] = cus > 0 ? cus : 1;
        g_ptr[dev] = p;
    }
    *ptr = g_ptr[dev];
    *n_cu = g_cus[dev];
    return hipSuccess;
}

}  // namespace kva
