/*
 * A fixed device scratch area for the entry points that must not allocate
 * (q38_full_core_noalloc): callers under HIP graph capture, in tight serving
 * loops, or in harnesses that forbid hipMalloc.
 *
 * `scratch` is a file-scope device array of Q38_NOALLOC_SCRATCH_BYTES; every
 * device the library runs on holds its own copy, at its own address, until
 * the process ends.  In host code the name `scratch` is only a host-side
 * stand-in: its device address comes from hipGetSymbolAddress, called once
 * per device with that device current (from q38_ctx_create), and that
 * address -- never the array's name -- is what kernels receive.
 *
 * All calls on one device share the array and it keeps the last call's
 * contents: calls that overlap on one device (two streams, two contexts)
 * race on it.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../../include/q38_attn.h"
#include "q38_scratch.h"

static __device__ __align__(256) unsigned char scratch[Q38_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mutex;
void *g_scratch_ptr[Q38_SCRATCH_MAX_DEVICES];
}  // namespace

extern "C" __attribute__((visibility("hidden"))) int q38_scratch_address(int device, void **ptr) {
    if (ptr == nullptr) return (int)hipErrorInvalidValue;
    *ptr = nullptr;
    if (device < 0 || device >= Q38_SCRATCH_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        int current = -1;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return (int)e;
        if (current != device) return (int)hipErrorInvalidDevice;
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (p == nullptr) return (int)hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *ptr = g_scratch_ptr[device];
    return 0;
}
