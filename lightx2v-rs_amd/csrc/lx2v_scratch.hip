// lx2v_scratch.hip -- the device scratch behind lx2v_hip_linear_noalloc: a
// file-scope device array, so that a linear can run with no allocation at
// all (callers under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  `linear` keeps its per-token e4m3 activations (and its
// bf16 -> f32 bias / f32 -> bf16 activation staging) in context workspaces it
// grows with hipMalloc; the no-alloc variant puts them here instead.
//
// The array's address on each device is resolved once, at context creation
// with that device current (scratch_setup), with hipGetSymbolAddress; host
// code uses only that address, never the array's name (which names a
// host-side stand-in).  Each device holds its own copy until the process
// ends, and every call on one device shares it: calls that overlap on a
// device (two streams, two contexts) race on its contents.  Nothing in it
// needs to start at zero: each call writes every byte it later reads.
#include <hip/hip_runtime.h>

#include <mutex>

#include "runtime.hpp"

namespace lx2v {

namespace {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
    bool tried = false;
    hipError_t err = hipSuccess;
    void *ptr = nullptr;
};

std::mutex g_mu;
DeviceScratch g_dev[kMaxDevices];

}  // namespace

hipError_t scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceScratch &d = g_dev[device];
    if (!d.tried) {
        d.tried = true;
        void *p = nullptr;
        d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // the device current here
        d.ptr = d.err == hipSuccess ? p : nullptr;
    }
    return d.err;
}

void *scratch_ptr(int device, hipError_t *err) {
    if (device < 0 || device >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    const DeviceScratch &d = g_dev[device];
    *err = d.tried ? d.err : hipErrorNotInitialized;
    return d.ptr;
}

}  // namespace lx2v
