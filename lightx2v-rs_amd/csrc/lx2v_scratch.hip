// lx2v_scratch.hip -- the device scratch behind lx2v_hip_linear_noalloc: a
// file-scope device array, so that a linear can run with no allocation at
// all (callers under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  `linear` keeps its per-token e4m3 activations (and its
// bf16 -> f32 bias / f32 -> bf16 activation staging, and split K's partial
// sums) in context workspaces it grows with hipMalloc; the no-alloc variant
// puts them here instead.
//
// The array's address on each device is resolved with hipGetSymbolAddress
// with that device current (scratch_setup, called at context creation and
// again by the entry point until it succeeds); host code uses only that
// address, never the array's name (which names a host-side stand-in).  Each
// device holds its own copy until the process ends.
//
// Ownership: one context at a time may have scratch work in flight on a
// device.  A context claims the array for the length of one call (or one
// graph launch whose graph holds such calls; a call being captured runs
// nothing yet and only takes the address) under the device's lock and
// records its completion event before the lock is released; another
// context's claim succeeds only once that event has completed, and fails
// (ScratchClaim::Busy) while it has not.  Calls of one context are ordered
// on its one stream, so they never race with each other.  Nothing in the
// array needs to start at zero: each call writes every byte it later reads.
#include <hip/hip_runtime.h>

#include <mutex>

#include "runtime.hpp"

namespace lx2v {

namespace {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
    std::mutex mu;
    void *ptr = nullptr;          // null until hipGetSymbolAddress has succeeded
    const void *owner = nullptr;  // the context whose work last used the array
    hipEvent_t owner_done = nullptr;
};

DeviceScratch g_dev[kMaxDevices];

// With the device current and d.mu held.
hipError_t resolve(DeviceScratch &d) {
    if (d.ptr) return hipSuccess;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) d.ptr = p;  // a failure is not cached: the next call tries again
    return e;
}

}  // namespace

hipError_t scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    DeviceScratch &d = g_dev[device];
    std::lock_guard<std::mutex> lock(d.mu);
    return resolve(d);
}

void *scratch_address(int device, hipError_t *err) {
    if (device < 0 || device >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    DeviceScratch &d = g_dev[device];
    std::lock_guard<std::mutex> lock(d.mu);
    *err = resolve(d);
    return d.ptr;
}

ScratchClaim scratch_claim(int device, const void *owner, hipEvent_t owner_done, void **ptr, hipError_t *err) {
    *ptr = nullptr;
    *err = hipSuccess;
    if (device < 0 || device >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return ScratchClaim::Error;
    }
    DeviceScratch &d = g_dev[device];
    d.mu.lock();
    if ((*err = resolve(d)) != hipSuccess) {
        d.mu.unlock();
        return ScratchClaim::Error;
    }
    if (d.owner && d.owner != owner) {
        const hipError_t q = hipEventQuery(d.owner_done);
        if (q == hipErrorNotReady) {
            d.mu.unlock();
            return ScratchClaim::Busy;
        }
        if (q != hipSuccess) {
            *err = q;
            d.mu.unlock();
            return ScratchClaim::Error;
        }
    }
    d.owner = owner;
    d.owner_done = owner_done;
    *ptr = d.ptr;
    return ScratchClaim::Held;  // the caller enqueues, records owner_done, then scratch_unlock
}

void scratch_unlock(int device) { g_dev[device].mu.unlock(); }

void scratch_release(int device, const void *owner) {
    if (device < 0 || device >= kMaxDevices) return;
    DeviceScratch &d = g_dev[device];
    std::lock_guard<std::mutex> lock(d.mu);
    if (d.owner == owner) {
        d.owner = nullptr;
        d.owner_done = nullptr;
    }
}

}  // namespace lx2v
