// Fixed device scratch for the allocation-free matmul entry point
// (ihip_gemm_q_noalloc): callers that cannot allocate (code under graph
// capture, tight serving loops) get the workspace of ihip_gemm_q from a
// file-scope device array instead of a caller buffer.
//
// Each GPU the library runs on holds its own copy of the array from module
// load until the process ends. In host code `scratch` names a host-side
// stand-in, not a device address: the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current
// (by ihip_init, so that no lookup happens inside a graph capture, or else
// on the first call on a device) and kept in a per-device table; only that
// address is handed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.h"

#define IHIP_NOALLOC_SCRATCH_BYTES (64u << 20)

static __device__ __align__(256) uint8_t scratch[IHIP_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES];  // device address of `scratch` per device (null: not looked up yet)
}  // namespace

size_t noalloc_scratch_bytes() { return IHIP_NOALLOC_SCRATCH_BYTES; }

// Device address of the current device's scratch (looked up on the first
// call per device, with that device current). Returns the HIP error of the
// lookup, or hipErrorInvalidDevice for a device index past the table.
hipError_t noalloc_scratch(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return hipSuccess;
}

// Looks up `device`'s scratch address now (ihip_init), with that device
// current for the lookup and the caller's device restored afterwards.
hipError_t noalloc_prepare(int device) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return e;
    void *p = nullptr;
    e = noalloc_scratch(&p);
    if (cur != device) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
    }
    return e;
}
