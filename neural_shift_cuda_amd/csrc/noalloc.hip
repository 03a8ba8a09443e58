// noalloc.hip -- accumulate_uz forward for callers that cannot allocate.
//
// nsh_accumulate_uz_forward takes its scatter-path workspace (the spilled
// borders of the per-tile LDS windows plus a small header) from the caller.
// Code under HIP graph capture, tight serving loops and harnesses that forbid
// hipMalloc cannot provide one per call, so this entry point uses a static
// device array instead: `scratch`, NSH_NOALLOC_SCRATCH_BYTES per GPU, held by
// every GPU the library runs on until the process ends.
//
// In host code `scratch` is only a host-side stand-in for the symbol; its
// device address differs per GPU and comes from hipGetSymbolAddress, called
// once per device with that device current and kept in g_scratch[].  Only
// that address ever reaches a kernel.
//
// Nothing in the workspace has to start at zero: the forward kernel writes
// the header word the fix-up reads and every spill entry before the fix-up
// launch (which follows on the same stream) reads it, so leftover contents of
// an earlier call are never read.  All calls on one GPU share its array:
// calls that overlap on one GPU (other streams, other threads) race and must
// be serialized by the caller.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "neural_shift_hip.h"
#include "nsh_common.hpp"

namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[NSH_NOALLOC_SCRATCH_BYTES];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of the current device's scratch into *out (NSH_OK, else an
// error code with the message set).  First call per device:
// hipGetSymbolAddress with that device current; later calls read the cached
// address.  The kernels run on the
// caller's stream, so a stream that belongs to another device than the
// current one is rejected (its kernels would be handed this device's array).
int device_scratch(hipStream_t stream, void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return nsh_host::fail(NSH_ERR_HIP, "accumulate_uz_forward_noalloc: no current HIP device");
    if (stream != nullptr) {
        int sdev = -1;
        const hipError_t e = hipStreamGetDevice(stream, &sdev);
        if (e != hipSuccess)
            return nsh_host::fail(NSH_ERR_HIP,
                                  "accumulate_uz_forward_noalloc: hipStreamGetDevice: %s",
                                  hipGetErrorString(e));
        if (sdev != dev)
            return nsh_host::fail(NSH_ERR_INVALID,
                                  "accumulate_uz_forward_noalloc: the stream belongs to device %d "
                                  "but device %d is current; make the stream's device current",
                                  sdev, dev);
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return nsh_host::fail(NSH_ERR_HIP,
                                  "accumulate_uz_forward_noalloc: hipGetSymbolAddress(scratch) "
                                  "failed on device %d: %s", dev, hipGetErrorString(e));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return NSH_OK;
}

}  // namespace

extern "C" int nsh_accumulate_uz_forward_noalloc(const void* x, const void* weights,
                                                 const int64_t* shifts, int64_t S, int64_t B,
                                                 int64_t C, int64_t H, int64_t W, int dtype,
                                                 void* U, void* Z, void* stream) {
    const int64_t need = nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, dtype, 0);
    if (need < 0) {
        // invalid arguments: the regular entry point reports which
        return nsh_accumulate_uz_forward(x, weights, shifts, S, B, C, H, W, dtype, U, Z, nullptr,
                                         0, stream);
    }
    if (need > NSH_NOALLOC_SCRATCH_BYTES)
        return nsh_host::fail(NSH_ERR_INVALID,
                              "accumulate_uz_forward_noalloc: this shape needs a %lld-byte "
                              "workspace, above the %lld-byte static scratch; use "
                              "nsh_accumulate_uz_forward with a caller workspace",
                              (long long)need, (long long)NSH_NOALLOC_SCRATCH_BYTES);
    if (need == 0)  // the shape takes the gather kernels, which use no workspace
        return nsh_accumulate_uz_forward(x, weights, shifts, S, B, C, H, W, dtype, U, Z, nullptr,
                                         0, stream);
    void* ws = nullptr;
    if (int rc = device_scratch(static_cast<hipStream_t>(stream), &ws)) return rc;
    return nsh_accumulate_uz_forward(x, weights, shifts, S, B, C, H, W, dtype, U, Z, ws,
                                     NSH_NOALLOC_SCRATCH_BYTES, stream);
}
