// nsh_capi.cpp -- host-side pieces of the C ABI: the thread-local error
// channel, launch checking, and the ABI/version markers.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "neural_shift_hip.h"

#ifndef NSH_BUILD_ID
#define NSH_BUILD_ID "unknown"
#endif

namespace {
thread_local char g_last_error[512] = "";
}

namespace nsh_host {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NSH_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return NSH_OK;
}

bool aligned(const void* p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

int64_t ceil_div(int64_t a, int64_t b) { return a <= 0 ? 0 : 1 + (a - 1) / b; }

int compute_units() {
    constexpr int kFallback = 256;  // MI355X
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cached[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();  // no device: leave no sticky error behind
        return kFallback;
    }
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
        (void)hipGetLastError();
        return kFallback;
    }
    cached[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace nsh_host

extern "C" const char* nsh_last_error(void) { return g_last_error; }

extern "C" int nsh_index_width_bits(void) { return 64; }

extern "C" const char* nsh_version(void) { return "neural_shift_hip gfx950 " NSH_BUILD_ID; }
