// probe.hip -- streaming bandwidth probes: the measured ceilings the
// shift-window kernels are compared against (read, copy, fill of a large
// buffer with 16-byte accesses).  Measurement only; no counterpart in the
// reference.
//
// Each workgroup of 256 lanes moves chunks of 256 x 16 x kUnroll bytes: lane
// t touches 16-byte elements t + j * 256 of its chunk (every load or store
// instruction of a wave covers 1 KiB of consecutive bytes), all kUnroll
// loads are issued before any is consumed, and chunks are walked grid-stride
// so that a launch of a few workgroups per CU keeps the whole buffer in
// flight.  The read kernel folds what it loads into one value per lane and
// stores it only when a lane sees an impossible bit pattern, so the loads
// cannot be removed and nothing is written in practice.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "neural_shift_hip.h"
#include "nsh_common.hpp"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kLanes = 256;
constexpr int kUnroll = 8;
constexpr int64_t kChunk = int64_t(kLanes) * kUnroll;  // 16-byte elements per chunk

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__global__ __launch_bounds__(kLanes) void probe_read_kernel(const u32x4* __restrict__ src,
                                                            int64_t n, u32x4* __restrict__ sink) {
    u32x4 acc = {0u, 0u, 0u, 0u};
    const int64_t full = n / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const u32x4* p = src + c * kChunk + threadIdx.x;
        u32x4 v[kUnroll];
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) v[j] = ld<NT>(p + j * kLanes);
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) acc ^= v[j];
    }
    for (int64_t i = full * kChunk + blockIdx.x * int64_t(kLanes) + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * kLanes)
        acc ^= src[i];
    if (acc.x == 0x7fc00001u && acc.y == 0x7fc00002u && acc.z == 0x7fc00003u &&
        acc.w == 0x7fc00004u)
        sink[threadIdx.x] = acc;
}

__global__ __launch_bounds__(kLanes) void probe_copy_kernel(const u32x4* __restrict__ src,
                                                            u32x4* __restrict__ dst, int64_t n) {
    const int64_t full = n / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t base = c * kChunk + threadIdx.x;
        u32x4 v[kUnroll];
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) v[j] = __builtin_nontemporal_load(src + base + j * kLanes);
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) __builtin_nontemporal_store(v[j], dst + base + j * kLanes);
    }
    for (int64_t i = full * kChunk + blockIdx.x * int64_t(kLanes) + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * kLanes)
        dst[i] = src[i];
}

__global__ __launch_bounds__(kLanes) void probe_fill_kernel(u32x4* __restrict__ dst, int64_t n,
                                                            unsigned int value) {
    const u32x4 v = {value, value, value, value};
    const int64_t full = n / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t base = c * kChunk + threadIdx.x;
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) __builtin_nontemporal_store(v, dst + base + j * kLanes);
    }
    for (int64_t i = full * kChunk + blockIdx.x * int64_t(kLanes) + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * kLanes)
        dst[i] = v;
}

}  // namespace

extern "C" int nsh_stream_probe(int kind, const void* src, void* dst, int64_t bytes,
                                int workgroups, void* stream) {
    using nsh_host::fail;
    if (bytes <= 0 || bytes % 16 != 0)
        return fail(NSH_ERR_INVALID, "stream_probe: bytes must be a positive multiple of 16");
    if (workgroups < 1 || workgroups > (1 << 20))
        return fail(NSH_ERR_INVALID, "stream_probe: workgroups must be in [1, 2^20]");
    const bool needs_src = kind == NSH_PROBE_READ || kind == NSH_PROBE_READ_NT ||
                           kind == NSH_PROBE_COPY;
    if ((needs_src && (!src || !nsh_host::aligned(src, 16))) || !dst ||
        !nsh_host::aligned(dst, 16))
        return fail(NSH_ERR_INVALID, "stream_probe: null or unaligned buffer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t n = bytes / 16;
    const auto* s = static_cast<const u32x4*>(src);
    auto* d = static_cast<u32x4*>(dst);
    const dim3 grid(static_cast<unsigned>(workgroups)), block(kLanes);
    switch (kind) {
        case NSH_PROBE_READ:
            hipLaunchKernelGGL(probe_read_kernel<false>, grid, block, 0, st, s, n, d);
            break;
        case NSH_PROBE_READ_NT:
            hipLaunchKernelGGL(probe_read_kernel<true>, grid, block, 0, st, s, n, d);
            break;
        case NSH_PROBE_COPY:
            hipLaunchKernelGGL(probe_copy_kernel, grid, block, 0, st, s, d, n);
            break;
        case NSH_PROBE_FILL:
            hipLaunchKernelGGL(probe_fill_kernel, grid, block, 0, st, d, n, 0x3f800000u);
            break;
        default:
            return fail(NSH_ERR_INVALID, "stream_probe: unknown kind %d", kind);
    }
    return nsh_host::check_launch("stream_probe");
}
