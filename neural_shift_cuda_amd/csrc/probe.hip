// probe.hip -- streaming bandwidth probes: the measured ceilings the
// shift-window kernels are compared against (read, copy, fill of a large
// buffer with 16-byte accesses).  Measurement only; no counterpart in the
// reference.
//
// Each workgroup of LANES lanes moves chunks of LANES x 16 x UNROLL bytes:
// lane t touches 16-byte elements t + j * LANES of its chunk (every load or
// store instruction of a wave covers 1 KiB of consecutive bytes), all UNROLL
// loads are issued before any is consumed, and chunks are walked grid-stride
// so that a launch of a few workgroups per CU keeps the whole buffer in
// flight.  The read kernel folds what it loads into one value per lane and
// stores it only when a lane sees an impossible bit pattern, so the loads
// cannot be removed and nothing is written in practice.
//
// Variants (bits above the kind, NSH_PROBE_*): UNROLL 4, 8 or 16 loads in
// flight per lane, plain (temporal) or streaming (nontemporal) loads and
// stores for copy and fill, 256 or 1024 lanes per workgroup, and for copy a
// per-lane prefetch ring (interleaved loads and stores) instead of bursts.
// The ceiling of a kind is the best of its variants.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "neural_shift_hip.h"
#include "nsh_common.hpp"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ __forceinline__ void st(u32x4 v, u32x4* p) {
    if constexpr (NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

template <int LANES, int UNROLL, bool NTL>
__global__ __launch_bounds__(LANES) void probe_read_kernel(const u32x4* __restrict__ src,
                                                           int64_t n, u32x4* __restrict__ sink) {
    constexpr int64_t kChunk = int64_t(LANES) * UNROLL;
    u32x4 acc = {0u, 0u, 0u, 0u};
    const int64_t full = n / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const u32x4* p = src + c * kChunk + threadIdx.x;
        u32x4 v[UNROLL];
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) v[j] = ld<NTL>(p + j * LANES);
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) acc ^= v[j];
    }
    for (int64_t i = full * kChunk + blockIdx.x * int64_t(LANES) + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * LANES)
        acc ^= src[i];
    if (acc.x == 0x7fc00001u && acc.y == 0x7fc00002u && acc.z == 0x7fc00003u &&
        acc.w == 0x7fc00004u)
        sink[threadIdx.x % 256] = acc;
}

template <int LANES, int UNROLL, bool NTL, bool NTS>
__global__ __launch_bounds__(LANES) void probe_copy_kernel(const u32x4* __restrict__ src,
                                                           u32x4* __restrict__ dst, int64_t n) {
    constexpr int64_t kChunk = int64_t(LANES) * UNROLL;
    const int64_t full = n / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t base = c * kChunk + threadIdx.x;
        u32x4 v[UNROLL];
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) v[j] = ld<NTL>(src + base + j * LANES);
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) st<NTS>(v[j], dst + base + j * LANES);
    }
    for (int64_t i = full * kChunk + blockIdx.x * int64_t(LANES) + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * LANES)
        dst[i] = src[i];
}

// Copy with a prefetch ring per lane (the shift kernels' pattern): UNROLL
// loads in flight, each step stores the oldest and loads UNROLL steps ahead,
// so loads and stores interleave evenly instead of in bursts.  The lane's
// elements are i0 + k * stride (grid-stride).
template <int LANES, int UNROLL, bool NTL, bool NTS>
__global__ __launch_bounds__(LANES) void probe_copy_ring_kernel(const u32x4* __restrict__ src,
                                                                u32x4* __restrict__ dst,
                                                                int64_t n) {
    const int64_t stride = int64_t(gridDim.x) * LANES;
    const int64_t i0 = int64_t(blockIdx.x) * LANES + threadIdx.x;
    if (i0 >= n) return;
    const int64_t last = n - 1;
    u32x4 v[UNROLL];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) v[j] = ld<NTL>(src + min(i0 + j * stride, last));
    int64_t i = i0;
    // whole rings: the slot of step j is consumed and refilled UNROLL steps ahead
    for (; i + (UNROLL - 1) * stride < n; i += UNROLL * stride) {
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) {
            const u32x4 t = v[j];
            v[j] = ld<NTL>(src + min(i + (j + UNROLL) * stride, last));
            st<NTS>(t, dst + i + j * stride);
        }
    }
#pragma unroll
    for (int j = 0; j < UNROLL; ++j)
        if (i + j * stride < n) st<NTS>(v[j], dst + i + j * stride);
}

template <int LANES, int UNROLL, bool NTS>
__global__ __launch_bounds__(LANES) void probe_fill_kernel(u32x4* __restrict__ dst, int64_t n,
                                                           unsigned int value) {
    constexpr int64_t kChunk = int64_t(LANES) * UNROLL;
    const u32x4 v = {value, value, value, value};
    const int64_t full = n / kChunk;
    for (int64_t c = blockIdx.x; c < full; c += gridDim.x) {
        const int64_t base = c * kChunk + threadIdx.x;
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) st<NTS>(v, dst + base + j * LANES);
    }
    for (int64_t i = full * kChunk + blockIdx.x * int64_t(LANES) + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * LANES)
        dst[i] = v;
}

template <int LANES, int UNROLL>
int launch(int kind, bool ntl, bool nts, bool ring, const u32x4* s, u32x4* d, int64_t n,
           int workgroups, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(workgroups)), block(LANES);
    if (kind == NSH_PROBE_COPY && ring) {
        if (ntl && nts)
            hipLaunchKernelGGL((probe_copy_ring_kernel<LANES, UNROLL, true, true>), grid, block,
                               0, st, s, d, n);
        else if (ntl)
            hipLaunchKernelGGL((probe_copy_ring_kernel<LANES, UNROLL, true, false>), grid, block,
                               0, st, s, d, n);
        else if (nts)
            hipLaunchKernelGGL((probe_copy_ring_kernel<LANES, UNROLL, false, true>), grid, block,
                               0, st, s, d, n);
        else
            hipLaunchKernelGGL((probe_copy_ring_kernel<LANES, UNROLL, false, false>), grid,
                               block, 0, st, s, d, n);
        return nsh_host::check_launch("stream_probe");
    }
    switch (kind) {
        case NSH_PROBE_READ:
        case NSH_PROBE_READ_NT:
            if (ntl)
                hipLaunchKernelGGL((probe_read_kernel<LANES, UNROLL, true>), grid, block, 0, st,
                                   s, n, d);
            else
                hipLaunchKernelGGL((probe_read_kernel<LANES, UNROLL, false>), grid, block, 0, st,
                                   s, n, d);
            break;
        case NSH_PROBE_COPY:
            if (ntl && nts)
                hipLaunchKernelGGL((probe_copy_kernel<LANES, UNROLL, true, true>), grid, block, 0,
                                   st, s, d, n);
            else if (ntl)
                hipLaunchKernelGGL((probe_copy_kernel<LANES, UNROLL, true, false>), grid, block,
                                   0, st, s, d, n);
            else if (nts)
                hipLaunchKernelGGL((probe_copy_kernel<LANES, UNROLL, false, true>), grid, block,
                                   0, st, s, d, n);
            else
                hipLaunchKernelGGL((probe_copy_kernel<LANES, UNROLL, false, false>), grid, block,
                                   0, st, s, d, n);
            break;
        default:
            if (nts)
                hipLaunchKernelGGL((probe_fill_kernel<LANES, UNROLL, true>), grid, block, 0, st,
                                   d, n, 0x3f800000u);
            else
                hipLaunchKernelGGL((probe_fill_kernel<LANES, UNROLL, false>), grid, block, 0, st,
                                   d, n, 0x3f800000u);
            break;
    }
    return nsh_host::check_launch("stream_probe");
}

}  // namespace

extern "C" int nsh_stream_probe(int kind, const void* src, void* dst, int64_t bytes,
                                int workgroups, void* stream) {
    using nsh_host::fail;
    const int base = kind & NSH_PROBE_KIND_MASK;
    const int ulog = (kind & NSH_PROBE_UNROLL_MASK) >> 8;
    const bool plain_loads = (kind & NSH_PROBE_PLAIN_LOADS) != 0;
    const bool plain_stores = (kind & NSH_PROBE_PLAIN_STORES) != 0;
    const bool wide = (kind & NSH_PROBE_1024_LANES) != 0;
    const bool ring = (kind & NSH_PROBE_RING) != 0;
    if (base > NSH_PROBE_FILL || (kind & ~(NSH_PROBE_KIND_MASK | NSH_PROBE_UNROLL_MASK |
                                           NSH_PROBE_PLAIN_LOADS | NSH_PROBE_PLAIN_STORES |
                                           NSH_PROBE_1024_LANES | NSH_PROBE_RING)) != 0 ||
        (ulog != 0 && (ulog < 2 || ulog > 4)))
        return fail(NSH_ERR_INVALID, "stream_probe: unknown kind %d", kind);
    if (bytes <= 0 || bytes % 16 != 0)
        return fail(NSH_ERR_INVALID, "stream_probe: bytes must be a positive multiple of 16");
    if (workgroups < 1 || workgroups > (1 << 20))
        return fail(NSH_ERR_INVALID, "stream_probe: workgroups must be in [1, 2^20]");
    const bool needs_src = base != NSH_PROBE_FILL;
    if ((needs_src && (!src || !nsh_host::aligned(src, 16))) || !dst ||
        !nsh_host::aligned(dst, 16))
        return fail(NSH_ERR_INVALID, "stream_probe: null or unaligned buffer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t n = bytes / 16;
    const auto* s = static_cast<const u32x4*>(src);
    auto* d = static_cast<u32x4*>(dst);
    // defaults: 8 loads in flight, 256 lanes; READ plain loads, READ_NT
    // streaming loads; COPY and FILL streaming loads and stores
    const int unroll = ulog == 0 ? 8 : 1 << ulog;
    const bool ntl = base == NSH_PROBE_READ_NT || (base == NSH_PROBE_COPY && !plain_loads);
    const bool nts = !plain_stores;
    if (wide) {
        switch (unroll) {
            case 4: return launch<1024, 4>(base, ntl, nts, ring, s, d, n, workgroups, st);
            case 16: return launch<1024, 16>(base, ntl, nts, ring, s, d, n, workgroups, st);
            default: return launch<1024, 8>(base, ntl, nts, ring, s, d, n, workgroups, st);
        }
    }
    switch (unroll) {
        case 4: return launch<256, 4>(base, ntl, nts, ring, s, d, n, workgroups, st);
        case 16: return launch<256, 16>(base, ntl, nts, ring, s, d, n, workgroups, st);
        default: return launch<256, 8>(base, ntl, nts, ring, s, d, n, workgroups, st);
    }
}
