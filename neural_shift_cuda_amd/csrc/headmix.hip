// headmix.hip -- head mixing of per-head weight planes into per-channel
// planes on gfx950: the (C, heads) mixing matrix of the attention installers
// (reference integration/nekde_drunet_attn_patch.py:117-140 `_mix_heads_vec`,
// its matrix case: an einsum "ch,sbhij->sbcij"), with its backward.
//
//   out[n, c, p] = sum_j mix[c, j] w[n, j, p]              (n: a (shift, batch) plane)
//   gw[n, j, p]  = sum_c mix[c, j] gout[n, c, p]
//   gmix[c, j]   = sum_{n, p} gout[n, c, p] w[n, j, p]
//
// Each pass reads every element of its inputs once and writes its outputs
// once (heads + C planes forward, C + 2 heads backward): HBM streams with
// 16-byte vectors.  One workgroup owns kMixChunk pixels of a plane and walks
// the planes n = blockIdx.y, blockIdx.y + gridDim.y, ...; sums are in the
// accumulator type.  gmix is a deterministic two-level reduction: each
// workgroup's partial sums (wave butterflies, then the waves in order) go to
// a workspace, and one workgroup per (c, j) adds them in index order.
#include <algorithm>
#include <initializer_list>

#include "nsh_common.hpp"

namespace nsh {

constexpr int kMixThreads = 256;
constexpr int kMixChunk = 1024;  // pixels of one plane per workgroup
constexpr int kMixMaxC = 8;      // channels served
constexpr int kMixMaxParts = 16384;
constexpr int kMixFinalThreads = 1024;

template <typename T, int NH, int VEC>
__global__ __launch_bounds__(kMixThreads) void head_mix_fwd_kernel(
    const T* __restrict__ w, const acc_t<T>* __restrict__ mix, int64_t N, int C, int64_t P,
    T* __restrict__ out) {
    using A = acc_t<T>;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kMixChunk;
    for (int64_t n = blockIdx.y; n < N; n += gridDim.y) {
        const T* wn = w + n * NH * P;
        T* on = out + n * C * P;
#pragma unroll
        for (int it = 0; it < kMixChunk / (kMixThreads * VEC); ++it) {
            const int64_t p = p0 + (static_cast<int64_t>(it) * kMixThreads + threadIdx.x) * VEC;
            if (p >= P) break;
            A wv[NH][VEC];
#pragma unroll
            for (int j = 0; j < NH; ++j) load_acc<T, VEC>(wn + j * P + p, wv[j]);
            for (int c = 0; c < C; ++c) {
                A o[VEC];
                const A m0 = mix[c * NH];
#pragma unroll
                for (int k = 0; k < VEC; ++k) o[k] = m0 * wv[0][k];
#pragma unroll
                for (int j = 1; j < NH; ++j) {
                    const A mj = mix[c * NH + j];
#pragma unroll
                    for (int k = 0; k < VEC; ++k) o[k] = fma_acc(mj, wv[j][k], o[k]);
                }
                store_acc<T, VEC>(on + c * P + p, o, false);
            }
        }
    }
}

template <typename A>
__device__ __forceinline__ A wave_sum(A v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <typename T, int NH, int VEC>
__global__ __launch_bounds__(kMixThreads) void head_mix_bwd_kernel(
    const T* __restrict__ w, const acc_t<T>* __restrict__ mix, const T* __restrict__ gout,
    int64_t N, int C, int64_t P, T* __restrict__ gw, acc_t<T>* __restrict__ part) {
    using A = acc_t<T>;
    __shared__ A red[kMixThreads / 64][kMixMaxC * NH];
    A pm[kMixMaxC][NH];
#pragma unroll
    for (int c = 0; c < kMixMaxC; ++c)
#pragma unroll
        for (int j = 0; j < NH; ++j) pm[c][j] = A(0);
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kMixChunk;
    for (int64_t n = blockIdx.y; n < N; n += gridDim.y) {
        const T* wn = w + n * NH * P;
        const T* gn = gout + n * C * P;
        T* gwn = gw + n * NH * P;
#pragma unroll
        for (int it = 0; it < kMixChunk / (kMixThreads * VEC); ++it) {
            const int64_t p = p0 + (static_cast<int64_t>(it) * kMixThreads + threadIdx.x) * VEC;
            if (p >= P) break;
            A wv[NH][VEC], gv[NH][VEC];
#pragma unroll
            for (int j = 0; j < NH; ++j) {
                load_acc<T, VEC>(wn + j * P + p, wv[j]);
#pragma unroll
                for (int k = 0; k < VEC; ++k) gv[j][k] = A(0);
            }
#pragma unroll
            for (int c = 0; c < kMixMaxC; ++c) {
                if (c >= C) break;
                A g[VEC];
                load_acc<T, VEC>(gn + c * P + p, g);
#pragma unroll
                for (int j = 0; j < NH; ++j) {
                    const A mj = mix[c * NH + j];
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        gv[j][k] = fma_acc(mj, g[k], gv[j][k]);
                        pm[c][j] = fma_acc(g[k], wv[j][k], pm[c][j]);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < NH; ++j) store_acc<T, VEC>(gwn + j * P + p, gv[j], false);
        }
    }
    // the workgroup's partial gmix: wave butterflies, then the waves in order
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
#pragma unroll
    for (int c = 0; c < kMixMaxC; ++c) {
        if (c >= C) break;
#pragma unroll
        for (int j = 0; j < NH; ++j) {
            const A v = wave_sum(pm[c][j]);
            if (lane == 0) red[wave][c * NH + j] = v;
        }
    }
    __syncthreads();
    const int CH = C * NH;
    if (threadIdx.x < CH) {
        A s = red[0][threadIdx.x];
#pragma unroll
        for (int v = 1; v < kMixThreads / 64; ++v) s += red[v][threadIdx.x];
        const int64_t blk = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
        part[blk * CH + threadIdx.x] = s;
    }
}

// gmix[e] = sum over the workgroups' partials of entry e, in index order
// (one workgroup per entry: strided lane sums, then an LDS tree).
template <typename A>
__global__ __launch_bounds__(kMixFinalThreads) void head_mix_gmix_kernel(
    const A* __restrict__ part, int64_t nparts, int CH, A* __restrict__ gmix) {
    __shared__ A red[kMixFinalThreads];
    const int e = blockIdx.x;
    A s = A(0);
    for (int64_t b = threadIdx.x; b < nparts; b += kMixFinalThreads) s += part[b * CH + e];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = kMixFinalThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) gmix[e] = red[0];
}

// Grid of both passes from the shape alone (the workspace size must not
// depend on pointer values): kMixChunk pixels per workgroup across, planes
// down (looped), at most kMixMaxParts workgroups.
static void mix_grid(int64_t N, int64_t P, unsigned* gx, unsigned* gy) {
    const int64_t x = nsh_host::ceil_div(P, kMixChunk);
    *gx = static_cast<unsigned>(x);
    *gy = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(N, kMixMaxParts / x)));
}

template <typename T>
static int mix_vec(int64_t P, std::initializer_list<const void*> ptrs) {
    constexpr int v = sizeof(T) == 8 ? 2 : 4;
    if (P % v) return 1;
    for (const void* p : ptrs)
        if (!nsh_host::aligned(p, v * sizeof(T))) return 1;
    return v;
}

template <typename T, int NH>
static int mix_fwd(const void* w, const void* mix, int64_t N, int C, int64_t P, void* out,
                   hipStream_t st) {
    using A = acc_t<T>;
    unsigned gx, gy;
    mix_grid(N, P, &gx, &gy);
    const int v = mix_vec<T>(P, {w, out});
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(gx, gy), dim3(kMixThreads), 0, st,
                           static_cast<const T*>(w), static_cast<const A*>(mix), N, C, P,
                           static_cast<T*>(out));
    };
    if (v == 4) {
        if constexpr (sizeof(T) < 8) launch(head_mix_fwd_kernel<T, NH, 4>);
    } else if (v == 2) {
        if constexpr (sizeof(T) == 8) launch(head_mix_fwd_kernel<T, NH, 2>);
    } else {
        launch(head_mix_fwd_kernel<T, NH, 1>);
    }
    return nsh_host::check_launch("head_mix_forward");
}

template <typename T, int NH>
static int mix_bwd(const void* w, const void* mix, const void* gout, int64_t N, int C, int64_t P,
                   void* gw, void* gmix, void* ws, hipStream_t st) {
    using A = acc_t<T>;
    unsigned gx, gy;
    mix_grid(N, P, &gx, &gy);
    const int v = mix_vec<T>(P, {w, gout, gw});
    A* part = static_cast<A*>(ws);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(gx, gy), dim3(kMixThreads), 0, st,
                           static_cast<const T*>(w), static_cast<const A*>(mix),
                           static_cast<const T*>(gout), N, C, P, static_cast<T*>(gw), part);
    };
    if (v == 4) {
        if constexpr (sizeof(T) < 8) launch(head_mix_bwd_kernel<T, NH, 4>);
    } else if (v == 2) {
        if constexpr (sizeof(T) == 8) launch(head_mix_bwd_kernel<T, NH, 2>);
    } else {
        launch(head_mix_bwd_kernel<T, NH, 1>);
    }
    if (int rc = nsh_host::check_launch("head_mix_backward")) return rc;
    const int CH = C * NH;
    hipLaunchKernelGGL((head_mix_gmix_kernel<A>), dim3(CH), dim3(kMixFinalThreads), 0, st,
                       static_cast<const A*>(part), static_cast<int64_t>(gx) * gy, CH,
                       static_cast<A*>(gmix));
    return nsh_host::check_launch("head_mix_backward (matrix gradient)");
}

}  // namespace nsh

using nsh_host::fail;

// 0 when served, NSH_ERR_UNSUPPORTED for head or channel counts outside the
// kernels' range, NSH_ERR_INVALID otherwise.
static int mix_check(const char* op, int64_t N, int64_t heads, int64_t C, int64_t P, int dtype) {
    if (N < 1 || P < 1 || heads < 1 || C < 1) return fail(NSH_ERR_INVALID, "%s: empty tensor", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    if (P * 8 >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one plane must stay below 2^31 bytes", op);
    if (heads < 2 || heads > 4 || C > nsh::kMixMaxC)
        return fail(NSH_ERR_UNSUPPORTED, "%s: %lld heads, %lld channels (2..4 heads, up to %d "
                    "channels are served)", op, static_cast<long long>(heads),
                    static_cast<long long>(C), nsh::kMixMaxC);
    return NSH_OK;
}

#define NSH_MIX_DISPATCH(FN, ...)                                                           \
    switch (dtype) {                                                                         \
        case NSH_DTYPE_FLOAT16:                                                              \
            return heads == 2 ? nsh::FN<nsh::f16, 2>(__VA_ARGS__)                            \
                 : heads == 3 ? nsh::FN<nsh::f16, 3>(__VA_ARGS__) : nsh::FN<nsh::f16, 4>(__VA_ARGS__); \
        case NSH_DTYPE_BFLOAT16:                                                             \
            return heads == 2 ? nsh::FN<nsh::bf16, 2>(__VA_ARGS__)                           \
                 : heads == 3 ? nsh::FN<nsh::bf16, 3>(__VA_ARGS__) : nsh::FN<nsh::bf16, 4>(__VA_ARGS__); \
        case NSH_DTYPE_FLOAT32:                                                              \
            return heads == 2 ? nsh::FN<float, 2>(__VA_ARGS__)                               \
                 : heads == 3 ? nsh::FN<float, 3>(__VA_ARGS__) : nsh::FN<float, 4>(__VA_ARGS__); \
        default:                                                                             \
            return heads == 2 ? nsh::FN<double, 2>(__VA_ARGS__)                              \
                 : heads == 3 ? nsh::FN<double, 3>(__VA_ARGS__) : nsh::FN<double, 4>(__VA_ARGS__); \
    }

extern "C" int nsh_head_mix_forward(const void* w, const void* mix, int64_t N, int64_t heads,
                                    int64_t C, int64_t P, int dtype, void* out, void* stream) {
    if (int rc = mix_check("head_mix_forward", N, heads, C, P, dtype)) return rc;
    if (!w || !mix || !out) return fail(NSH_ERR_INVALID, "head_mix_forward: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int c = static_cast<int>(C);
    NSH_MIX_DISPATCH(mix_fwd, w, mix, N, c, P, out, st)
}

extern "C" int64_t nsh_head_mix_workspace_bytes(int64_t N, int64_t heads, int64_t C, int64_t P,
                                                int dtype) {
    if (mix_check("head_mix_backward", N, heads, C, P, dtype) != NSH_OK) return -1;
    unsigned gx, gy;
    nsh::mix_grid(N, P, &gx, &gy);
    const int64_t ab = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    return (static_cast<int64_t>(gx) * gy * C * heads * ab + 255) / 256 * 256;
}

extern "C" int nsh_head_mix_backward(const void* w, const void* mix, const void* grad_out,
                                     int64_t N, int64_t heads, int64_t C, int64_t P, int dtype,
                                     void* grad_w, void* grad_mix, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    if (int rc = mix_check("head_mix_backward", N, heads, C, P, dtype)) return rc;
    if (!w || !mix || !grad_out || !grad_w || !grad_mix || !workspace)
        return fail(NSH_ERR_INVALID, "head_mix_backward: null pointer argument");
    if (workspace_bytes < nsh_head_mix_workspace_bytes(N, heads, C, P, dtype))
        return fail(NSH_ERR_INVALID, "head_mix_backward: workspace smaller than "
                    "nsh_head_mix_workspace_bytes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int c = static_cast<int>(C);
    NSH_MIX_DISPATCH(mix_bwd, w, mix, grad_out, N, c, P, grad_w, grad_mix, workspace, st)
}
