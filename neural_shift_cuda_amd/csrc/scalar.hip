// scalar.hip -- accumulate_uz_scalar (GASD scalar-per-transform weights).
//
// Semantics (reference csrc/shift_ops_cuda.cu:806-980, ops.py:350-390):
//   U[b,c,p]  = sum_s w[s,b,c] x[b,c,(p+s) mod]        Z[b,c,p] = sum_s w[s,b,c]
//   gx[q]     = sum_s w[s,b,c] gU[(q-s) mod]
//   gw[s,b,c] = sum_{p} gU[p] x[(p+s) mod] + gZ[p]
// Forward and gx reuse the tile + LDS-halo layout of accumulate_uz; the
// weights are per-workgroup uniforms (scalar loads).  gw is a deterministic
// two-level reduction: each workgroup reduces one chunk of one (s, b, c)
// plane (lane partials, then a wave64 xor-shuffle butterfly, then the four
// wave sums in fixed order) into a caller workspace, and a second kernel
// adds the chunk partials of each (s, b, c) in index order.
#include <initializer_list>

#include "nsh_common.hpp"

namespace nsh {

template <int VEC>
struct SGeo {
    static constexpr int TW = kTPR * VEC;
    static constexpr int TH = kRows;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
};

// MODE 0: forward (src = x, writes U and Z);  MODE 1: gx (src = gU).
template <typename T, int VEC, int MODE>
__global__ __launch_bounds__(kThreads) void scalar_tile_kernel(
    const void* __restrict__ src_v, const T* __restrict__ w, const int64_t* __restrict__ shifts,
    int cols, int S, int B, int C, int H, int W, int ntw, int nth, void* __restrict__ out0,
    acc_t<T>* __restrict__ out1) {
    using A = acc_t<T>;
    using G = SGeo<VEC>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* st = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    stage_shifts(shl, shifts, S, cols, H, W);
    if (MODE == 0)
        stage_tile<T, A>(st, static_cast<const T*>(src_v) + ti.bc * HW, H, W, ti.h0, ti.w0, G::LH, G::LW);
    else
        stage_tile_acc<A>(st, static_cast<const A*>(src_v) + ti.bc * HW, H, W, ti.h0, ti.w0, G::LH, G::LW);
    __syncthreads();

    const int tx = threadIdx.x % kTPR;
    const int ty = threadIdx.x / kTPR;
    const int h = ti.h0 + ty;
    const int w0 = ti.w0 + tx * VEC;
    if (h >= H || w0 >= W) return;
    const uint32_t own = static_cast<uint32_t>(h) * static_cast<uint32_t>(W) + w0;
    const int lc = (ty + kRmax) * G::LW + tx * VEC + kRmax;
    const int64_t BC = static_cast<int64_t>(B) * C;

    A u[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) u[k] = A(0);
    A z = A(0);
    for (int s = 0; s < S; ++s) {
        const ShiftRec r = read_shift(shl, s);
        const A ws = to_acc(w[s * BC + ti.bc]);
        z += ws;
        const int sgn = MODE == 0 ? 1 : -1;
        if (shift_in_lds(r)) {
            const A* sr = st + lc + sgn * (r.dx * G::LW + r.dy);
#pragma unroll
            for (int k = 0; k < VEC; ++k) u[k] = fma_acc(ws, sr[k], u[k]);
        } else {
            int hh = MODE == 0 ? h + r.dxm : h - r.dxm;
            hh = MODE == 0 ? (hh >= H ? hh - H : hh) : (hh < 0 ? hh + H : hh);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int ww = MODE == 0 ? w0 + k + r.dym : w0 + k - r.dym;
                ww = MODE == 0 ? (ww >= W ? ww - W : ww) : (ww < 0 ? ww + W : ww);
                const uint32_t i = static_cast<uint32_t>(hh) * W + ww;
                const A v = MODE == 0 ? to_acc(static_cast<const T*>(src_v)[ti.bc * HW + i])
                                      : static_cast<const A*>(src_v)[ti.bc * HW + i];
                u[k] = fma_acc(ws, v, u[k]);
            }
        }
    }
    if (MODE == 0) {
        A zz[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) zz[k] = z;
        store_out<A, VEC>(static_cast<A*>(out0) + ti.bc * HW + own, u);
        store_out<A, VEC>(out1 + ti.bc * HW + own, zz);
    } else {
        store_acc<T, VEC>(static_cast<T*>(out0) + ti.bc * HW + own, u, false);
    }
}

template <typename A>
__device__ __forceinline__ A block_sum(A v, A* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    A t = A(0);
    if (threadIdx.x == 0)
        for (int i = 0; i < kThreads / 64; ++i) t += red[i];
    return t;  // valid in thread 0
}

// gw partials: block (sbc, split) reduces pixels [split*chunk, ...) of plane (b, c) for shift s.
template <typename T>
__global__ __launch_bounds__(kThreads) void scalar_gw_partial_kernel(
    const T* __restrict__ x, const acc_t<T>* __restrict__ gU, const acc_t<T>* __restrict__ gZ,
    const int64_t* __restrict__ shifts, int cols, int B, int C, int H, int W, int nsplit,
    acc_t<T>* __restrict__ partial) {
    using A = acc_t<T>;
    __shared__ A red[kThreads / 64];
    const int64_t sbc = blockIdx.x / nsplit;
    const int split = static_cast<int>(blockIdx.x - sbc * nsplit);
    const int64_t BC = static_cast<int64_t>(B) * C;
    const int64_t s = sbc / BC;
    const int64_t bc = sbc - s * BC;
    const int dxm = static_cast<int>(mod_pos(shifts[s * cols + 0], H));
    const int dym = static_cast<int>(mod_pos(shifts[s * cols + 1], W));
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t chunk = (HW + nsplit - 1) / nsplit;
    const int64_t p0 = split * chunk;
    const int64_t p1 = p0 + chunk < HW ? p0 + chunk : HW;
    const T* xp = x + bc * HW;
    const A* up = gU + bc * HW;
    const A* zp = gZ + bc * HW;
    A acc = A(0);
    for (int64_t p = p0 + threadIdx.x; p < p1; p += kThreads) {
        const int h = static_cast<int>(p / W);
        const int w = static_cast<int>(p - static_cast<int64_t>(h) * W);
        int hh = h + dxm;
        hh -= hh >= H ? H : 0;
        int ww = w + dym;
        ww -= ww >= W ? W : 0;
        acc += fma_acc(up[p], to_acc(xp[static_cast<uint32_t>(hh) * W + ww]), zp[p]);
    }
    const A t = block_sum(acc, red);
    if (threadIdx.x == 0) partial[sbc * nsplit + split] = t;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void scalar_gw_final_kernel(const acc_t<T>* __restrict__ partial,
                                                                   int64_t n, int nsplit,
                                                                   T* __restrict__ gw) {
    using A = acc_t<T>;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    A t = A(0);
    for (int k = 0; k < nsplit; ++k) t += partial[i * nsplit + k];
    gw[i] = from_acc<T>(t);
}

template <int VEC>
static size_t s_lds(int S, size_t ab) {
    return static_cast<size_t>(S) * sizeof(int4) + static_cast<size_t>(SGeo<VEC>::LH) * SGeo<VEC>::LW * ab;
}

template <typename T, int VEC, int MODE>
static int s_tile_launch(const void* src, const void* w, const int64_t* sh, int cols, int S, int B,
                         int C, int H, int W, void* out0, void* out1, hipStream_t st) {
    using G = SGeo<VEC>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(H, G::TH));
    const int64_t tiles = static_cast<int64_t>(B) * C * ntw * nth;
    hipLaunchKernelGGL((scalar_tile_kernel<T, VEC, MODE>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), s_lds<VEC>(S, sizeof(acc_t<T>)), st, src,
                       static_cast<const T*>(w), sh, cols, S, B, C, H, W, ntw, nth, out0,
                       static_cast<acc_t<T>*>(out1));
    return nsh_host::check_launch(MODE == 0 ? "accumulate_uz_scalar_forward"
                                            : "accumulate_uz_scalar_backward");
}

template <typename T, int MODE>
static int s_tile(const void* src, const void* w, const int64_t* sh, int cols, int S, int B, int C,
                  int H, int W, void* out0, void* out1, hipStream_t st) {
    // vector width limited by the narrowest-element tensors in play
    int v = 1;
    for (int cand = 16 / static_cast<int>(sizeof(T)); cand > 1; cand /= 2) {
        if (W % cand) continue;
        bool ok = nsh_host::aligned(src, cand * (MODE == 0 ? sizeof(T) : sizeof(acc_t<T>))) &&
                  nsh_host::aligned(out0, cand * (MODE == 0 ? sizeof(acc_t<T>) : sizeof(T))) &&
                  (out1 == nullptr || nsh_host::aligned(out1, cand * sizeof(acc_t<T>)));
        if (ok) {
            v = cand;
            break;
        }
    }
    switch (v) {
        case 8: if constexpr (sizeof(T) == 2) return s_tile_launch<T, 8, MODE>(src, w, sh, cols, S, B, C, H, W, out0, out1, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return s_tile_launch<T, 4, MODE>(src, w, sh, cols, S, B, C, H, W, out0, out1, st); break;
        case 2: return s_tile_launch<T, 2, MODE>(src, w, sh, cols, S, B, C, H, W, out0, out1, st);
        default: break;
    }
    return s_tile_launch<T, 1, MODE>(src, w, sh, cols, S, B, C, H, W, out0, out1, st);
}

static int scalar_splits(int64_t H, int64_t W) {
    const int64_t HW = H * W;
    int64_t n = (HW + 16383) / 16384;
    if (n < 1) n = 1;
    if (n > 256) n = 256;
    return static_cast<int>(n);
}

template <typename T>
static int s_gw(const void* x, const void* gU, const void* gZ, const int64_t* sh, int cols, int S,
                int B, int C, int H, int W, void* gw, void* partial, hipStream_t st) {
    using A = acc_t<T>;
    const int nsplit = scalar_splits(H, W);
    const int64_t n = static_cast<int64_t>(S) * B * C;
    const int64_t blocks = n * nsplit;
    if (blocks > 0x7fffffff) return nsh_host::fail(NSH_ERR_INVALID, "accumulate_uz_scalar: grid too large");
    hipLaunchKernelGGL((scalar_gw_partial_kernel<T>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kThreads), 0, st, static_cast<const T*>(x), static_cast<const A*>(gU),
                       static_cast<const A*>(gZ), sh, cols, B, C, H, W, nsplit,
                       static_cast<A*>(partial));
    if (int rc = nsh_host::check_launch("accumulate_uz_scalar_backward (gw partial)")) return rc;
    hipLaunchKernelGGL((scalar_gw_final_kernel<T>),
                       dim3(static_cast<unsigned>(nsh_host::ceil_div(n, kThreads))), dim3(kThreads),
                       0, st, static_cast<const A*>(partial), n, nsplit, static_cast<T*>(gw));
    return nsh_host::check_launch("accumulate_uz_scalar_backward (gw final)");
}

}  // namespace nsh

using nsh_host::fail;

static int s_check(const char* op, int64_t S, int64_t cols, int64_t B, int64_t C, int64_t H,
                   int64_t W, int dtype) {
    if (S < 1 || S > 1024) return fail(NSH_ERR_INVALID, "%s: tree reduction requires 1 <= S <= 1024", op);
    if (cols != 2 && cols != 3) return fail(NSH_ERR_INVALID, "%s: shifts must have 2 or 3 columns", op);
    if (B < 1 || C < 1 || H < 1 || W < 1) return fail(NSH_ERR_INVALID, "%s: empty tensor", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (B * C > (int64_t(1) << 24)) return fail(NSH_ERR_INVALID, "%s: B*C too large", op);
    return NSH_OK;
}

extern "C" int nsh_scalar_backward_splits(int64_t H, int64_t W) { return nsh::scalar_splits(H, W); }

extern "C" int nsh_accumulate_uz_scalar_forward(const void* x, const void* weights,
                                                const int64_t* shifts, int64_t S,
                                                int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                                int64_t W, int dtype, void* U, void* Z,
                                                void* stream) {
    if (int rc = s_check("accumulate_uz_scalar", S, shift_cols, B, C, H, W, dtype)) return rc;
    if (!x || !weights || !shifts || !U || !Z)
        return fail(NSH_ERR_INVALID, "accumulate_uz_scalar: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int s = (int)S, c = (int)shift_cols, b = (int)B, ch = (int)C, h = (int)H, w = (int)W;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::s_tile<nsh::f16, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
        case NSH_DTYPE_BFLOAT16: return nsh::s_tile<nsh::bf16, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
        case NSH_DTYPE_FLOAT32: return nsh::s_tile<float, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
        default: return nsh::s_tile<double, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
    }
}

extern "C" int nsh_accumulate_uz_scalar_backward(const void* x, const void* weights,
                                                 const void* grad_U, const void* grad_Z,
                                                 const int64_t* shifts, int64_t S,
                                                 int64_t shift_cols, int64_t B, int64_t C,
                                                 int64_t H, int64_t W, int dtype, void* grad_x,
                                                 void* grad_w, void* grad_w_partial, void* stream) {
    if (int rc = s_check("accumulate_uz_scalar_backward", S, shift_cols, B, C, H, W, dtype)) return rc;
    if (!x || !weights || !grad_U || !grad_Z || !shifts || !grad_x || !grad_w || !grad_w_partial)
        return fail(NSH_ERR_INVALID, "accumulate_uz_scalar_backward: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int s = (int)S, c = (int)shift_cols, b = (int)B, ch = (int)C, h = (int)H, w = (int)W;
    int rc = NSH_OK;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            rc = nsh::s_tile<nsh::f16, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<nsh::f16>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
        case NSH_DTYPE_BFLOAT16:
            rc = nsh::s_tile<nsh::bf16, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<nsh::bf16>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
        case NSH_DTYPE_FLOAT32:
            rc = nsh::s_tile<float, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<float>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
        default:
            rc = nsh::s_tile<double, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<double>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
    }
}
