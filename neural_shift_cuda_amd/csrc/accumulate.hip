// accumulate.hip -- accumulate_uz forward and fused backward for gfx950.
//
// Semantics (reference: csrc/shift_ops_cuda.cu:255-458, ops.py:157-206):
//   U[p]    = sum_s w_s[p] x[(p+s) mod] + sum_{s:inv, box(p-s)} w_s[p-s] x[p-s]
//   Z[p]    = sum_s w_s[p]              + sum_{s:inv, box(p-s)} w_s[p-s]
//   gx[q]   = sum_s w_s[(q-s) mod] gU[(q-s) mod] + sum_{s:inv, box(q+s)} w_s[q] gU[q+s]
//   gw_s[q] = x[(q+s) mod] gU[q] + gZ[q] + [inv, box(q+s)] (x[q] gU[q+s] + gZ[q+s])
//
// Layout of the work.  One workgroup (256 lanes, 4 waves) owns a
// kRows x (kTPR*VEC) pixel tile of one (b, c) plane and walks all S shift
// planes of that tile.  The image operands it re-reads S times (x; gU and gZ
// in the backward) are staged once, with a kRmax halo, in LDS; the weight
// planes are streamed from HBM with one 16-byte load per lane per shift
// (coalesced: 16 lanes cover one 256-byte tile row).  Each lane keeps its
// VEC pixels' sums in registers and folds the shift axis serially, the
// mirror (inverse-shift) term included, so the reduction needs no
// cross-lane traffic at all.  The mirror term re-reads w_s at p-s: the
// same cache lines the tile (or its neighbour on the same XCD) has just
// streamed, so that read is served by L1/L2 rather than HBM.
#include <initializer_list>

#include "nsh_common.hpp"

namespace nsh {

template <int VEC>
struct Geo {
    static constexpr int TW = kTPR * VEC;
    static constexpr int TH = kRows;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
};

// Whole-tile range tests for a shift: are all of the tile's pixels p such
// that p + sgn*s stays inside the image (no wrap, box true)?
__device__ __forceinline__ bool tile_inside(int h0, int w0, int TH, int TW, int H, int W,
                                            int dx, int dy) {
    const int h1 = (h0 + TH < H ? h0 + TH : H) - 1;
    const int w1 = (w0 + TW < W ? w0 + TW : W) - 1;
    return h0 + dx >= 0 && h1 + dx < H && w0 + dy >= 0 && w1 + dy < W;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void accumulate_uz_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const int64_t* __restrict__ shifts,
    int S, int C, int H, int W, int ntw, int nth, int64_t plane_step,
    acc_t<T>* __restrict__ U, acc_t<T>* __restrict__ Z) {
    using A = acc_t<T>;
    using G = Geo<VEC>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;

    stage_shifts(shl, shifts, S, 3, H, W);
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    __syncthreads();

    const int tx = threadIdx.x % kTPR;
    const int ty = threadIdx.x / kTPR;
    const int h = ti.h0 + ty;
    const int w0 = ti.w0 + tx * VEC;
    if (h >= H || w0 >= W) return;

    const uint32_t own = static_cast<uint32_t>(h) * static_cast<uint32_t>(W) + w0;
    const int lc = (ty + kRmax) * G::LW + tx * VEC + kRmax;  // own pixel in the LDS tile
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    // Plane of shift 0 for this (b, c); shift s adds s * plane_step (= B*C*HW).
    const T* wp = w + (b * C + c) * HW;

    A u[VEC], z[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) u[k] = z[k] = A(0);

    for (int s = 0; s < S; ++s, wp += plane_step) {
        const ShiftRec r = read_shift(shl, s);
        const bool lds = shift_in_lds(r);

        A wv[VEC];
        load_acc<T, VEC>(wp + own, wv);
        A xv[VEC];
        if (lds) {
            const A* xr = xt + lc + r.dx * G::LW + r.dy;
#pragma unroll
            for (int k = 0; k < VEC; ++k) xv[k] = xr[k];
        } else {
            int hh = h + r.dxm;
            hh -= hh >= H ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int ww = w0 + k + r.dym;
                ww -= ww >= W ? W : 0;
                xv[k] = to_acc(xp[static_cast<uint32_t>(hh) * W + ww]);
            }
        }
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            u[k] = __builtin_fma(wv[k], xv[k], u[k]);
            z[k] += wv[k];
        }

        if (r.inv) {
            // Mirror: source pixel p - s, taken only where it lies inside
            // the image (the box test of shift_ops_cuda.cu:313).
            const int off = -(r.dx * W + r.dy);  // valid whenever the box holds
            if (lds && tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, -r.dx, -r.dy)) {
                const A* xr = xt + lc - r.dx * G::LW - r.dy;
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const A wi = to_acc(wp[static_cast<int64_t>(own) + off + k]);
                    u[k] = __builtin_fma(wi, xr[k], u[k]);
                    z[k] += wi;
                }
            } else {
                const int hs = h - r.dx;
                const bool rok = in_range(hs, H);
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const int ws = w0 + k - r.dy;
                    if (rok && in_range(ws, W)) {
                        const uint32_t src = static_cast<uint32_t>(hs) * W + ws;
                        const A wi = to_acc(wp[src]);
                        const A xi = lds ? xt[lc - r.dx * G::LW - r.dy + k] : to_acc(xp[src]);
                        u[k] = __builtin_fma(wi, xi, u[k]);
                        z[k] += wi;
                    }
                }
            }
        }
    }
    store_out<A, VEC>(U + ti.bc * HW + own, u);
    store_out<A, VEC>(Z + ti.bc * HW + own, z);
}

// ---------------------------------------------------------------------------
// Fused backward: one pass over the weight planes produces gw (written once)
// and gx (register sums).  x, gU and gZ tiles with halo live in LDS.
// ---------------------------------------------------------------------------
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void accumulate_uz_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const acc_t<T>* __restrict__ gU,
    const acc_t<T>* __restrict__ gZ, const int64_t* __restrict__ shifts, int S, int C, int H,
    int W, int ntw, int nth, int64_t plane_step, T* __restrict__ gx, T* __restrict__ gw) {
    using A = acc_t<T>;
    using G = Geo<VEC>;
    constexpr int LT = G::LH * G::LW;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));
    A* ut = xt + LT;
    A* zt = ut + LT;

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;
    const A* up = gU + ti.bc * HW;
    const A* zp = gZ + ti.bc * HW;

    stage_shifts(shl, shifts, S, 3, H, W);
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(ut, up, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(zt, zp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    __syncthreads();

    const int tx = threadIdx.x % kTPR;
    const int ty = threadIdx.x / kTPR;
    const int h = ti.h0 + ty;
    const int w0 = ti.w0 + tx * VEC;
    if (h >= H || w0 >= W) return;

    const uint32_t own = static_cast<uint32_t>(h) * static_cast<uint32_t>(W) + w0;
    const int lc = (ty + kRmax) * G::LW + tx * VEC + kRmax;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* wp = w + (b * C + c) * HW;
    T* gp = gw + (b * C + c) * HW;

    A xo[VEC], uo[VEC], zo[VEC], gxa[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        xo[k] = xt[lc + k];
        uo[k] = ut[lc + k];
        zo[k] = zt[lc + k];
        gxa[k] = A(0);
    }

    for (int s = 0; s < S; ++s, wp += plane_step, gp += plane_step) {
        const ShiftRec r = read_shift(shl, s);
        const bool lds = shift_in_lds(r);

        // Values at q + s (circular for the forward term, box for the mirror)
        // and at q - s (circular) for the gx forward term.
        A xf[VEC], up_[VEC], zp_[VEC], um[VEC];
        bool okp[VEC];
        const bool plus_inside = tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, r.dx, r.dy);
        if (lds) {
            const A* xr = xt + lc + r.dx * G::LW + r.dy;
            const A* ur = ut + lc + r.dx * G::LW + r.dy;
            const A* zr = zt + lc + r.dx * G::LW + r.dy;
            const A* um_r = ut + lc - r.dx * G::LW - r.dy;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                xf[k] = xr[k];
                up_[k] = ur[k];
                zp_[k] = zr[k];
                um[k] = um_r[k];
            }
        } else {
            int hp = h + r.dxm;
            hp -= hp >= H ? H : 0;
            int hm = h - r.dxm;
            hm += hm < 0 ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int wq = w0 + k + r.dym;
                wq -= wq >= W ? W : 0;
                int wm = w0 + k - r.dym;
                wm += wm < 0 ? W : 0;
                const uint32_t ip = static_cast<uint32_t>(hp) * W + wq;
                const uint32_t im = static_cast<uint32_t>(hm) * W + wm;
                xf[k] = to_acc(xp[ip]);
                up_[k] = up[ip];
                zp_[k] = zp[ip];
                um[k] = up[im];
            }
        }
        if (plus_inside) {
#pragma unroll
            for (int k = 0; k < VEC; ++k) okp[k] = true;
        } else {
            const bool rok = in_range(h + r.dx, H);
#pragma unroll
            for (int k = 0; k < VEC; ++k) okp[k] = rok && in_range(w0 + k + r.dy, W);
        }

        // gw_s[q]
        A g[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) g[k] = __builtin_fma(xf[k], uo[k], zo[k]);
        if (r.inv) {
#pragma unroll
            for (int k = 0; k < VEC; ++k)
                if (okp[k]) g[k] += __builtin_fma(xo[k], up_[k], zp_[k]);
        }
        store_acc<T, VEC>(gp + own, g, true);

        // gx[q]: forward term w_s[(q-s) mod] gU[(q-s) mod]
        if (tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, -r.dx, -r.dy)) {
            const int off = -(r.dx * W + r.dy);
#pragma unroll
            for (int k = 0; k < VEC; ++k)
                gxa[k] = __builtin_fma(to_acc(wp[static_cast<int64_t>(own) + off + k]), um[k], gxa[k]);
        } else {
            int hm = h - r.dxm;
            hm += hm < 0 ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int wm = w0 + k - r.dym;
                wm += wm < 0 ? W : 0;
                gxa[k] = __builtin_fma(to_acc(wp[static_cast<uint32_t>(hm) * W + wm]), um[k], gxa[k]);
            }
        }
        // gx[q]: mirror term w_s[q] gU[q+s] where box(q+s)
        if (r.inv) {
            A wv[VEC];
            load_acc<T, VEC>(wp + own, wv);
#pragma unroll
            for (int k = 0; k < VEC; ++k)
                if (okp[k]) gxa[k] = __builtin_fma(wv[k], up_[k], gxa[k]);
        }
    }
    store_acc<T, VEC>(gx + ti.bc * HW + own, gxa, false);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int VEC>
static size_t fwd_lds(int S, size_t acc_bytes) {
    return static_cast<size_t>(S) * sizeof(int4) + static_cast<size_t>(Geo<VEC>::LH) * Geo<VEC>::LW * acc_bytes;
}
template <int VEC>
static size_t bwd_lds(int S, size_t acc_bytes) {
    return static_cast<size_t>(S) * sizeof(int4) +
           3 * static_cast<size_t>(Geo<VEC>::LH) * Geo<VEC>::LW * acc_bytes;
}

constexpr size_t kLdsLimit = 64 * 1024;

struct Dims {
    int S, B, C, H, W;
};

template <typename T, int VEC>
static int launch_fwd(const void* x, const void* w, const int64_t* shifts, Dims d, void* U,
                      void* Z, hipStream_t st) {
    using G = Geo<VEC>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const size_t lds = fwd_lds<VEC>(d.S, sizeof(acc_t<T>));
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    hipLaunchKernelGGL((accumulate_uz_fwd_kernel<T, VEC>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), lds, st, static_cast<const T*>(x),
                       static_cast<const T*>(w), shifts, d.S, d.C, d.H, d.W, ntw, nth, step,
                       static_cast<acc_t<T>*>(U), static_cast<acc_t<T>*>(Z));
    return nsh_host::check_launch("accumulate_uz_forward");
}

template <typename T, int VEC>
static int launch_bwd(const void* x, const void* w, const void* gU, const void* gZ,
                      const int64_t* shifts, Dims d, void* gx, void* gw, hipStream_t st) {
    using G = Geo<VEC>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const size_t lds = bwd_lds<VEC>(d.S, sizeof(acc_t<T>));
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    hipLaunchKernelGGL((accumulate_uz_bwd_kernel<T, VEC>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), lds, st, static_cast<const T*>(x),
                       static_cast<const T*>(w), static_cast<const acc_t<T>*>(gU),
                       static_cast<const acc_t<T>*>(gZ), shifts, d.S, d.C, d.H, d.W, ntw, nth,
                       step, static_cast<T*>(gx), static_cast<T*>(gw));
    return nsh_host::check_launch("accumulate_uz_backward");
}

// Widest vector such that every row start is aligned for it and the LDS
// budget holds; VEC = 1 handles any shape.
template <typename T>
static int pick_vec(int W, std::initializer_list<const void*> ptrs, int S, bool bwd) {
    const int maxv = 16 / static_cast<int>(sizeof(T));
    for (int v = maxv; v > 1; v /= 2) {
        if (W % v) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && nsh_host::aligned(p, v * sizeof(T));
        if (!ok) continue;
        size_t lds = 0;
        switch (v) {
            case 8: lds = bwd ? bwd_lds<8>(S, sizeof(acc_t<T>)) : fwd_lds<8>(S, sizeof(acc_t<T>)); break;
            case 4: lds = bwd ? bwd_lds<4>(S, sizeof(acc_t<T>)) : fwd_lds<4>(S, sizeof(acc_t<T>)); break;
            default: lds = bwd ? bwd_lds<2>(S, sizeof(acc_t<T>)) : fwd_lds<2>(S, sizeof(acc_t<T>)); break;
        }
        if (lds <= kLdsLimit) return v;
    }
    return 1;
}

template <typename T>
static int run_fwd(const void* x, const void* w, const int64_t* shifts, Dims d, void* U, void* Z,
                   hipStream_t st) {
    switch (pick_vec<T>(d.W, {x, w, U, Z}, d.S, false)) {
        case 8: if constexpr (sizeof(T) == 2) return launch_fwd<T, 8>(x, w, shifts, d, U, Z, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return launch_fwd<T, 4>(x, w, shifts, d, U, Z, st); break;
        case 2: return launch_fwd<T, 2>(x, w, shifts, d, U, Z, st);
        default: break;
    }
    return launch_fwd<T, 1>(x, w, shifts, d, U, Z, st);
}

template <typename T>
static int run_bwd(const void* x, const void* w, const void* gU, const void* gZ,
                   const int64_t* shifts, Dims d, void* gx, void* gw, hipStream_t st) {
    switch (pick_vec<T>(d.W, {x, w, gU, gZ, gx, gw}, d.S, true)) {
        case 8: if constexpr (sizeof(T) == 2) return launch_bwd<T, 8>(x, w, gU, gZ, shifts, d, gx, gw, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return launch_bwd<T, 4>(x, w, gU, gZ, shifts, d, gx, gw, st); break;
        case 2: return launch_bwd<T, 2>(x, w, gU, gZ, shifts, d, gx, gw, st);
        default: break;
    }
    return launch_bwd<T, 1>(x, w, gU, gZ, shifts, d, gx, gw, st);
}

}  // namespace nsh

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using nsh_host::fail;

static int check_acc_dims(const char* op, int64_t S, int64_t B, int64_t C, int64_t H, int64_t W,
                          int dtype, nsh::Dims* d) {
    if (S < 1 || S > 1024)
        return fail(NSH_ERR_INVALID, "%s: tree reduction requires 1 <= S <= 1024", op);
    if (B < 1 || C < 1 || H < 1 || W < 1)
        return fail(NSH_ERR_INVALID, "%s: empty tensor (B=%lld C=%lld H=%lld W=%lld)", op,
                    (long long)B, (long long)C, (long long)H, (long long)W);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;  // widest per-plane element (acc)
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (B * C > (int64_t(1) << 24))
        return fail(NSH_ERR_INVALID, "%s: B*C too large", op);
    d->S = static_cast<int>(S);
    d->B = static_cast<int>(B);
    d->C = static_cast<int>(C);
    d->H = static_cast<int>(H);
    d->W = static_cast<int>(W);
    return NSH_OK;
}

extern "C" int nsh_accumulate_uz_forward(const void* x, const void* weights, const int64_t* shifts,
                                         int64_t S, int64_t B, int64_t C, int64_t H, int64_t W,
                                         int dtype, void* U, void* Z, void* stream) {
    nsh::Dims d;
    if (int rc = check_acc_dims("accumulate_uz", S, B, C, H, W, dtype, &d)) return rc;
    if (!x || !weights || !shifts || !U || !Z)
        return fail(NSH_ERR_INVALID, "accumulate_uz: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::run_fwd<nsh::f16>(x, weights, shifts, d, U, Z, st);
        case NSH_DTYPE_BFLOAT16: return nsh::run_fwd<nsh::bf16>(x, weights, shifts, d, U, Z, st);
        case NSH_DTYPE_FLOAT32: return nsh::run_fwd<float>(x, weights, shifts, d, U, Z, st);
        default: return nsh::run_fwd<double>(x, weights, shifts, d, U, Z, st);
    }
}

extern "C" int nsh_accumulate_uz_backward(const void* x, const void* weights, const void* grad_U,
                                          const void* grad_Z, const int64_t* shifts, int64_t S,
                                          int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                                          void* grad_x, void* grad_w, void* stream) {
    nsh::Dims d;
    if (int rc = check_acc_dims("accumulate_uz_backward", S, B, C, H, W, dtype, &d)) return rc;
    if (!x || !weights || !grad_U || !grad_Z || !shifts || !grad_x || !grad_w)
        return fail(NSH_ERR_INVALID, "accumulate_uz_backward: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            return nsh::run_bwd<nsh::f16>(x, weights, grad_U, grad_Z, shifts, d, grad_x, grad_w, st);
        case NSH_DTYPE_BFLOAT16:
            return nsh::run_bwd<nsh::bf16>(x, weights, grad_U, grad_Z, shifts, d, grad_x, grad_w, st);
        case NSH_DTYPE_FLOAT32:
            return nsh::run_bwd<float>(x, weights, grad_U, grad_Z, shifts, d, grad_x, grad_w, st);
        default:
            return nsh::run_bwd<double>(x, weights, grad_U, grad_Z, shifts, d, grad_x, grad_w, st);
    }
}
