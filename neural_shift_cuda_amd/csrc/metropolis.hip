// metropolis.hip -- fused Metropolis-Hastings aggregation (inference) on gfx950.
//
// Semantics (reference csrc/metropolis_cuda.cu:70-240, metropolis.py:54-114):
//   w_half is batch-major (B, S, C, H, W): plane (b, s, c).  For shift s the
//   forward edge of pixel p goes to j = (p+s) mod with weight w_s[p]; the
//   inverse twin (has_inv rows) goes to j = (p-s) mod with the circularly
//   shifted forward weight w_s[j].  With use_box, an edge whose neighbour is
//   reached only by wrap-around is dropped.
//     pass 1: d[p]   = sum of p's edge weights                    (K e)
//     pass 2: wk     = w / max(d_p, d_j, eps) per edge            (K_hat)
//             khat_x = sum wk img[j],  d_hat = sum wk
//             Wx     = img - d_hat img + khat_x   (fused: no extra pass)
//   Each edge weight is formed from the same stored element and the same
//   symmetric denominator on both of its endpoints, so K_hat (and W) is
//   exactly symmetric.
// Both passes use the accumulate_uz tile layout: the image and degree tiles
// with a kRmax halo sit in LDS, weights stream from HBM once per pass (the
// inverse term's shifted re-read is an L1/L2 hit).
#include <initializer_list>

#include "nsh_common.hpp"

namespace nsh {

template <int VEC>
struct MGeo {
    static constexpr int TW = kTPR * VEC;
    static constexpr int TH = kRows;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
};

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void metropolis_degree_kernel(
    const T* __restrict__ wh, const int64_t* __restrict__ shifts, int S, int C, int H, int W,
    int ntw, int nth, int use_box, acc_t<T>* __restrict__ d) {
    using A = acc_t<T>;
    using G = MGeo<VEC>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    stage_shifts(shl, shifts, S, 3, H, W);

    const int tx = threadIdx.x % kTPR;
    const int ty = threadIdx.x / kTPR;
    const int h = ti.h0 + ty;
    const int w0 = ti.w0 + tx * VEC;
    if (h >= H || w0 >= W) return;
    const uint32_t own = static_cast<uint32_t>(h) * static_cast<uint32_t>(W) + w0;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* wp = wh + (b * S * C + c) * HW;  // plane (b, 0, c); shift s adds C*HW
    const int64_t step = static_cast<int64_t>(C) * HW;

    A acc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = A(0);

    for (int s = 0; s < S; ++s, wp += step) {
        const ShiftRec r = read_shift(shl, s);
        A wv[VEC];
        load_acc<T, VEC>(wp + own, wv);
        const bool frow = in_range(h + r.dx, H);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const bool keep = !use_box || (frow && in_range(w0 + k + r.dy, W));
            acc[k] += keep ? wv[k] : A(0);
        }
        if (r.inv) {
            int hm = h - r.dxm;
            hm += hm < 0 ? H : 0;
            const bool irow = in_range(h - r.dx, H);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const bool keep = !use_box || (irow && in_range(w0 + k - r.dy, W));
                if (keep) {
                    int wm = w0 + k - r.dym;
                    wm += wm < 0 ? W : 0;
                    acc[k] += to_acc(wp[static_cast<uint32_t>(hm) * W + wm]);
                }
            }
        }
    }
    store_out<A, VEC>(d + ti.bc * HW + own, acc);
}

template <typename A>
__device__ __forceinline__ A metro_wk(A wv, A di, A dj, A eps) {
    const A den = di > dj ? di : dj;
    return wv / (den > eps ? den : eps);
}

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void metropolis_aggregate_kernel(
    const T* __restrict__ wh, const T* __restrict__ img, const acc_t<T>* __restrict__ d,
    const int64_t* __restrict__ shifts, int S, int C, int H, int W, int ntw, int nth, int use_box,
    acc_t<T> eps, T* __restrict__ Wx, T* __restrict__ dhat) {
    using A = acc_t<T>;
    using G = MGeo<VEC>;
    constexpr int LT = G::LH * G::LW;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* it = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));
    A* dt = it + LT;

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* ip = img + ti.bc * HW;
    const A* dp = d + ti.bc * HW;
    stage_shifts(shl, shifts, S, 3, H, W);
    stage_tile<T, A>(it, ip, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(dt, dp, H, W, ti.h0, ti.w0, G::LH, G::LW);
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
    const T* wp = wh + (b * S * C + c) * HW;
    const int64_t step = static_cast<int64_t>(C) * HW;

    A di[VEC], kx[VEC], dh[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        di[k] = dt[lc + k];
        kx[k] = A(0);
        dh[k] = A(0);
    }

    for (int s = 0; s < S; ++s, wp += step) {
        const ShiftRec r = read_shift(shl, s);
        const bool lds = shift_in_lds(r);
        A wv[VEC];
        load_acc<T, VEC>(wp + own, wv);
        // forward edge j = (p+s) mod
        {
            const bool frow = in_range(h + r.dx, H);
            int hp = h + r.dxm;
            hp -= hp >= H ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const bool keep = !use_box || (frow && in_range(w0 + k + r.dy, W));
                A dj, vj;
                if (lds) {
                    dj = dt[lc + r.dx * G::LW + r.dy + k];
                    vj = it[lc + r.dx * G::LW + r.dy + k];
                } else {
                    int wq = w0 + k + r.dym;
                    wq -= wq >= W ? W : 0;
                    const uint32_t j = static_cast<uint32_t>(hp) * W + wq;
                    dj = dp[j];
                    vj = to_acc(ip[j]);
                }
                if (keep) {
                    const A wk = metro_wk(wv[k], di[k], dj, eps);
                    kx[k] = fma_acc(wk, vj, kx[k]);
                    dh[k] += wk;
                }
            }
        }
        // inverse edge j = (p-s) mod, weight w_s[j]
        if (r.inv) {
            const bool irow = in_range(h - r.dx, H);
            int hm = h - r.dxm;
            hm += hm < 0 ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const bool keep = !use_box || (irow && in_range(w0 + k - r.dy, W));
                if (keep) {
                    int wm = w0 + k - r.dym;
                    wm += wm < 0 ? W : 0;
                    const uint32_t j = static_cast<uint32_t>(hm) * W + wm;
                    const A wj = to_acc(wp[j]);
                    A dj, vj;
                    if (lds) {
                        dj = dt[lc - r.dx * G::LW - r.dy + k];
                        vj = it[lc - r.dx * G::LW - r.dy + k];
                    } else {
                        dj = dp[j];
                        vj = to_acc(ip[j]);
                    }
                    const A wk = metro_wk(wj, di[k], dj, eps);
                    kx[k] = fma_acc(wk, vj, kx[k]);
                    dh[k] += wk;
                }
            }
        }
    }
    A wx[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const A xi = it[lc + k];
        wx[k] = xi - dh[k] * xi + kx[k];
    }
    store_acc<T, VEC>(Wx + ti.bc * HW + own, wx, false);
    store_acc<T, VEC>(dhat + ti.bc * HW + own, dh, false);
}

constexpr size_t kMLdsLimit = 64 * 1024;

template <typename T>
static size_t m_lds(int v, int S) {
    const size_t ab = sizeof(acc_t<T>);
    size_t tile = 0;
    switch (v) {
        case 8: tile = static_cast<size_t>(MGeo<8>::LH) * MGeo<8>::LW; break;
        case 4: tile = static_cast<size_t>(MGeo<4>::LH) * MGeo<4>::LW; break;
        case 2: tile = static_cast<size_t>(MGeo<2>::LH) * MGeo<2>::LW; break;
        default: tile = static_cast<size_t>(MGeo<1>::LH) * MGeo<1>::LW; break;
    }
    return static_cast<size_t>(S) * sizeof(int4) + 2 * tile * ab;
}

template <typename T, int VEC>
static int m_launch(const void* wh, const void* img, const int64_t* sh, int B, int S, int C, int H,
                    int W, int use_box, double eps, void* Wx, void* dhat, void* deg,
                    hipStream_t st) {
    using G = MGeo<VEC>;
    using A = acc_t<T>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(H, G::TH));
    const int64_t tiles = static_cast<int64_t>(B) * C * ntw * nth;
    hipLaunchKernelGGL((metropolis_degree_kernel<T, VEC>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), static_cast<size_t>(S) * sizeof(int4), st,
                       static_cast<const T*>(wh), sh, S, C, H, W, ntw, nth, use_box,
                       static_cast<A*>(deg));
    if (int rc = nsh_host::check_launch("metropolis_aggregate (degree)")) return rc;
    hipLaunchKernelGGL((metropolis_aggregate_kernel<T, VEC>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), m_lds<T>(VEC, S), st, static_cast<const T*>(wh),
                       static_cast<const T*>(img), static_cast<const A*>(deg), sh, S, C, H, W, ntw,
                       nth, use_box, static_cast<A>(eps), static_cast<T*>(Wx),
                       static_cast<T*>(dhat));
    return nsh_host::check_launch("metropolis_aggregate (aggregate)");
}

template <typename T>
static int m_run(const void* wh, const void* img, const int64_t* sh, int B, int S, int C, int H,
                 int W, int use_box, double eps, void* Wx, void* dhat, void* deg, hipStream_t st) {
    int v = 1;
    for (int cand = 16 / static_cast<int>(sizeof(T)); cand > 1; cand /= 2) {
        if (W % cand) continue;
        bool ok = true;
        for (const void* p : std::initializer_list<const void*>{wh, img, Wx, dhat})
            ok = ok && nsh_host::aligned(p, cand * sizeof(T));
        ok = ok && nsh_host::aligned(deg, cand * sizeof(acc_t<T>));
        if (ok && m_lds<T>(cand, S) <= kMLdsLimit) {
            v = cand;
            break;
        }
    }
    switch (v) {
        case 8: if constexpr (sizeof(T) == 2) return m_launch<T, 8>(wh, img, sh, B, S, C, H, W, use_box, eps, Wx, dhat, deg, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return m_launch<T, 4>(wh, img, sh, B, S, C, H, W, use_box, eps, Wx, dhat, deg, st); break;
        case 2: return m_launch<T, 2>(wh, img, sh, B, S, C, H, W, use_box, eps, Wx, dhat, deg, st);
        default: break;
    }
    return m_launch<T, 1>(wh, img, sh, B, S, C, H, W, use_box, eps, Wx, dhat, deg, st);
}

}  // namespace nsh

using nsh_host::fail;

extern "C" int nsh_metropolis_aggregate(const void* w_half, const void* img, const int64_t* shifts,
                                        int64_t B, int64_t S, int64_t C, int64_t H, int64_t W,
                                        int dtype, int use_box, double eps, void* Wx, void* d_hat,
                                        void* degree, void* stream) {
    const char* op = "metropolis_aggregate";
    if (S < 1 || S > 1024) return fail(NSH_ERR_INVALID, "%s: requires 1 <= S <= 1024", op);
    if (B < 1 || C < 1 || H < 1 || W < 1) return fail(NSH_ERR_INVALID, "%s: empty tensor", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (B * C > (int64_t(1) << 24) || B * S * C > (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: B*S*C too large", op);
    if (!w_half || !img || !shifts || !Wx || !d_hat || !degree)
        return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int b = static_cast<int>(B), s = static_cast<int>(S), c = static_cast<int>(C);
    const int h = static_cast<int>(H), w = static_cast<int>(W);
    const int ub = use_box ? 1 : 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::m_run<nsh::f16>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, st);
        case NSH_DTYPE_BFLOAT16: return nsh::m_run<nsh::bf16>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, st);
        case NSH_DTYPE_FLOAT32: return nsh::m_run<float>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, st);
        default: return nsh::m_run<double>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, st);
    }
}
