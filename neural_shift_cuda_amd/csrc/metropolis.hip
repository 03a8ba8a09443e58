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
#include <algorithm>
#include <cstdlib>
#include <initializer_list>
#include <type_traits>

#include "nsh_common.hpp"
#include "scatter.hpp"

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
    stage_shifts(shl, shifts, S, 3, H, W, false);

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

// Metropolis edge weight w / max(d_i, d_j, eps).  Symmetric in (d_i, d_j),
// so both ends of an edge compute the same value.  fp32 multiplies by the
// hardware reciprocal (v_rcp_f32, 1 ulp; den >= eps > 0 is a normal number),
// fp64 divides.
__device__ __forceinline__ float metro_wk(float wv, float di, float dj, float eps) {
    return wv * __builtin_amdgcn_rcpf(__builtin_fmaxf(__builtin_fmaxf(di, dj), eps));
}
__device__ __forceinline__ double metro_wk(double wv, double di, double dj, double eps) {
    return wv / __builtin_fmax(__builtin_fmax(di, dj), eps);
}
// Per-pixel factor rho = 1 / max(d, eps): the edge weight is then
// w * min(rho_i, rho_j), symmetric in its two ends (one min and one multiply
// per edge instead of two max and a reciprocal).
__device__ __forceinline__ float metro_rho(float d, float eps) {
    return __builtin_amdgcn_rcpf(__builtin_fmaxf(d, eps));
}
__device__ __forceinline__ double metro_rho(double d, double eps) {
    return 1.0 / __builtin_fmax(d, eps);
}
__device__ __forceinline__ float metro_wk_rho(float wv, float ri, float rj) {
    return wv * __builtin_fminf(ri, rj);
}
__device__ __forceinline__ double metro_wk_rho(double wv, double ri, double rj) {
    return wv * __builtin_fmin(ri, rj);
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
    A* it = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* dt = it + LT;

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* ip = img + ti.bc * HW;
    const A* dp = d + ti.bc * HW;
    stage_shifts(shl, shifts, S, 3, H, W, false);
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

// ---------------------------------------------------------------------------
// Scatter form: every w_half element is read once per pass, aligned.
//
// The kernels above gather the inverse edge of pixel p from w_s[p - s]: a
// scalar read R rows/columns into the neighbouring tile, mostly missed in
// L2 by the time it is issued.  Both passes below use the adjoint form
// instead.  For shift s the lane owning pixel q holds w_s[q], the weight of
// the edge {q, j = (q + s) mod}.  That one value serves both ends of the
// edge: the forward edge of q (added in registers) and the inverse edge of
// j (added into an LDS window at q + s that covers the tile plus a kRmax
// border).  With use_box an edge is kept iff q + s does not wrap, which is
// the condition of both of its ends (p - s = q without wrap iff q + s does
// not wrap).  Pass 2 forms the edge weight w / max(d_q, d_j, eps) once and
// adds it at both ends, so K_hat stays exactly symmetric.
//
// The window border is spilled to the workspace; pass 1's border goes
// through spill_fixup_kernel (degree, in place), pass 2's through
// metropolis_fixup_kernel, which also finishes Wx on the pixels near a tile
// edge (the main kernel stores their partial sums in the workspace).
// Shifts beyond the LDS halo (|dx| or |dy| > kRmax) keep the gather form
// inside the same kernels; the window radius R counts only the inverse rows
// that scatter.
// ---------------------------------------------------------------------------

// Largest max(|dx|, |dy|) over the rows (has_inverse rows only when
// `only_inv`) that stay within the LDS halo of HALO pixels; uniform across
// the workgroup (every wave computes it).
template <int HALO = kRmax>
__device__ __forceinline__ int near_inverse_radius(const int4* shl, int S, bool only_inv = true) {
    const int lane = threadIdx.x & 63;
    int m = 0;
    for (int s = lane; s < S; s += 64) {
        const int4 r = shl[s];
        if (only_inv && r.z >= 0) continue;
        const int ax = r.x < 0 ? -r.x : r.x;
        const int ay = r.y < 0 ? -r.y : r.y;
        const int a = max(ax, ay);
        if (a <= HALO) m = max(m, a);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    return __builtin_amdgcn_readfirstlane(m);
}

// Weight loads of the two forward scatter passes as nontemporal (streaming)
// loads: c4 forward 8.72 -> 8.45 ms.  The backward edge pass keeps plain
// loads (12.0 -> 12.3 ms with streaming ones).
constexpr bool kMetroNtLoads = true;

// Pass 1: d = K e.  D = weight prefetch depth in shifts.
template <typename T, int VEC, int TPR, int ROWS, int D, bool BOX>
__global__ __launch_bounds__(TPR * ROWS, kScatterWavesPerEU<TPR * ROWS>) void metropolis_degree_scatter_kernel(
    const T* __restrict__ wh, const int64_t* __restrict__ shifts, int S, int C, int H, int W,
    int ntw, int nth, acc_t<T>* __restrict__ d, int* __restrict__ hdr,
    acc_t<T>* __restrict__ spill) {
    constexpr bool use_box = BOX;
    using A = acc_t<T>;
    using G = SGeo<VEC, ROWS, TPR>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* md = reinterpret_cast<A*>(smem + shift_lds_bytes(S));

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    stage_shifts(shl, shifts, S, 3, H, W, false);
    const int R = near_inverse_radius(shl, S);
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr[0] = R;  // for both fix-ups
    lds_zero(md, G::TILE);  // also used at R = 0 by a (0, 0) mirror row
    __syncthreads();

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + kRmax) * G::PITCH + tx + kRmax;  // pixel k at lc + k*TPR
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* wplane = wh + (b * S * C + c) * HW;  // plane (b, 0, c); shift s adds C*HW
    const int64_t step = static_cast<int64_t>(C) * HW;

    A acc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = A(0);
    // Prefetch ring; loads are unconditional (the tail re-reads plane S-1)
    // so that none sits behind a branch.
    // Raw slots promoted where consumed; the next refill's plane and the
    // next shift's record advance one shift at a time.
    PixSlot<T, VEC> wb[D];
#pragma unroll
    for (int dd = 0; dd < D; ++dd)
        slot_load_pixels<T, VEC, TPR, kMetroNtLoads>(
            wplane + static_cast<int64_t>(min(dd, S - 1)) * step, px, wb[dd]);
    const T* wr = wplane + static_cast<int64_t>(min(D, S - 1)) * step;
    ShiftRec rn = read_shift(shl, 0);

    int last_dx = kClamp;
    auto body = [&](int s, PixSlot<T, VEC>& slot) {
        const ShiftRec rc = rn;
        rn = read_shift(shl, min(s + 1, S - 1));
        A wv[VEC];
        slot_get_pixels<T, VEC>(slot, wv);
        slot_load_pixels<T, VEC, TPR, kMetroNtLoads>(wr, px, slot);
        wr += s + D + 1 < S ? step : 0;
        const bool rok = !use_box || in_range(h + rc.dx, H);
        A kw[VEC];  // the edge weight if kept, else 0
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const bool keep =
                px.act[k] && rok && (!use_box || in_range(ti.w0 + tx + k * TPR + rc.dy, W));
            kw[k] = keep ? wv[k] : A(0);
            acc[k] += kw[k];
        }
        if (rc.inv && shift_in_lds(rc)) {
            // Same dx: the wave's targets are its own rows shifted by dx,
            // disjoint from every other wave's; barrier only on a new dx.
            // Every lane adds (0 for a dropped edge or an idle pixel): the
            // targets of one shift are distinct and inside the window.
            if (rc.dx != last_dx) {
                lds_barrier();
                last_dx = rc.dx;
            }
            A* pm = md + lc + rc.dx * G::PITCH + rc.dy;
#pragma unroll
            for (int k = 0; k < VEC; ++k) pm[k * TPR] += kw[k];
        }
    };
    // The ring loop issues no other global load (a conditional load would
    // make the compiler's wait counts drain the prefetch ring).
    const int S_ring = S - S % D;
    for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
        for (int dd = 0; dd < D; ++dd) body(s0 + dd, wb[dd]);
    }
#pragma unroll
    for (int dd = 0; dd < D; ++dd)
        if (S_ring + dd < S) body(S_ring + dd, wb[dd]);
    // Inverse rows beyond the halo: gather form, w_s at j = (p - s) mod.
    for (int s = 0; s < S && px.any; ++s) {
        const ShiftRec rc = read_shift(shl, s);
        if (!rc.inv || shift_in_lds(rc)) continue;
        const bool irow = in_range(h - rc.dx, H);
        int hm = h - rc.dxm;
        hm += hm < 0 ? H : 0;
        const T* wp = wplane + static_cast<int64_t>(s) * step;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const int w = ti.w0 + tx + k * TPR;
            if (px.act[k] && (!use_box || (irow && in_range(w - rc.dy, W)))) {
                int wm = w - rc.dym;
                wm += wm < 0 ? W : 0;
                acc[k] += to_acc(wp[static_cast<uint32_t>(hm) * W + wm]);
            }
        }
    }

    A* dout = d + ti.bc * HW;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!px.act[k]) continue;
        dout[px.own[k]] = acc[k] + md[lc + k * TPR];
    }
    if (R == 0) return;
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    const int n = spill_count(th, tw, R);
    A* sd = spill + t * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        sd[e] = md[(i + kRmax) * G::PITCH + j + kRmax];
    }
}

// Pass 2: K_hat x and d_hat = K_hat e, then Wx = x - d_hat x + K_hat x.
// LDS holds (image, rho = 1/max(degree, eps)) pairs of the tile plus halo and
// (K_hat x, d_hat) pairs of the window, so each neighbour costs one 8-byte LDS
// read and each mirror term one read-modify-write.  Pixels within R of the tile edge still
// miss their neighbours' spills: the kernel stores their partial sums (ring
// slot order) in `part` (two arrays of ring_stride entries per tile) and
// metropolis_fixup_kernel finishes them.
template <typename T, int VEC, int TPR, int ROWS, int D, bool BOX, int WPE>
__global__ __launch_bounds__(TPR * ROWS, WPE) void metropolis_aggregate_scatter_kernel(
    const T* __restrict__ wh, const T* __restrict__ img, const acc_t<T>* __restrict__ d,
    const int64_t* __restrict__ shifts, int S, int C, int H, int W, int ntw, int nth,
    acc_t<T> eps, T* __restrict__ Wx, T* __restrict__ dhat, acc_t<T>* __restrict__ spill,
    acc_t<T>* __restrict__ part, int ring_stride, int64_t ntiles) {
    constexpr bool use_box = BOX;
    using A = acc_t<T>;
    using V2 = A __attribute__((ext_vector_type(2)));
    using G = SGeo<VEC, ROWS, TPR>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    V2* xd = reinterpret_cast<V2*>(smem + shift_lds_bytes(S));  // (x, rho)
    V2* mw = xd + G::TILE;                                                      // (kx, dh)

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t off = ti.bc * HW;
    const T* ip = img + off;
    const A* dp = d + off;
    stage_shifts(shl, shifts, S, 3, H, W, false);
    {
        const bool cheap = H >= G::LH && W >= G::LW;
        for (int i = threadIdx.x; i < G::LH * G::LW; i += blockDim.x) {
            const int r = i / G::LW;
            const int cc = i - r * G::LW;
            int gh = ti.h0 - kRmax + r;
            int gw = ti.w0 - kRmax + cc;
            if (cheap) {
                gh = wrap1(gh, H);
                gw = wrap1(gw, W);
            } else {
                gh = static_cast<int>(mod_pos(gh, H));
                gw = static_cast<int>(mod_pos(gw, W));
            }
            const uint32_t g = static_cast<uint32_t>(gh) * static_cast<uint32_t>(W) +
                               static_cast<uint32_t>(gw);
            V2 v;
            v.x = to_acc(ip[g]);
            v.y = metro_rho(dp[g], eps);
            xd[r * G::PITCH + cc] = v;
        }
    }
    const int R = near_inverse_radius(shl, S);
    // the window is also used at R = 0 by a (0, 0) mirror row
    for (int i = threadIdx.x; i < G::TILE; i += blockDim.x) mw[i] = V2{A(0), A(0)};
    __syncthreads();

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + kRmax) * G::PITCH + tx + kRmax;  // pixel k at lc + k*TPR
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* wplane = wh + (b * S * C + c) * HW;
    const int64_t step = static_cast<int64_t>(C) * HW;

    A xi[VEC], ri[VEC], kx[VEC], dh[VEC];  // ri: own rho
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const V2 v = xd[lc + k * TPR];
        xi[k] = v.x;
        ri[k] = v.y;
        kx[k] = A(0);
        dh[k] = A(0);
    }
    PixSlot<T, VEC> wb[D];  // raw slots, promoted where consumed (see pass 1)
#pragma unroll
    for (int dd = 0; dd < D; ++dd)
        slot_load_pixels<T, VEC, TPR, kMetroNtLoads>(
            wplane + static_cast<int64_t>(min(dd, S - 1)) * step, px, wb[dd]);
    const T* wr = wplane + static_cast<int64_t>(min(D, S - 1)) * step;
    ShiftRec rn = read_shift(shl, 0);

    // Interior tiles (every pixel, and every q + s of the rows within the
    // halo, inside the image) keep every edge: a second copy of the loop
    // without the per-pixel box and activity selects.
    const int R_near = near_inverse_radius(shl, S, false);
    const bool interior = ti.h0 >= R_near && ti.h0 + G::TH + R_near <= H &&
                          ti.w0 >= R_near && ti.w0 + G::TW + R_near <= W;
    int last_dx = kClamp;
    auto run_loop = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        auto body = [&](int s, PixSlot<T, VEC>& slot) {
            const ShiftRec rc = rn;
            rn = read_shift(shl, min(s + 1, S - 1));
            A wv[VEC];
            slot_get_pixels<T, VEC>(slot, wv);
            slot_load_pixels<T, VEC, TPR, kMetroNtLoads>(wr, px, slot);
            wr += s + D + 1 < S ? step : 0;
            if (shift_in_lds(rc)) {
                // Branch-free: every pixel forms its edge weight and selects it.
                const bool rok = !use_box || in_range(h + rc.dx, H);
                const int op = lc + rc.dx * G::PITCH + rc.dy;  // window index of q + s
                A wk[VEC], mx[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const V2 nb = xd[op + k * TPR];
                    const A e = metro_wk_rho(wv[k], ri[k], nb.y);
                    if constexpr (FAST) {
                        wk[k] = e;
                        kx[k] = fma_acc(e, nb.x, kx[k]);
                        mx[k] = e * xi[k];
                    } else {
                        const bool keep = px.act[k] && rok &&
                                          (!use_box || in_range(ti.w0 + tx + k * TPR + rc.dy, W));
                        wk[k] = keep ? e : A(0);
                        kx[k] = keep ? fma_acc(e, nb.x, kx[k]) : kx[k];
                        mx[k] = keep ? e * xi[k] : A(0);
                    }
                    dh[k] += wk[k];
                }
                if (rc.inv) {
                    // as in pass 1: every lane adds, 0 for a dropped edge
                    if (rc.dx != last_dx) {
                        lds_barrier();
                        last_dx = rc.dx;
                    }
                    V2* pm = mw + op;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        V2 m = pm[k * TPR];
                        m.x += mx[k];
                        m.y += wk[k];
                        pm[k * TPR] = m;
                    }
                }
            }
        };
        // The ring loop issues no other global load (a conditional load
        // would make the compiler's wait counts drain the prefetch ring).
        const int S_ring = S - S % D;
        for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
            for (int dd = 0; dd < D; ++dd) body(s0 + dd, wb[dd]);
        }
#pragma unroll
        for (int dd = 0; dd < D; ++dd)
            if (S_ring + dd < S) body(S_ring + dd, wb[dd]);
    };
    if (interior)
        run_loop(std::true_type{});
    else
        run_loop(std::false_type{});
    // Shifts beyond the halo: gather form (as metropolis_aggregate_kernel).
    for (int s = 0; s < S && px.any; ++s) {
        const ShiftRec rc = read_shift(shl, s);
        if (shift_in_lds(rc)) continue;
        const T* wp = wplane + static_cast<int64_t>(s) * step;
        const bool rok = in_range(h + rc.dx, H);
        const bool irow = in_range(h - rc.dx, H);
        int hp = h + rc.dxm;
        hp -= hp >= H ? H : 0;
        int hm = h - rc.dxm;
        hm += hm < 0 ? H : 0;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            if (!px.act[k]) continue;
            const int w = ti.w0 + tx + k * TPR;
            if (!use_box || (rok && in_range(w + rc.dy, W))) {
                int wj = w + rc.dym;
                wj -= wj >= W ? W : 0;
                const uint32_t j = static_cast<uint32_t>(hp) * W + wj;
                const A wk = metro_wk_rho(to_acc(wp[px.own[k]]), ri[k], metro_rho(dp[j], eps));
                kx[k] = fma_acc(wk, to_acc(ip[j]), kx[k]);
                dh[k] += wk;
            }
            if (rc.inv && (!use_box || (irow && in_range(w - rc.dy, W)))) {
                int wm = w - rc.dym;
                wm += wm < 0 ? W : 0;
                const uint32_t j = static_cast<uint32_t>(hm) * W + wm;
                const A wk = metro_wk_rho(to_acc(wp[j]), ri[k], metro_rho(dp[j], eps));
                kx[k] = fma_acc(wk, to_acc(ip[j]), kx[k]);
                dh[k] += wk;
            }
        }
    }

    __syncthreads();
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    A* pk = part + 2 * t * ring_stride;
    A* ph = pk + ring_stride;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!px.act[k]) continue;
        const V2 m = mw[lc + k * TPR];
        kx[k] += m.x;
        dh[k] += m.y;
        if (R > 0) {
            const int slot = ring_slot(ty, tx + k * TPR, th, tw, R);
            if (slot >= 0) {  // finished by the fix-up
                pk[slot] = kx[k];
                ph[slot] = dh[k];
                continue;
            }
        }
        Wx[off + px.own[k]] = from_acc<T>(xi[k] - dh[k] * xi[k] + kx[k]);
        dhat[off + px.own[k]] = from_acc<T>(dh[k]);
    }
    if (R == 0) return;
    const int n = spill_count(th, tw, R);
    A* sk = spill + t * G::SPILL;
    A* sh = spill + (ntiles + t) * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        const V2 m = mw[(i + kRmax) * G::PITCH + j + kRmax];
        sk[e] = m.x;
        sh[e] = m.y;
    }
}

// Finishes the ring pixels of pass 2: K_hat x and d_hat = own partial sums
// plus the neighbouring tiles' spills, then Wx = x - d_hat x + K_hat x.
template <typename T>
__global__ __launch_bounds__(256) void metropolis_fixup_kernel(
    int H, int W, int TH, int TW, int ntw, int nth, int spill_stride, int ring_stride,
    const int* __restrict__ hdr, const acc_t<T>* __restrict__ spill,
    const acc_t<T>* __restrict__ part, int64_t ntiles, const T* __restrict__ img,
    T* __restrict__ Wx, T* __restrict__ dhat) {
    using A = acc_t<T>;
    const int R = __builtin_amdgcn_readfirstlane(hdr[0]);
    if (R == 0) return;
    const FixTile f = fix_tile(blockIdx.x, H, W, TH, TW, ntw, nth);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const A* pk = part + 2 * static_cast<int64_t>(blockIdx.x) * ring_stride;
    const A* ph = pk + ring_stride;
    int lg;
    if (fix_slots_ok(f, R, TW, false, lg)) {
        // ring tiles: the slot enumeration, kFixBatch slots per lane with
        // all their loads issued before any sum (spill_sum's order)
        const FixRing g = fix_ring<false>(f, R, lg, HW, W, spill_stride);
        const int64_t qstride = ntiles * spill_stride;
        const int step = static_cast<int>(blockDim.x);
        for (int s0 = threadIdx.x; s0 < g.n; s0 += step * kFixBatch) {
            int lr[kFixBatch], lc[kFixBatch];
            bool act[kFixBatch];
            uint32_t pp[kFixBatch];
            int64_t e[kFixBatch][3];
            A own[kFixBatch][2], xi[kFixBatch], sv[kFixBatch][2][3];
#pragma unroll
            for (int k = 0; k < kFixBatch; ++k) {
                fix_slot<false>(f, g, s0 + k * step, W, lr[k], lc[k], act[k], pp[k], e[k]);
                const int ri = ring_slot(lr[k], lc[k], f.th, f.tw, R);
                own[k][0] = pk[ri];
                own[k][1] = ph[ri];
                xi[k] = to_acc(img[g.pb + pp[k]]);
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int c = 0; c < 3; ++c)
                        sv[k][q][c] = spill[e[k][c] >= 0 ? q * qstride + e[k][c] : 0];
            }
#pragma unroll
            for (int k = 0; k < kFixBatch; ++k) {
                if (!act[k]) continue;
                A acc[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    acc[q] = A(0);
#pragma unroll
                    for (int c = 0; c < 3; ++c) acc[q] += e[k][c] >= 0 ? sv[k][q][c] : A(0);
                }
                const A kx = own[k][0] + acc[0];
                const A dh = own[k][1] + acc[1];
                Wx[g.pb + pp[k]] = from_acc<T>(xi[k] - dh * xi[k] + kx);
                dhat[g.pb + pp[k]] = from_acc<T>(dh);
            }
        }
        return;
    }
    const int n = ring_count(f.th, f.tw, R);
    for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
        int lr, lc;
        ring_pixel(idx, f.th, f.tw, R, lr, lc);
        A acc[2];
        spill_sum<A, 2>(f, R, lr, lc, spill, ntiles, spill_stride, acc);
        const A kx = pk[idx] + acc[0];
        const A dh = ph[idx] + acc[1];
        const int64_t p = f.bc * HW + static_cast<int64_t>(f.h0 + lr) * W + (f.w0 + lc);
        const A xi = to_acc(img[p]);
        Wx[p] = from_acc<T>(xi - dh * xi + kx);
        dhat[p] = from_acc<T>(dh);
    }
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
    return shift_lds_bytes(S) + 2 * tile * ab;
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
                       dim3(kThreads), shift_lds_bytes(S), st,
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

// ---------------------------------------------------------------------------
// Backward (training).  The reference differentiates its explicit-edge path
// (metropolis.py:117-192: every has_inverse row becomes a forward and a
// mirror edge, d = Z of accumulate_uz, wk = w / clamp(max(d, shifted d), eps),
// then accumulate_uz again) through autograd.  Per weight element w_s[q],
// the edge {q, j = (q+s) mod} with kept weight om (0 for a box-dropped edge),
// m = max(d_q, d_j, eps) and wk = om / m, the same gradients are
//   G      = gWx_q (x_j - x_q) + gdhat_q + [inv] (gWx_j (x_q - x_j) + gdhat_j)
//          = a_q x_j + b_q + [inv] (a_j x_q + b_j),  a = gWx, b = gdhat - gWx x
//   mu     = -G wk / m  (d(loss)/dm; zero when max(d_q, d_j) < eps, the clamp)
//   gd_q  += mu s_q,  gd_j += mu (1 - s_q)   (s_q = 1, 1/2 or 0 as d_q >, ==, < d_j:
//                                              torch.maximum's tie rule)
//   gx_j  += wk a_q,  gx_q += [inv] wk a_j,  gx += gWx (1 - dhat)
//   gw_s[q] = [kept] (G / m + gd_q + [inv] gd_j)
// Pass 1 (metropolis_bwd_edge_kernel) scatters gd and gx through an LDS
// window (every near row scatters: its far end's degree enters m), its
// border through the workspace and spill_fixup_kernel; pass 2
// (metropolis_bwd_weight_kernel) streams gw out, reading no weights, and
// converts gx.  Shifts
// beyond the LDS halo take the gather form in separate loops.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float fmax_acc(float a, float b) { return __builtin_fmaxf(a, b); }
__device__ __forceinline__ double fmax_acc(double a, double b) { return __builtin_fmax(a, b); }
__device__ __forceinline__ float fmin_acc(float a, float b) { return __builtin_fminf(a, b); }
__device__ __forceinline__ double fmin_acc(double a, double b) { return __builtin_fmin(a, b); }
// 1/m as the forward forms it (fp32: v_rcp_f32; fp64: divide)
__device__ __forceinline__ float rcp_acc(float m) { return __builtin_amdgcn_rcpf(m); }
__device__ __forceinline__ double rcp_acc(double m) { return 1.0 / m; }

// rho = 1 / max(d, eps) per pixel.  The edge factor 1 / max(d_q, d_j, eps)
// of the forward is then min(rho_q, rho_j): the reciprocal does not increase
// with its argument, so one min replaces two max and a reciprocal per edge.
template <typename A>
__device__ __forceinline__ A m_rho(A d, A eps) {
    return rcp_acc(fmax_acc(d, eps));
}

// min of two rho values known to be positive and not NaN (eps > 0): their
// bit patterns order as unsigned integers, which skips the NaN quieting a
// float min needs.
__device__ __forceinline__ float min_pos(float a, float b) {
    return __uint_as_float(min(__float_as_uint(a), __float_as_uint(b)));
}
__device__ __forceinline__ double min_pos(double a, double b) { return __builtin_fmin(a, b); }

// G = a_q x_j + b_q + [inv] (a_j x_q + b_j)
template <typename A>
__device__ __forceinline__ A m_G(A aq, A xj, A bq, A aj, A xq, A bj, bool inv) {
    const A g = fma_acc(aq, xj, bq);
    return inv ? g + fma_acc(aj, xq, bj) : g;
}

// The share of d(loss)/dm that goes to the end with degree `mine`:
// torch.maximum's rule (all of it to the larger, half each on a tie).  The
// other end's share is mu minus this, exactly.
template <typename A>
__device__ __forceinline__ A tie_part(A mu, A mine, A other) {
    return mine > other ? mu : (mine == other ? A(0.5) * mu : A(0));
}

// The same rule as two shares, 1, 1/2 or 0 for `mine` and 1 minus that for
// `other`, from clamped products: (mine - other) * 2^K + 1/2 clamped to [0, 1].
// Exact when both degrees are at least kTieMinEps (the FAST tiles' gate):
// two distinct such values differ by at least 2^(1-K), so the scaled
// difference lies outside (-1/2, 1/2) unless it is 0 (then both shares are
// 1/2), and an overflow to infinity clamps to 0 or 1.  Two clamped FMAs
// replace two compares and three selects per edge end.
template <typename A> struct TieScale;
template <> struct TieScale<float> {
    static constexpr float kScale = 0x1p126f;    // K = 126
    static constexpr float kMinEps = 0x1p-104f;  // ulp(2^-104) = 2^-127
};
template <> struct TieScale<double> {
    static constexpr double kScale = 0x1p1022;
    static constexpr double kMinEps = 0x1p-970;  // ulp(2^-970) = 2^-1022
};
__device__ __forceinline__ float clamp01(float v) { return __builtin_amdgcn_fmed3f(v, 0.0f, 1.0f); }
__device__ __forceinline__ double clamp01(double v) {
    return __builtin_fmin(__builtin_fmax(v, 0.0), 1.0);
}
template <typename A>
__device__ __forceinline__ void tie_shares(A mine, A other, A& s_mine, A& s_other) {
    const A d = mine - other;
    s_mine = clamp01(fma_acc(d, TieScale<A>::kScale, A(0.5)));
    s_other = clamp01(fma_acc(d, -TieScale<A>::kScale, A(0.5)));
}

// Pass 1.  FAST tiles (uniform per workgroup): every pixel of the tile is in
// the image, no near edge is dropped by the box (the tile and its halo lie
// inside the image) and no staged degree is below eps (clamp gate open on
// every near edge), so the per-edge masks drop out; with eps at least
// TieScale::kMinEps the tie rule takes the clamped form (tie_shares).
// Waves per SIMD the launch bounds ask for: the fp64 edge pass holds one
// workgroup per CU (its LDS; the fp32 one two), the weight pass two.
template <int THREADS, int BLOCKS>
constexpr int kMBwdWaves = BLOCKS * THREADS / 256 > 0 ? BLOCKS * THREADS / 256 : 1;

// Nontemporal weight loads in the edge pass: c4 backward 12.0 -> 11.8-12.0 ms,
// within the run-to-run spread; left off.
constexpr bool kMBwdEdgeNtLoads = false;

// Pass-1 tile geometry.  HALO = kRmax: SGeo's.  The narrow border (HALO <
// kRmax, fp32-class types, for tables whose near shifts all lie within it)
// stores its rows at the plain LW pitch -- the pass-1 arrays are 8-byte
// cells that two 32-lane rows of a wave read, covering every bank at any
// pitch -- and keeps no rho array (rho = 1/max(d, eps) is formed from the
// staged degree where it is used), so that three 512-lane workgroups share a
// CU.  The spill stride stays the kRmax border's: the workspace does not
// depend on the border.
template <int VEC, int ROWS, int TPR, int HALO>
struct MEdgeGeo : SGeo<VEC, ROWS, TPR, true, HALO> {
    using Base = SGeo<VEC, ROWS, TPR, true, HALO>;
    static constexpr bool kRhoLds = HALO == kRmax;
    static constexpr int PITCH = kRhoLds ? Base::PITCH : Base::LW;
    static constexpr int TILE = Base::LH * PITCH;
    static constexpr int SPILL = SGeo<VEC, ROWS, TPR>::SPILL;
    static constexpr int WORDS = kRhoLds ? 7 : 6;  // accumulator words per cell
};
constexpr int kMNarrowHalo = 6;

// Register budget: the kRmax border's LDS admits two workgroups per CU (the
// fp64 one one), the narrow border's three, which need six waves per SIMD.
template <typename T, int VEC, int TPR, int ROWS, int D, bool BOX, int HALO = kRmax>
__global__ __launch_bounds__(TPR * ROWS, (kMBwdWaves<TPR * ROWS, HALO == kRmax ? 1 : 3>)) void
metropolis_bwd_edge_kernel(const T* __restrict__ wh, const T* __restrict__ img,
                           const acc_t<T>* __restrict__ deg, const T* __restrict__ dhat,
                           const T* __restrict__ gWx, const T* __restrict__ gdh,
                           const int64_t* __restrict__ shifts, int S, int C, int H, int W, int ntw,
                           int nth, acc_t<T> eps, acc_t<T>* __restrict__ gd,
                           acc_t<T>* __restrict__ gxp, int* __restrict__ hdr,
                           acc_t<T>* __restrict__ spill, int64_t ntiles) {
    using A = acc_t<T>;
    using V2 = A __attribute__((ext_vector_type(2)));
    using G = MEdgeGeo<VEC, ROWS, TPR, HALO>;
    static_assert(G::kRhoLds || sizeof(A) == 4, "the narrow border is built for fp32 sums");
    constexpr bool use_box = BOX;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    V2* dxt = reinterpret_cast<V2*>(smem + shift_lds_bytes(S));  // (d, x)
    V2* abt = dxt + G::TILE;                                                         // (a, b)
    V2* mw = abt + G::TILE;                                        // (gd, gx) window
    A* rht = reinterpret_cast<A*>(mw + G::TILE);                   // rho (kRhoLds)

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t off = ti.bc * HW;
    stage_shifts(shl, shifts, S, 3, H, W, false);

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + HALO) * G::PITCH + tx + HALO;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* wplane = wh + (b * S * C + c) * HW;
    const int64_t step = static_cast<int64_t>(C) * HW;
    // the weight stream does not depend on the staged tiles: start it first
    // (raw slots, promoted where consumed; the next refill's plane advances
    // one shift at a time)
    PixSlot<T, VEC> wb[D];
#pragma unroll
    for (int dd = 0; dd < D; ++dd)
        slot_load_pixels<T, VEC, TPR, kMBwdEdgeNtLoads>(wplane + static_cast<int64_t>(min(dd, S - 1)) * step, px,
                                      wb[dd]);
    const T* wr = wplane + static_cast<int64_t>(min(D, S - 1)) * step;

    // Stage (d, x), (a, b) and (on the kRmax border) rho for the tile and its
    // halo: every load of the thread is issued before the first LDS write.
    int low = 0;  // a staged degree below eps (or NaN)
    {
        constexpr int NT = TPR * ROWS;
        constexpr int NCELL = G::LH * G::LW;
        constexpr int NST = (NCELL + NT - 1) / NT;
        const bool cheap = H >= G::LH && W >= G::LW;
        A sd[NST], sx[NST], sa[NST], sg[NST];
        int sl[NST];
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const int i = threadIdx.x + u * NT;
            sl[u] = 0;
            if ((u + 1) * NT <= NCELL || i < NCELL) {
                const int64_t g = off + halo_offset<HALO>(i, G::LW, ti.h0, ti.w0, H, W, cheap);
                sd[u] = deg[g];
                sx[u] = to_acc(img[g]);
                sa[u] = to_acc(gWx[g]);
                sg[u] = to_acc(gdh[g]);
                const int r = i / G::LW;
                sl[u] = r * G::PITCH + (i - r * G::LW);
            }
        }
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            if ((u + 1) * NT <= NCELL || threadIdx.x + u * NT < NCELL) {
                const int li = sl[u];
                low |= !(sd[u] >= eps);
                dxt[li] = V2{sd[u], sx[u]};
                abt[li] = V2{sa[u], sg[u] - sa[u] * sx[u]};
                if constexpr (G::kRhoLds) rht[li] = m_rho(sd[u], eps);
            }
        }
    }
    const int R = near_inverse_radius<HALO>(shl, S, false);
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr[0] = R;  // for the fix-up
    for (int i = threadIdx.x; i < G::TILE; i += blockDim.x) mw[i] = V2{A(0), A(0)};
    const int any_low = __syncthreads_or(low);
    const bool inside = ti.h0 >= HALO && ti.h0 + G::TH + HALO <= H && ti.w0 >= HALO &&
                        ti.w0 + G::TW + HALO <= W;
    const bool full = ti.h0 + G::TH <= H && ti.w0 + G::TW <= W;
    const bool fast = __builtin_amdgcn_readfirstlane(static_cast<int>(
                          !any_low && eps >= TieScale<A>::kMinEps &&
                          (use_box ? inside : full))) != 0;

    A dq[VEC], xq[VEC], aq[VEC], bq[VEC], rq[VEC], gdq[VEC], gxq[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const V2 u = dxt[lc + k * TPR];
        const V2 v = abt[lc + k * TPR];
        dq[k] = u.x;
        xq[k] = u.y;
        aq[k] = v.x;
        bq[k] = v.y;
        if constexpr (G::kRhoLds)
            rq[k] = rht[lc + k * TPR];
        else
            rq[k] = m_rho(u.x, eps);
        gdq[k] = A(0);
        gxq[k] = A(0);
    }

    int last_dx = kClamp;
    // One near shift for the VEC pixels of the lane: all LDS reads first (the
    // neighbour arrays and the window cells, distinct for distinct k), then
    // the arithmetic, then the window writes.
    auto near = [&](const ShiftRec& rc, A (&wv)[VEC], auto fast_tag, auto inv_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        constexpr bool INV = decltype(inv_tag)::value;
        const bool rok = !use_box || in_range(h + rc.dx, H);
        const int op = lc + rc.dx * G::PITCH + rc.dy;
        V2 u[VEC], v[VEC], m[VEC];
        A rj[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            u[k] = dxt[op + k * TPR];
            v[k] = abt[op + k * TPR];
            if constexpr (G::kRhoLds) rj[k] = rht[op + k * TPR];
            m[k] = mw[op + k * TPR];
        }
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const A gsum = m_G<A>(aq[k], u[k].y, bq[k], v[k].x, xq[k], v[k].y, INV);
            A wk, mu;
            if constexpr (!G::kRhoLds) {
                // every staged degree of a FAST tile is >= eps: max(d, eps) = d
                rj[k] = FAST ? rcp_acc(u[k].x) : m_rho(u[k].x, eps);
            }
            if constexpr (FAST) {
                const A r = min_pos(rq[k], rj[k]);
                wk = wv[k] * r;
                mu = -(gsum * wk) * r;
            } else {
                const A r = fmin_acc(rq[k], rj[k]);
                const bool keep = px.act[k] && rok &&
                                  (!use_box || in_range(ti.w0 + tx + k * TPR + rc.dy, W));
                wk = keep ? wv[k] * r : A(0);
                mu = (keep && fmax_acc(dq[k], u[k].x) >= eps) ? -(gsum * wk) * r : A(0);
            }
            if constexpr (FAST) {
                A sq, sj;
                tie_shares<A>(dq[k], u[k].x, sq, sj);
                gdq[k] = fma_acc(mu, sq, gdq[k]);
                m[k].x = fma_acc(mu, sj, m[k].x);
            } else {
                const A muq = tie_part<A>(mu, dq[k], u[k].x);
                gdq[k] += muq;
                // every lane adds (0 for a dropped edge or an idle pixel)
                m[k].x += mu - muq;
            }
            if constexpr (INV) gxq[k] += wk * v[k].x;
            m[k].y += wk * aq[k];
        }
#pragma unroll
        for (int k = 0; k < VEC; ++k) mw[op + k * TPR] = m[k];
    };
    ShiftRec rn = read_shift(shl, 0);  // the next shift's record, read one shift ahead
    auto body = [&](int s, PixSlot<T, VEC>& slot, auto fast_tag) {
        const ShiftRec rc = rn;
        rn = read_shift(shl, min(s + 1, S - 1));
        A wv[VEC];
        slot_get_pixels<T, VEC>(slot, wv);
        slot_load_pixels<T, VEC, TPR, kMBwdEdgeNtLoads>(wr, px, slot);
        wr += s + D + 1 < S ? step : 0;
        if (shift_in_lds<HALO>(rc)) {
            if (rc.dx != last_dx) {
                lds_barrier();
                last_dx = rc.dx;
            }
            if (rc.inv)
                near(rc, wv, fast_tag, std::integral_constant<bool, true>{});
            else
                near(rc, wv, fast_tag, std::integral_constant<bool, false>{});
        }
    };
    auto ring = [&](auto fast_tag) {
        const int S_ring = S - S % D;
        for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
            for (int dd = 0; dd < D; ++dd) body(s0 + dd, wb[dd], fast_tag);
        }
#pragma unroll
        for (int dd = 0; dd < D; ++dd)
            if (S_ring + dd < S) body(S_ring + dd, wb[dd], fast_tag);
    };
    if (fast)
        ring(std::integral_constant<bool, true>{});
    else
        ring(std::integral_constant<bool, false>{});
    // Shifts beyond the halo: gather form.  A pixel p is the owner q of the
    // edge {p, p+s} and the far end j of the edge {p-s, p}.
    for (int s = 0; s < S && px.any; ++s) {
        const ShiftRec rc = read_shift(shl, s);
        if (shift_in_lds<HALO>(rc)) continue;
        const T* wp = wplane + static_cast<int64_t>(s) * step;
        int hp = h + rc.dxm;
        hp -= hp >= H ? H : 0;
        int hm = h - rc.dxm;
        hm += hm < 0 ? H : 0;
        const bool rok = !use_box || in_range(h + rc.dx, H);
        const bool mok = !use_box || in_range(h - rc.dx, H);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            if (!px.act[k]) continue;
            const int w = ti.w0 + tx + k * TPR;
            {  // owner
                int wj = w + rc.dym;
                wj -= wj >= W ? W : 0;
                const int64_t j = off + static_cast<uint32_t>(hp) * W + wj;
                const bool keep = rok && (!use_box || in_range(w + rc.dy, W));
                const A dj = deg[j], xj = to_acc(img[j]), aj = to_acc(gWx[j]);
                const A r = fmin_acc(rq[k], m_rho(dj, eps));
                const A wk = keep ? to_acc(*elem_ptr(wp, px.own[k])) * r : A(0);
                const A gsum = m_G<A>(aq[k], xj, bq[k], aj, xq[k], to_acc(gdh[j]) - aj * xj,
                                      rc.inv);
                const A mu = (keep && fmax_acc(dq[k], dj) >= eps) ? -(gsum * wk) * r : A(0);
                gdq[k] += tie_part<A>(mu, dq[k], dj);
                gxq[k] += rc.inv ? wk * aj : A(0);
            }
            {  // far end of the edge owned by q = p - s
                int wm = w - rc.dym;
                wm += wm < 0 ? W : 0;
                const uint32_t qi = static_cast<uint32_t>(hm) * W + wm;
                const int64_t q = off + qi;
                const bool keep = mok && (!use_box || in_range(w - rc.dy, W));
                const A dqo = deg[q], xo = to_acc(img[q]), ao = to_acc(gWx[q]);
                const A r = fmin_acc(m_rho(dqo, eps), rq[k]);
                const A wk = keep ? to_acc(wp[qi]) * r : A(0);
                const A gsum = m_G<A>(ao, xq[k], to_acc(gdh[q]) - ao * xo, aq[k], xo, bq[k],
                                      rc.inv);
                const A mu = (keep && fmax_acc(dqo, dq[k]) >= eps) ? -(gsum * wk) * r : A(0);
                gdq[k] += tie_part<A>(mu, dq[k], dqo);
                gxq[k] += wk * ao;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!px.act[k]) continue;
        const V2 m = mw[lc + k * TPR];
        const int64_t o = off + px.own[k];
        gd[o] = gdq[k] + m.x;
        gxp[o] = gxq[k] + m.y + aq[k] * (A(1) - to_acc(dhat[o]));
    }
    if (R == 0) return;
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    const int n = spill_count(th, tw, R);
    A* s0p = spill + t * G::SPILL;
    A* s1p = spill + (ntiles + t) * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        const V2 m = mw[(i + HALO) * G::PITCH + j + HALO];
        s0p[e] = m.x;
        s1p[e] = m.y;
    }
}

// gw is written once and not read again here: streaming stores (each
// half-wave writes a whole 128-byte row piece).
template <typename T>
__device__ __forceinline__ void gw_store(T* p, T v) {
    store_elem_nt<T>(p, v);
}
// The same into plane p at element offset i (a buffer store: uniform base).
template <typename T>
__device__ __forceinline__ void gw_store_at(T* p, uint32_t i, T v) {
    store_elem_at<T, true>(p, i * static_cast<uint32_t>(sizeof(T)), v);
}

// Pass 2: gw.  FAST tiles as in pass 1, without the degree condition (gw
// does not pass through the clamp gate).
template <typename T, int VEC, int TPR, int ROWS, bool BOX>
__global__ __launch_bounds__(TPR * ROWS, (kMBwdWaves<TPR * ROWS, 2>)) void
metropolis_bwd_weight_kernel(const T* __restrict__ img,
                             const acc_t<T>* __restrict__ deg, const T* __restrict__ gWx,
                             const T* __restrict__ gdh, const acc_t<T>* __restrict__ gd,
                             const acc_t<T>* __restrict__ gxp, const int64_t* __restrict__ shifts,
                             int S, int C, int H, int W, int ntw, int nth, acc_t<T> eps,
                             T* __restrict__ gw, T* __restrict__ gimg) {
    using A = acc_t<T>;
    using V2 = A __attribute__((ext_vector_type(2)));
    using G = SGeo<VEC, ROWS, TPR>;
    constexpr bool use_box = BOX;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    V2* rxt = reinterpret_cast<V2*>(smem + shift_lds_bytes(S));  // (rho, x)
    V2* abt = rxt + G::TILE;                                                         // (a, b)
    A* gdt = reinterpret_cast<A*>(abt + G::TILE);                                    // gd

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t off = ti.bc * HW;
    stage_shifts(shl, shifts, S, 3, H, W, false);
    {  // all loads of the thread first, then the LDS writes
        constexpr int NT = TPR * ROWS;
        constexpr int NCELL = G::LH * G::LW;
        constexpr int NST = (NCELL + NT - 1) / NT;
        const bool cheap = H >= G::LH && W >= G::LW;
        A sd[NST], sx[NST], sa[NST], sg[NST], sq[NST];
        int sl[NST];
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const int i = threadIdx.x + u * NT;
            sl[u] = 0;
            if ((u + 1) * NT <= NCELL || i < NCELL) {
                const int64_t g = off + halo_offset(i, G::LW, ti.h0, ti.w0, H, W, cheap);
                sd[u] = deg[g];
                sx[u] = to_acc(img[g]);
                sa[u] = to_acc(gWx[g]);
                sg[u] = to_acc(gdh[g]);
                sq[u] = gd[g];
                const int r = i / G::LW;
                sl[u] = r * G::PITCH + (i - r * G::LW);
            }
        }
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            if ((u + 1) * NT <= NCELL || threadIdx.x + u * NT < NCELL) {
                const int li = sl[u];
                rxt[li] = V2{m_rho(sd[u], eps), sx[u]};
                abt[li] = V2{sa[u], sg[u] - sa[u] * sx[u]};
                gdt[li] = sq[u];
            }
        }
    }
    __syncthreads();
    const bool inside = ti.h0 >= kRmax && ti.h0 + G::TH + kRmax <= H && ti.w0 >= kRmax &&
                        ti.w0 + G::TW + kRmax <= W;
    const bool full = ti.h0 + G::TH <= H && ti.w0 + G::TW <= W;
    const bool fast = eps > A(0) && (use_box ? inside : full);

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + kRmax) * G::PITCH + tx + kRmax;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    T* gplane = gw + (b * S * C + c) * HW;
    const int64_t step = static_cast<int64_t>(C) * HW;

    A rq[VEC], xq[VEC], aq[VEC], bq[VEC], gq[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const V2 u = rxt[lc + k * TPR];
        const V2 v = abt[lc + k * TPR];
        rq[k] = u.x;
        xq[k] = u.y;
        aq[k] = v.x;
        bq[k] = v.y;
        gq[k] = gdt[lc + k * TPR];
        if (px.act[k]) gimg[off + px.own[k]] = from_acc<T>(gxp[off + px.own[k]]);
    }

    // gw does not depend on w itself: this pass reads no weights, it streams
    // the S gradient planes out.
    auto run = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        // the shift's gradient plane advances one plane at a time; the next
        // shift's record is read one shift ahead
        T* gs = gplane;
        ShiftRec rn = read_shift(shl, 0);
        for (int s = 0; s < S; ++s, gs += step) {
            const ShiftRec rc = rn;
            rn = read_shift(shl, min(s + 1, S - 1));
            const bool rok = !use_box || in_range(h + rc.dx, H);
            if (shift_in_lds(rc)) {
                const int op = lc + rc.dx * G::PITCH + rc.dy;
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const int i = op + k * TPR;
                    const V2 u = rxt[i];
                    const V2 v = abt[i];
                    const A r = FAST ? min_pos(rq[k], u.x) : fmin_acc(rq[k], u.x);
                    const A gsum = m_G<A>(aq[k], u.y, bq[k], v.x, xq[k], v.y, rc.inv);
                    A g = fma_acc(gsum, r, gq[k]) + (rc.inv ? gdt[i] : A(0));
                    if constexpr (!FAST) {
                        const bool keep = px.act[k] && rok &&
                                          (!use_box || in_range(ti.w0 + tx + k * TPR + rc.dy, W));
                        g = keep ? g : A(0);
                    }
                    if (FAST || px.act[k]) gw_store_at<T>(gs, px.own[k], from_acc<T>(g));
                }
            } else if (px.any) {
                // beyond the halo: gather form
                int hp = h + rc.dxm;
                hp -= hp >= H ? H : 0;
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    if (!px.act[k]) continue;
                    const int w = ti.w0 + tx + k * TPR;
                    int wj = w + rc.dym;
                    wj -= wj >= W ? W : 0;
                    const int64_t j = off + static_cast<uint32_t>(hp) * W + wj;
                    const bool keep = rok && (!use_box || in_range(w + rc.dy, W));
                    const A xj = to_acc(img[j]), aj = to_acc(gWx[j]);
                    const A r = fmin_acc(rq[k], m_rho(deg[j], eps));
                    const A gsum = m_G<A>(aq[k], xj, bq[k], aj, xq[k], to_acc(gdh[j]) - aj * xj,
                                          rc.inv);
                    const A g = keep ? fma_acc(gsum, r, gq[k]) + (rc.inv ? gd[j] : A(0)) : A(0);
                    gw_store<T>(elem_ptr(gs, px.own[k]), from_acc<T>(g));
                }
            }
        }
    };
    if (fast)
        run(std::integral_constant<bool, true>{});
    else
        run(std::integral_constant<bool, false>{});
}

// ---------------------------------------------------------------------------
// Scatter path: geometry, workspace and launch
// ---------------------------------------------------------------------------
// Pass 1 and pass 2 tiles: TPR lanes x VEC pixels across, ROWS rows down.
// fp32-class types use 128 x 32 tiles of 1024 lanes in both passes (32 lanes
// x 4 pixels per row, so each weight plane is read in 512-byte row
// segments): 9.0 ms at 8192^2, S = 85, against 9.8 ms for the 64 x 64 / 64
// x 32 tiles of 16 lanes per row.  Pass 2 keeps four LDS arrays (image,
// degree and two windows: 110 KB, one workgroup per CU).  fp64 uses 32 x 32
// tiles.  Pass 2 measured at c4 (8192^2, S = 85) with other shapes: 128 x 16
// tiles (two workgroups per CU) 4.48 ms plus a 0.35 ms fix-up against 4.50
// plus 0.25 ms; 64 x 32 5.70 ms; 64 x 16 5.90 ms; 128 x 16 at prefetch depth
// 4 4.94 ms.  Depth 3 in pass 2: 8.44 ms for the forward against 8.48 at 2
// and 8.44 at 4.
template <typename T>
struct MScatterCfg {
    static constexpr int VEC = sizeof(T) == 8 ? 2 : 4;
    static constexpr int TPR1 = sizeof(T) == 8 ? kTPR : 32;
    static constexpr int ROWS1 = 32;
    static constexpr int D1 = sizeof(T) == 8 ? 2 : 3;
    static constexpr int TPR2 = sizeof(T) == 8 ? kTPR : 32;
    static constexpr int ROWS2 = 32;
    static constexpr int D2 = sizeof(T) == 8 ? 2 : 3;
    // Register budget of pass 2 (waves per SIMD): its four LDS arrays admit
    // one 1024-lane (fp32) or two 512-lane (fp64) workgroups per CU.
    static constexpr int WPE2 = 4;
};

constexpr size_t kMScatterLds = 160 * 1024 - 1024;
constexpr int64_t kMHeader = 256;

struct MPlan {
    bool ok = false;
    int ntw1 = 0, nth1 = 0, ntw2 = 0, nth2 = 0, spill1 = 0, spill2 = 0, ring = 0;
    int64_t tiles1 = 0, tiles2 = 0, spill_bytes = 0, part_bytes = 0, total = 0;
    size_t lds1 = 0, lds2 = 0;
};

static int64_t m_align256(int64_t b) { return (b + 255) / 256 * 256; }

template <typename T>
static MPlan m_plan(int B, int S, int C, int H, int W) {
    using Cfg = MScatterCfg<T>;
    using G1 = SGeo<Cfg::VEC, Cfg::ROWS1, Cfg::TPR1>;
    using G2 = SGeo<Cfg::VEC, Cfg::ROWS2, Cfg::TPR2>;
    const int64_t ab = sizeof(acc_t<T>);
    MPlan p;
    p.ntw1 = static_cast<int>(nsh_host::ceil_div(W, G1::TW));
    p.nth1 = static_cast<int>(nsh_host::ceil_div(H, G1::TH));
    p.ntw2 = static_cast<int>(nsh_host::ceil_div(W, G2::TW));
    p.nth2 = static_cast<int>(nsh_host::ceil_div(H, G2::TH));
    p.tiles1 = static_cast<int64_t>(B) * C * p.ntw1 * p.nth1;
    p.tiles2 = static_cast<int64_t>(B) * C * p.ntw2 * p.nth2;
    p.lds1 = shift_lds_bytes(S) + static_cast<size_t>(G1::TILE) * ab;
    p.lds2 = shift_lds_bytes(S) + 4 * static_cast<size_t>(G2::TILE) * ab;
    p.spill1 = G1::SPILL;
    p.spill2 = G2::SPILL;
    p.ring = G2::RING;
    auto fits = [&](int ntw, int nth, int TW, int TH) {
        return ntw >= 3 && nth >= 3 && W - (ntw - 1) * TW >= kRmax && H - (nth - 1) * TH >= kRmax;
    };
    p.ok = fits(p.ntw1, p.nth1, G1::TW, G1::TH) &&
           fits(p.ntw2, p.nth2, G2::TW, G2::TH) && p.lds1 <= kMScatterLds &&
           p.lds2 <= kMScatterLds;
    p.spill_bytes = m_align256(std::max(p.tiles1 * p.spill1, 2 * p.tiles2 * p.spill2) * ab);
    p.part_bytes = m_align256(2 * p.tiles2 * p.ring * ab);
    p.total = kMHeader + p.spill_bytes + p.part_bytes;
    return p;
}

template <typename T>
static int m_scatter(const void* wh, const void* img, const int64_t* sh, int B, int S, int C,
                     int H, int W, int use_box, double eps, void* Wx, void* dhat, void* deg,
                     const MPlan& p, void* ws, hipStream_t st) {
    using Cfg = MScatterCfg<T>;
    using A = acc_t<T>;
    char* base = static_cast<char*>(ws);
    int* hdr = reinterpret_cast<int*>(base);
    A* spill = reinterpret_cast<A*>(base + kMHeader);
    A* part = reinterpret_cast<A*>(base + kMHeader + p.spill_bytes);
    constexpr int V = Cfg::VEC, T1 = Cfg::TPR1, T2 = Cfg::TPR2, R1 = Cfg::ROWS1, R2 = Cfg::ROWS2;
    if (use_box)
        hipLaunchKernelGGL((metropolis_degree_scatter_kernel<T, V, T1, R1, Cfg::D1, true>),
                           dim3(static_cast<unsigned>(p.tiles1)), dim3(T1 * R1), p.lds1, st,
                           static_cast<const T*>(wh), sh, S, C, H, W, p.ntw1, p.nth1,
                           static_cast<A*>(deg), hdr, spill);
    else
        hipLaunchKernelGGL((metropolis_degree_scatter_kernel<T, V, T1, R1, Cfg::D1, false>),
                           dim3(static_cast<unsigned>(p.tiles1)), dim3(T1 * R1), p.lds1, st,
                           static_cast<const T*>(wh), sh, S, C, H, W, p.ntw1, p.nth1,
                           static_cast<A*>(deg), hdr, spill);
    if (int rc = nsh_host::check_launch("metropolis_aggregate (degree)")) return rc;
    hipLaunchKernelGGL((spill_fixup_kernel<A, A, 1, false>), dim3(static_cast<unsigned>(p.tiles1)),
                       dim3(256), 0, st, H, W, R1, T1 * V, p.ntw1, p.nth1, p.spill1,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill), p.tiles1,
                       static_cast<const A*>(nullptr), static_cast<A*>(deg),
                       static_cast<A*>(nullptr));
    if (int rc = nsh_host::check_launch("metropolis_aggregate (degree fix-up)")) return rc;
    if (use_box)
        hipLaunchKernelGGL((metropolis_aggregate_scatter_kernel<T, V, T2, R2, Cfg::D2, true, Cfg::WPE2>),
                           dim3(static_cast<unsigned>(p.tiles2)), dim3(T2 * R2), p.lds2, st,
                           static_cast<const T*>(wh), static_cast<const T*>(img),
                           static_cast<const A*>(deg), sh, S, C, H, W, p.ntw2, p.nth2,
                           static_cast<A>(eps), static_cast<T*>(Wx), static_cast<T*>(dhat),
                           spill, part, p.ring, p.tiles2);
    else
        hipLaunchKernelGGL((metropolis_aggregate_scatter_kernel<T, V, T2, R2, Cfg::D2, false, Cfg::WPE2>),
                           dim3(static_cast<unsigned>(p.tiles2)), dim3(T2 * R2), p.lds2, st,
                           static_cast<const T*>(wh), static_cast<const T*>(img),
                           static_cast<const A*>(deg), sh, S, C, H, W, p.ntw2, p.nth2,
                           static_cast<A>(eps), static_cast<T*>(Wx), static_cast<T*>(dhat),
                           spill, part, p.ring, p.tiles2);
    if (int rc = nsh_host::check_launch("metropolis_aggregate (aggregate)")) return rc;
    hipLaunchKernelGGL((metropolis_fixup_kernel<T>), dim3(static_cast<unsigned>(p.tiles2)),
                       dim3(256), 0, st, H, W, R2, T2 * V, p.ntw2, p.nth2, p.spill2, p.ring,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill),
                       static_cast<const A*>(part), p.tiles2, static_cast<const T*>(img),
                       static_cast<T*>(Wx), static_cast<T*>(dhat));
    return nsh_host::check_launch("metropolis_aggregate (fix-up)");
}

static bool m_scatter_disabled() {
    static const bool off = [] {
        const char* e = getenv("NSH_METRO_SCATTER");
        return e != nullptr && e[0] == '0';
    }();
    return off;
}

template <typename T>
static int m_run(const void* wh, const void* img, const int64_t* sh, int B, int S, int C, int H,
                 int W, int use_box, double eps, void* Wx, void* dhat, void* deg, void* ws,
                 int64_t ws_bytes, hipStream_t st) {
    if (ws != nullptr && !m_scatter_disabled()) {
        const MPlan p = m_plan<T>(B, S, C, H, W);
        if (p.ok && ws_bytes >= p.total && nsh_host::aligned(ws, 256))
            return m_scatter<T>(wh, img, sh, B, S, C, H, W, use_box, eps, Wx, dhat, deg, p, ws,
                                st);
    }
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

// ---- backward --------------------------------------------------------------
// Pass 1 keeps three pair arrays in LDS (degree/image, a/b, the gd/gx
// window) and rho, pass 2 two pairs (rho/image, a/b) and the gd tile.
// fp32-class tiles are 64 x 16 pixels with 32 lanes x 2 pixels per row
// (512 lanes; 72 KB and 51 KB of LDS, so two and three workgroups share a
// CU), fp64 tiles 32 x 32 with 16 lanes x 2 pixels.
template <typename T>
struct MBwdCfg {
    // pass 1 (edge): VEC pixels per lane, TPR lanes per row, ROWS1 rows
    static constexpr int VEC = 2;
    static constexpr int TPR = sizeof(T) == 8 ? kTPR : 32;
    static constexpr int ROWS1 = sizeof(T) == 8 ? 32 : 16;
    // four shifts in flight: c4 edge pass 6.81 -> 6.66 ms (backward 11.95 ->
    // 11.76 ms, mean of three runs); depth 2 7.04 ms
    static constexpr int D1 = 4;
    // pass 2 (weight gradients): its own tile shape (gather form, no spill)
    static constexpr int VEC2 = 2;
    static constexpr int TPR2 = sizeof(T) == 8 ? kTPR : 32;
    static constexpr int ROWS2 = sizeof(T) == 8 ? 32 : 16;
};

constexpr size_t kMBwdLds = 160 * 1024 - 1024;

struct MBPlan {
    bool ok = false;
    bool narrow = false;  // pass 1 on the 6-pixel border (MEdgeGeo)
    int ntw1 = 0, nth1 = 0, ntw2 = 0, nth2 = 0, spill = 0;
    int64_t tiles1 = 0, tiles2 = 0, spill_bytes = 0, plane_bytes = 0, total = 0;
    size_t lds1 = 0, lds2 = 0;
};

template <typename T>
static MBPlan mb_plan(int B, int S, int C, int H, int W, bool narrow = false) {
    using Cfg = MBwdCfg<T>;
    using G1 = SGeo<Cfg::VEC, Cfg::ROWS1, Cfg::TPR>;
    using E1 = MEdgeGeo<Cfg::VEC, Cfg::ROWS1, Cfg::TPR, kRmax>;
    using E1n = MEdgeGeo<Cfg::VEC, Cfg::ROWS1, Cfg::TPR, kMNarrowHalo>;
    using G2 = SGeo<Cfg::VEC2, Cfg::ROWS2, Cfg::TPR2>;
    const int64_t ab = sizeof(acc_t<T>);
    MBPlan p;
    p.ntw1 = static_cast<int>(nsh_host::ceil_div(W, G1::TW));
    p.nth1 = static_cast<int>(nsh_host::ceil_div(H, G1::TH));
    p.ntw2 = static_cast<int>(nsh_host::ceil_div(W, G2::TW));
    p.nth2 = static_cast<int>(nsh_host::ceil_div(H, G2::TH));
    p.tiles1 = static_cast<int64_t>(B) * C * p.ntw1 * p.nth1;
    p.tiles2 = static_cast<int64_t>(B) * C * p.ntw2 * p.nth2;
    p.narrow = narrow && sizeof(acc_t<T>) == 4;
    p.lds1 = shift_lds_bytes(S) +
             (p.narrow ? static_cast<size_t>(E1n::WORDS) * E1n::TILE
                       : static_cast<size_t>(E1::WORDS) * E1::TILE) * ab;
    p.lds2 = shift_lds_bytes(S) + 5 * static_cast<size_t>(G2::TILE) * ab;
    p.spill = G1::SPILL;
    // the edge pass scatters across tile borders: at least 3 tiles per
    // direction, edge tiles at least kRmax (the weight pass only gathers)
    p.ok = p.ntw1 >= 3 && p.nth1 >= 3 && W - (p.ntw1 - 1) * G1::TW >= kRmax &&
           H - (p.nth1 - 1) * G1::TH >= kRmax && p.lds1 <= kMBwdLds && p.lds2 <= kMBwdLds;
    p.spill_bytes = m_align256(2 * p.tiles1 * p.spill * ab);
    p.plane_bytes = m_align256(static_cast<int64_t>(B) * C * H * W * ab);
    p.total = kMHeader + p.spill_bytes + 2 * p.plane_bytes;  // + gd and gx partials
    return p;
}

template <typename T, bool BOX>
static int mb_launch(const void* wh, const void* img, const int64_t* sh, int B, int S, int C,
                     int H, int W, double eps, const void* deg, const void* dhat, const void* gWx,
                     const void* gdh, void* gw, void* gimg, const MBPlan& p, void* ws,
                     hipStream_t st) {
    using Cfg = MBwdCfg<T>;
    using A = acc_t<T>;
    constexpr int V = Cfg::VEC, TPR = Cfg::TPR, R1 = Cfg::ROWS1, R2 = Cfg::ROWS2;
    char* base = static_cast<char*>(ws);
    int* hdr = reinterpret_cast<int*>(base);
    A* spill = reinterpret_cast<A*>(base + kMHeader);
    A* gd = reinterpret_cast<A*>(base + kMHeader + p.spill_bytes);
    A* gxp = reinterpret_cast<A*>(base + kMHeader + p.spill_bytes + p.plane_bytes);
    auto edge = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(p.tiles1)), dim3(TPR * R1), p.lds1,
                           st, static_cast<const T*>(wh), static_cast<const T*>(img),
                           static_cast<const A*>(deg), static_cast<const T*>(dhat),
                           static_cast<const T*>(gWx), static_cast<const T*>(gdh), sh, S, C, H, W,
                           p.ntw1, p.nth1, static_cast<A>(eps), gd, gxp, hdr, spill, p.tiles1);
    };
    if constexpr (sizeof(A) == 4) {
        if (p.narrow)
            edge(metropolis_bwd_edge_kernel<T, V, TPR, R1, Cfg::D1, BOX, kMNarrowHalo>);
        else
            edge(metropolis_bwd_edge_kernel<T, V, TPR, R1, Cfg::D1, BOX, kRmax>);
    } else {
        edge(metropolis_bwd_edge_kernel<T, V, TPR, R1, Cfg::D1, BOX, kRmax>);
    }
    if (int rc = nsh_host::check_launch("metropolis_aggregate_backward (edges)")) return rc;
    hipLaunchKernelGGL((spill_fixup_kernel<A, A, 2, false>), dim3(static_cast<unsigned>(p.tiles1)),
                       dim3(256), 0, st, H, W, R1, TPR * V, p.ntw1, p.nth1, p.spill,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill), p.tiles1,
                       static_cast<const A*>(nullptr), gd, gxp);
    if (int rc = nsh_host::check_launch("metropolis_aggregate_backward (fix-up)")) return rc;
    hipLaunchKernelGGL((metropolis_bwd_weight_kernel<T, Cfg::VEC2, Cfg::TPR2, R2, BOX>),
                       dim3(static_cast<unsigned>(p.tiles2)), dim3(Cfg::TPR2 * R2), p.lds2, st,
                       static_cast<const T*>(img),
                       static_cast<const A*>(deg), static_cast<const T*>(gWx),
                       static_cast<const T*>(gdh), static_cast<const A*>(gd),
                       static_cast<const A*>(gxp), sh, S, C, H, W, p.ntw2, p.nth2,
                       static_cast<A>(eps), static_cast<T*>(gw), static_cast<T*>(gimg));
    return nsh_host::check_launch("metropolis_aggregate_backward (weights)");
}

template <typename T>
static int mb_run(const void* wh, const void* img, const int64_t* sh, int B, int S, int C, int H,
                  int W, int use_box, double eps, const void* deg, const void* dhat,
                  const void* gWx, const void* gdh, void* gw, void* gimg, void* ws,
                  int64_t ws_bytes, bool narrow, hipStream_t st) {
    const MBPlan p = mb_plan<T>(B, S, C, H, W, narrow);
    if (!p.ok)
        return nsh_host::fail(NSH_ERR_INVALID,
                              "metropolis_aggregate_backward: needs at least 3 tiles of %dx%d "
                              "pixels per direction (edge tiles >= %d)",
                              SGeo<MBwdCfg<T>::VEC, MBwdCfg<T>::ROWS1, MBwdCfg<T>::TPR>::TH,
                              SGeo<MBwdCfg<T>::VEC, MBwdCfg<T>::ROWS1, MBwdCfg<T>::TPR>::TW, kRmax);
    if (ws == nullptr || ws_bytes < p.total || !nsh_host::aligned(ws, 256))
        return nsh_host::fail(NSH_ERR_INVALID,
                              "metropolis_aggregate_backward: workspace of %lld bytes required",
                              static_cast<long long>(p.total));
    return use_box ? mb_launch<T, true>(wh, img, sh, B, S, C, H, W, eps, deg, dhat, gWx, gdh, gw,
                                        gimg, p, ws, st)
                   : mb_launch<T, false>(wh, img, sh, B, S, C, H, W, eps, deg, dhat, gWx, gdh,
                                         gw, gimg, p, ws, st);
}

template <typename T>
static int64_t mb_workspace(int B, int S, int C, int H, int W) {
    const MBPlan p = mb_plan<T>(B, S, C, H, W);
    return p.ok ? p.total : 0;
}

template <typename T>
static int64_t m_workspace(int B, int S, int C, int H, int W) {
    const MPlan p = m_plan<T>(B, S, C, H, W);
    return p.ok ? p.total : 0;
}

}  // namespace nsh

using nsh_host::fail;

static int m_check(const char* op, int64_t B, int64_t S, int64_t C, int64_t H, int64_t W,
                   int dtype) {
    if (S < 1 || S > 1024) return fail(NSH_ERR_INVALID, "%s: requires 1 <= S <= 1024", op);
    if (B < 1 || C < 1 || H < 1 || W < 1) return fail(NSH_ERR_INVALID, "%s: empty tensor", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (B * C > (int64_t(1) << 24) || B * S * C > (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: B*S*C too large", op);
    return NSH_OK;
}

extern "C" int64_t nsh_metropolis_workspace_bytes(int64_t B, int64_t S, int64_t C, int64_t H,
                                                  int64_t W, int dtype) {
    if (m_check("metropolis_aggregate", B, S, C, H, W, dtype) != NSH_OK) return -1;
    const int b = static_cast<int>(B), s = static_cast<int>(S), c = static_cast<int>(C);
    const int h = static_cast<int>(H), w = static_cast<int>(W);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::m_workspace<nsh::f16>(b, s, c, h, w);
        case NSH_DTYPE_BFLOAT16: return nsh::m_workspace<nsh::bf16>(b, s, c, h, w);
        case NSH_DTYPE_FLOAT32: return nsh::m_workspace<float>(b, s, c, h, w);
        default: return nsh::m_workspace<double>(b, s, c, h, w);
    }
}

extern "C" int nsh_metropolis_aggregate(const void* w_half, const void* img, const int64_t* shifts,
                                        int64_t B, int64_t S, int64_t C, int64_t H, int64_t W,
                                        int dtype, int use_box, double eps, void* Wx, void* d_hat,
                                        void* degree, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
    const char* op = "metropolis_aggregate";
    if (int rc = m_check(op, B, S, C, H, W, dtype)) return rc;
    if (!w_half || !img || !shifts || !Wx || !d_hat || !degree)
        return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int b = static_cast<int>(B), s = static_cast<int>(S), c = static_cast<int>(C);
    const int h = static_cast<int>(H), w = static_cast<int>(W);
    const int ub = use_box ? 1 : 0;
    void* ws = workspace;
    const int64_t nws = workspace ? workspace_bytes : 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::m_run<nsh::f16>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, ws, nws, st);
        case NSH_DTYPE_BFLOAT16: return nsh::m_run<nsh::bf16>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, ws, nws, st);
        case NSH_DTYPE_FLOAT32: return nsh::m_run<float>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, ws, nws, st);
        default: return nsh::m_run<double>(w_half, img, shifts, b, s, c, h, w, ub, eps, Wx, d_hat, degree, ws, nws, st);
    }
}

extern "C" int64_t nsh_metropolis_backward_workspace_bytes(int64_t B, int64_t S, int64_t C,
                                                           int64_t H, int64_t W, int dtype) {
    dtype &= ~NSH_NARROW_HALO;  // the workspace does not depend on the border
    if (m_check("metropolis_aggregate_backward", B, S, C, H, W, dtype) != NSH_OK) return -1;
    const int b = static_cast<int>(B), s = static_cast<int>(S), c = static_cast<int>(C);
    const int h = static_cast<int>(H), w = static_cast<int>(W);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::mb_workspace<nsh::f16>(b, s, c, h, w);
        case NSH_DTYPE_BFLOAT16: return nsh::mb_workspace<nsh::bf16>(b, s, c, h, w);
        case NSH_DTYPE_FLOAT32: return nsh::mb_workspace<float>(b, s, c, h, w);
        default: return nsh::mb_workspace<double>(b, s, c, h, w);
    }
}

extern "C" int nsh_metropolis_aggregate_backward(
    const void* w_half, const void* img, const int64_t* shifts, int64_t B, int64_t S, int64_t C,
    int64_t H, int64_t W, int dtype, int use_box, double eps, const void* degree,
    const void* d_hat, const void* grad_Wx, const void* grad_d_hat, void* grad_w_half,
    void* grad_img, void* workspace, int64_t workspace_bytes, void* stream) {
    const char* op = "metropolis_aggregate_backward";
    const bool narrow = (dtype & NSH_NARROW_HALO) != 0;
    dtype &= ~NSH_NARROW_HALO;
    if (int rc = m_check(op, B, S, C, H, W, dtype)) return rc;
    if (!w_half || !img || !shifts || !degree || !d_hat || !grad_Wx || !grad_d_hat ||
        !grad_w_half || !grad_img)
        return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int b = static_cast<int>(B), s = static_cast<int>(S), c = static_cast<int>(C);
    const int h = static_cast<int>(H), w = static_cast<int>(W);
    const int ub = use_box ? 1 : 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            return nsh::mb_run<nsh::f16>(w_half, img, shifts, b, s, c, h, w, ub, eps, degree, d_hat, grad_Wx, grad_d_hat, grad_w_half, grad_img, workspace, workspace_bytes, narrow, st);
        case NSH_DTYPE_BFLOAT16:
            return nsh::mb_run<nsh::bf16>(w_half, img, shifts, b, s, c, h, w, ub, eps, degree, d_hat, grad_Wx, grad_d_hat, grad_w_half, grad_img, workspace, workspace_bytes, narrow, st);
        case NSH_DTYPE_FLOAT32:
            return nsh::mb_run<float>(w_half, img, shifts, b, s, c, h, w, ub, eps, degree, d_hat, grad_Wx, grad_d_hat, grad_w_half, grad_img, workspace, workspace_bytes, narrow, st);
        default:
            return nsh::mb_run<double>(w_half, img, shifts, b, s, c, h, w, ub, eps, degree, d_hat, grad_Wx, grad_d_hat, grad_w_half, grad_img, workspace, workspace_bytes, narrow, st);
    }
}
