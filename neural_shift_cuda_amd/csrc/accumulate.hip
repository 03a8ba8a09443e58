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
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include <type_traits>
#include "nsh_common.hpp"
#include "scatter.hpp"

namespace nsh {

// Tile geometry: kTPR lanes x VEC pixels across, ROWS lanes x RPT rows down
// (a lane owns rows ty, ty + ROWS, ... so each ROWS-row pass of the
// workgroup is contiguous); the workgroup has kTPR * ROWS lanes.  LDS tiles
// carry a kRmax halo and an odd row pitch.
template <int VEC, int RPT, int ROWS, int TPR = kTPR, int LP = 0>
struct Geo {
    static constexpr int THREADS = TPR * ROWS;
    static constexpr int TW = TPR * VEC;
    static constexpr int TH = ROWS * RPT;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
    static constexpr int PITCH = LP ? LP : LW + 1;  // LP: the pitch of a caller's tiles
    static constexpr int TILE = LH * PITCH;
};

// Whole-tile range test for a shift: do all of the tile's pixels p keep
// p + (dx, dy) inside the image (no wrap, box true)?
__device__ __forceinline__ bool tile_inside(int h0, int w0, int TH, int TW, int H, int W,
                                            int dx, int dy) {
    const int h1 = (h0 + TH < H ? h0 + TH : H) - 1;
    const int w1 = (w0 + TW < W ? w0 + TW : W) - 1;
    return h0 + dx >= 0 && h1 + dx < H && w0 + dy >= 0 && w1 + dy < W;
}

// The same test on a band (see Band): the tile's rows are image rows
// without wrapping and stay inside the image when displaced by dx.
__device__ __forceinline__ bool tile_inside_band(const Band& bd, int h0, int w0, int TH, int TW,
                                                 int H, int W, int dx, int dy) {
    const int h1 = (h0 + TH < H ? h0 + TH : H) - 1;
    const int w1 = (w0 + TW < W ? w0 + TW : W) - 1;
    return band_rows_inside(bd, h0, h1, dx) && w0 + dy >= 0 && w1 + dy < W;
}

// Per-lane pixel block: RPT rows x VEC columns.
template <int VEC, int RPT>
struct Lane {
    int w0;
    int h[RPT];
    bool row_ok[RPT];
    uint32_t own[RPT];  // h*W + w0
    int lc[RPT];        // LDS index of (h, w0)
};

template <int VEC, int RPT, int ROWS, int TPR = kTPR, int LP = 0>
__device__ __forceinline__ Lane<VEC, RPT> lane_of(const TileIdx& ti, int W, int H) {
    using G = Geo<VEC, RPT, ROWS, TPR, LP>;
    Lane<VEC, RPT> L;
    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    L.w0 = ti.w0 + tx * VEC;
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        L.h[r] = ti.h0 + ty + ROWS * r;
        L.row_ok[r] = L.h[r] < H;
        L.own[r] = static_cast<uint32_t>(L.row_ok[r] ? L.h[r] : ti.h0) * static_cast<uint32_t>(W) + L.w0;
        L.lc[r] = (ty + ROWS * r + kRmax) * G::PITCH + tx * VEC + kRmax;
    }
    return L;
}

// ---------------------------------------------------------------------------
// Forward.  Per chunk of P shifts every lane first issues all of the chunk's
// weight loads (P x RPT aligned vectors plus the mirror elements), then
// consumes them, so each wave keeps several KB of HBM reads in flight.
// ---------------------------------------------------------------------------
template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL, int TPR = kTPR, int LP = 0>
__device__ __forceinline__ void fwd_gather_tile(const T* __restrict__ x, const T* __restrict__ w,
                                                int S, int C, int H, int W, const TileIdx& ti,
                                                int64_t plane_step, bool wsh, acc_t<T>* __restrict__ U,
                                                acc_t<T>* __restrict__ Z, const int4* shl,
                                                const acc_t<T>* xt, const Band bd) {
    using A = acc_t<T>;
    using G = Geo<VEC, RPT, ROWS, TPR, LP>;
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;
    const Lane<VEC, RPT> L = lane_of<VEC, RPT, ROWS, TPR, LP>(ti, W, H);
    if (L.w0 >= W) return;
    int hr[RPT];  // image rows of the lane's rows (box tests)
#pragma unroll
    for (int r = 0; r < RPT; ++r) hr[r] = band_row(bd, L.row_ok[r] ? L.h[r] : ti.h0);
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* w_bc = w + weight_plane(b, c, C, wsh) * HW;  // shift s adds s * wstep
    const int64_t wstep = weight_step(plane_step, C, wsh);
    const bool full_rows = ti.h0 + G::TH <= H;  // every lane row inside the image

    A u[RPT][VEC], z[RPT][VEC];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
#pragma unroll
        for (int k = 0; k < VEC; ++k) u[r][k] = z[r][k] = A(0);

    for (int s0 = 0; s0 < S; s0 += P) {
        ShiftRec rc[P];
        bool act[P], inside[P], inside_g[P];
        const T* wp[P];
        A wv[P][RPT][VEC], wm[P][RPT][VEC];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            act[p] = s0 + p < S;
            rc[p] = read_shift(shl, act[p] ? s0 + p : s0);
            wp[p] = w_bc + static_cast<int64_t>(s0 + p) * wstep;
            // inside: the unwrapped mirror loads stay in the plane; inside_g:
            // no mirror source of the tile wraps the image (no mask needed)
            inside[p] = tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, -rc[p].dx, -rc[p].dy);
            inside_g[p] = tile_inside_band(bd, ti.h0, ti.w0, G::TH, G::TW, H, W, -rc[p].dx,
                                           -rc[p].dy);
        }
        // 1) weights at p
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (!act[p]) continue;
#pragma unroll
            for (int r = 0; r < RPT; ++r) load_acc<T, VEC, NTL>(wp[p] + L.own[r], wv[p][r]);
        }
        // 2) mirror weights at p - s (inside the image only).  A shift whose
        //    mirror source stays inside the image for the whole tile (the
        //    common case) loads unconditionally.
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (!act[p] || !rc[p].inv) continue;
            const int off = -(rc[p].dx * W + rc[p].dy);
            if (inside[p] && full_rows) {
#pragma unroll
                for (int r = 0; r < RPT; ++r)
#pragma unroll
                    for (int k = 0; k < VEC; ++k)
                        wm[p][r][k] = to_acc(wp[p][static_cast<int64_t>(L.own[r]) + off + k]);
            } else {
                // source (h - dx, w - dy), wrapped for a circular mirror
#pragma unroll
                for (int r = 0; r < RPT; ++r) {
                    const bool rok =
                        L.row_ok[r] && (rc[p].per || in_range(hr[r] - rc[p].dx, bd.Hg));
                    int hm = (L.row_ok[r] ? L.h[r] : ti.h0) - rc[p].dxm;
                    hm += hm < 0 ? H : 0;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        const bool ok = rok && (rc[p].per || in_range(L.w0 + k - rc[p].dy, W));
                        int wm_ = L.w0 + k - rc[p].dym;
                        wm_ += wm_ < 0 ? W : 0;
                        wm[p][r][k] = ok ? to_acc(wp[p][static_cast<uint32_t>(hm) * W + wm_]) : A(0);
                    }
                }
            }
        }
        // 3) accumulate
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (!act[p]) continue;
            const ShiftRec& sr = rc[p];
            const bool lds = shift_in_lds(sr);
            const bool fast = lds && inside[p] && inside_g[p] && full_rows;
#pragma unroll
            for (int r = 0; r < RPT; ++r) {
                A xv[VEC];
                if (lds) {
                    const A* xr = xt + L.lc[r] + sr.dx * G::PITCH + sr.dy;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) xv[k] = xr[k];
                } else {
                    int hh = (L.row_ok[r] ? L.h[r] : ti.h0) + sr.dxm;
                    hh -= hh >= H ? H : 0;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        int ww = L.w0 + k + sr.dym;
                        ww -= ww >= W ? W : 0;
                        xv[k] = to_acc(xp[static_cast<uint32_t>(hh) * W + ww]);
                    }
                }
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const A wf = fwd_kept(sr, hr[r], L.w0 + k, bd.Hg, W) ? wv[p][r][k] : A(0);
                    u[r][k] = fma_acc(wf, xv[k], u[r][k]);
                    z[r][k] += wf;
                }
                if (!sr.inv) continue;
                if (fast) {
                    const A* xr = xt + L.lc[r] - sr.dx * G::PITCH - sr.dy;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        u[r][k] = fma_acc(wm[p][r][k], xr[k], u[r][k]);
                        z[r][k] += wm[p][r][k];
                    }
                } else {
                    const bool rok = L.row_ok[r] && (sr.per || in_range(hr[r] - sr.dx, bd.Hg));
                    int hm = (L.row_ok[r] ? L.h[r] : ti.h0) - sr.dxm;
                    hm += hm < 0 ? H : 0;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        if (!(rok && (sr.per || in_range(L.w0 + k - sr.dy, W)))) continue;
                        int wm_ = L.w0 + k - sr.dym;
                        wm_ += wm_ < 0 ? W : 0;
                        const A xi = lds ? xt[L.lc[r] - sr.dx * G::PITCH - sr.dy + k]
                                         : to_acc(xp[static_cast<uint32_t>(hm) * W + wm_]);
                        u[r][k] = fma_acc(wm[p][r][k], xi, u[r][k]);
                        z[r][k] += wm[p][r][k];
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        if (!L.row_ok[r]) continue;
        store_out<A, VEC>(U + ti.bc * HW + L.own[r], u[r]);
        store_out<A, VEC>(Z + ti.bc * HW + L.own[r], z[r]);
    }
}

template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL>
__global__ __launch_bounds__(kTPR * ROWS) void accumulate_uz_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const int64_t* __restrict__ shifts,
    int S, int codes, int C, int H, int W, int ntw, int nth, int order, int band,
    int64_t plane_step, acc_t<T>* __restrict__ U, acc_t<T>* __restrict__ Z, Band bd) {
    using A = acc_t<T>;
    using G = Geo<VEC, RPT, ROWS>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW, order, band);
    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
    stage_tile<T, A>(xt, x + ti.bc * (static_cast<int64_t>(H) * W), H, W, ti.h0, ti.w0, G::LH,
                     G::LW, G::PITCH);
    __syncthreads();
    fwd_gather_tile<T, VEC, RPT, ROWS, P, NTL>(x, w, S, C, H, W, ti, plane_step,
                                               (codes & kCodesSharedW) != 0, U, Z, shl, xt, bd);
}

// ---------------------------------------------------------------------------
// Fused backward: one pass over the weight planes produces gw (written once,
// streaming) and gx (register sums).  x, gU and gZ tiles with halo live in
// LDS; weight loads of a chunk of P shifts are issued before any use.
// ---------------------------------------------------------------------------
template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL, int TPR = kTPR, int LP = 0>
__device__ __forceinline__ void bwd_gather_tile(
    const T* __restrict__ x, const T* __restrict__ w, const acc_t<T>* __restrict__ gU,
    const acc_t<T>* __restrict__ gZ, int S, int C, int H, int W, const TileIdx& ti,
    int64_t plane_step, bool wsh, T* __restrict__ gx, T* __restrict__ gw, const int4* shl,
    const acc_t<T>* xt, const acc_t<T>* ut, const acc_t<T>* zt, const Band bd) {
    using A = acc_t<T>;
    using G = Geo<VEC, RPT, ROWS, TPR, LP>;
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;
    const A* up = gU + ti.bc * HW;
    const A* zp = gZ + ti.bc * HW;
    const Lane<VEC, RPT> L = lane_of<VEC, RPT, ROWS, TPR, LP>(ti, W, H);
    if (L.w0 >= W) return;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* w_bc = w + weight_plane(b, c, C, wsh) * HW;
    const int64_t wstep = weight_step(plane_step, C, wsh);
    T* g_bc = gw + (b * C + c) * HW;  // the gradient has every channel
    int hr[RPT];  // image rows of the lane's rows (box tests)
#pragma unroll
    for (int r = 0; r < RPT; ++r) hr[r] = band_row(bd, L.row_ok[r] ? L.h[r] : ti.h0);

    A xo[RPT][VEC], uo[RPT][VEC], zo[RPT][VEC], gxa[RPT][VEC];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            xo[r][k] = xt[L.lc[r] + k];
            uo[r][k] = ut[L.lc[r] + k];
            zo[r][k] = zt[L.lc[r] + k];
            gxa[r][k] = A(0);
        }

    for (int s0 = 0; s0 < S; s0 += P) {
        ShiftRec rc[P];
        bool act[P], minus_in[P], plus_in[P];
        const T* wp[P];
        A ws[P][RPT][VEC], wv[P][RPT][VEC];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            act[p] = s0 + p < S;
            rc[p] = read_shift(shl, act[p] ? s0 + p : s0);
            wp[p] = w_bc + static_cast<int64_t>(s0 + p) * wstep;
            // minus_in: the unwrapped loads at q - s stay in the plane;
            // plus_in: no q + s of the tile wraps the image (no mask needed)
            minus_in[p] = tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, -rc[p].dx, -rc[p].dy);
            plus_in[p] = tile_inside_band(bd, ti.h0, ti.w0, G::TH, G::TW, H, W, rc[p].dx,
                                          rc[p].dy);
        }
        // 1) w_s[(q-s) mod] for the gx forward term
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (!act[p]) continue;
            const ShiftRec& sr = rc[p];
            if (minus_in[p]) {
                const int off = -(sr.dx * W + sr.dy);
#pragma unroll
                for (int r = 0; r < RPT; ++r)
#pragma unroll
                    for (int k = 0; k < VEC; ++k)
                        ws[p][r][k] = to_acc(wp[p][static_cast<int64_t>(L.own[r]) + off + k]);
            } else {
#pragma unroll
                for (int r = 0; r < RPT; ++r) {
                    int hm = (L.row_ok[r] ? L.h[r] : ti.h0) - sr.dxm;
                    hm += hm < 0 ? H : 0;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        int wm_ = L.w0 + k - sr.dym;
                        wm_ += wm_ < 0 ? W : 0;
                        ws[p][r][k] = to_acc(wp[p][static_cast<uint32_t>(hm) * W + wm_]);
                    }
                }
            }
        }
        // 2) w_s[q] for the gx mirror term
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (!act[p] || !rc[p].inv) continue;
#pragma unroll
            for (int r = 0; r < RPT; ++r) load_acc<T, VEC, NTL>(wp[p] + L.own[r], wv[p][r]);
        }
        // 3) gw_s[q] and gx[q]
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (!act[p]) continue;
            const ShiftRec& sr = rc[p];
            const bool lds = shift_in_lds(sr);
            T* gp = g_bc + static_cast<int64_t>(s0 + p) * plane_step;
#pragma unroll
            for (int r = 0; r < RPT; ++r) {
                A xf[VEC], up_[VEC], zp_[VEC], um[VEC];
                if (lds) {
                    const int op = L.lc[r] + sr.dx * G::PITCH + sr.dy;
                    const int om = L.lc[r] - sr.dx * G::PITCH - sr.dy;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        xf[k] = xt[op + k];
                        up_[k] = ut[op + k];
                        zp_[k] = zt[op + k];
                        um[k] = ut[om + k];
                    }
                } else {
                    const int hr = L.row_ok[r] ? L.h[r] : ti.h0;
                    int hp = hr + sr.dxm;
                    hp -= hp >= H ? H : 0;
                    int hm = hr - sr.dxm;
                    hm += hm < 0 ? H : 0;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        int wq = L.w0 + k + sr.dym;
                        wq -= wq >= W ? W : 0;
                        int wm_ = L.w0 + k - sr.dym;
                        wm_ += wm_ < 0 ? W : 0;
                        const uint32_t ip = static_cast<uint32_t>(hp) * W + wq;
                        const uint32_t im = static_cast<uint32_t>(hm) * W + wm_;
                        xf[k] = to_acc(xp[ip]);
                        up_[k] = up[ip];
                        zp_[k] = zp[ip];
                        um[k] = up[im];
                    }
                }
                bool okp[VEC];
                {
                    const bool rok = plus_in[p] || sr.per || in_range(hr[r] + sr.dx, bd.Hg);
#pragma unroll
                    for (int k = 0; k < VEC; ++k)
                        okp[k] = sr.inv && (plus_in[p] || sr.per ||
                                            (rok && in_range(L.w0 + k + sr.dy, W)));
                }
                A g[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    // forward box: a dropped forward term has no gradient
                    // (its mirror is dropped too: okp is false there)
                    g[k] = fwd_kept(sr, hr[r], L.w0 + k, bd.Hg, W)
                               ? fma_acc(xf[k], uo[r][k], zo[r][k]) : A(0);
                    if (okp[k]) g[k] += fma_acc(xo[r][k], up_[k], zp_[k]);
                    if (fwd_kept_src(sr, hr[r], L.w0 + k, bd.Hg, W))
                        gxa[r][k] = fma_acc(ws[p][r][k], um[k], gxa[r][k]);
                    if (okp[k]) gxa[r][k] = fma_acc(wv[p][r][k], up_[k], gxa[r][k]);
                }
                if (L.row_ok[r]) store_acc<T, VEC>(gp + L.own[r], g, true);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPT; ++r)
        if (L.row_ok[r]) store_acc<T, VEC>(gx + ti.bc * HW + L.own[r], gxa[r], false);
}

template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL>
__global__ __launch_bounds__(kTPR * ROWS) void accumulate_uz_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const acc_t<T>* __restrict__ gU,
    const acc_t<T>* __restrict__ gZ, const int64_t* __restrict__ shifts, int S, int codes, int C,
    int H, int W, int ntw, int nth, int order, int band, int64_t plane_step, T* __restrict__ gx,
    T* __restrict__ gw, Band bd) {
    using A = acc_t<T>;
    using G = Geo<VEC, RPT, ROWS>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* ut = xt + G::TILE;
    A* zt = ut + G::TILE;
    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW, order, band);
    const int64_t off = ti.bc * (static_cast<int64_t>(H) * W);
    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
    stage_tile<T, A>(xt, x + off, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    stage_tile<A, A>(ut, gU + off, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    stage_tile<A, A>(zt, gZ + off, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    __syncthreads();
    bwd_gather_tile<T, VEC, RPT, ROWS, P, NTL>(x, w, gU, gZ, S, C, H, W, ti, plane_step,
                                               (codes & kCodesSharedW) != 0, gx, gw, shl, xt, ut,
                                               zt, bd);
}

// ---------------------------------------------------------------------------
// Scatter kernels: every weight element is read once, aligned.
//
// The gather kernels above read w_s at shifted pixels (the forward mirror
// term w_s[p-s], the backward x term w_s[(q-s) mod]).  Those reads reach R
// rows/columns into the neighbouring tiles, whose lines have usually left L2
// by then (neighbouring tiles drift apart by several shift planes), so they
// come from HBM a second time: ~25-40% extra reads at 8192^2.  The scatter
// kernels use the adjoint form of the same terms instead: the lane that owns
// pixel q loads w_s[q] (aligned, once) and adds w_s[q] x[q] (forward) or
// w_s[q] gU[q] (backward) into an LDS accumulator window at q + s.  The window
// covers the tile plus an R-pixel border.
//
// Determinism: within one shift the map q -> q + s is injective, so the lanes
// of a workgroup update distinct LDS words; a workgroup barrier (LDS traffic
// only; the weight prefetches stay in flight) separates consecutive shifts.
// Every window word thus receives its terms in shift order, in every run.
//
// The window border (targets outside the tile) is spilled to a workspace
// block per tile; spill_fixup_kernel then adds, for every pixel
// within R of a tile edge, the spills of the (up to 8) neighbouring tiles in
// a fixed order.  Eligibility (host-checked): at least 2 tiles in each
// direction and edge tiles at least kRmax wide, so each window reaches only
// adjacent tiles and never its own tile.  With 2 tiles in a direction the
// neighbour on either side is the same tile, but a pixel near the left edge
// reads that tile's right border entries and a pixel near the right edge its
// left border entries (the window's wrap around the torus of tiles), which
// are distinct words.  Tables with a radius above kRmax take the gather path
// inside the same launch.
// ---------------------------------------------------------------------------

// Forward, scatter form of the mirror term.  D = weight prefetch depth in
// shifts (loads for shift s + D are issued right after shift s is consumed).
// HALO = the LDS border of the tiles and windows: every row of the table
// must stay within it (|dx|, |dy| <= HALO), else the tile runs the gather
// algorithm (on a kRmax-halo tile).
template <typename T, int VEC, int TPR, int ROWS, int D, bool NTL, int HALO>
__device__ __forceinline__ void fwd_scatter_tile(
    const T* __restrict__ x, const T* __restrict__ w, const int64_t* __restrict__ shifts, int S,
    int codes, int C, int H, int W, int ntw, int nth, int64_t plane_step, acc_t<T>* __restrict__ U,
    acc_t<T>* __restrict__ Z, int* __restrict__ hdr, acc_t<T>* __restrict__ spill,
    int64_t ntiles, Band bd) {
    using A = acc_t<T>;
    using G = SGeo<VEC, ROWS, TPR, true, HALO>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* mu = xt + G::TILE;
    A* mz = mu + G::TILE;

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;

    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
    // Every row's x read must come from the LDS tile (|dx|, |dy| <= HALO),
    // and the mirror scatter must reach only adjacent tiles (radius at most
    // the narrowest tile, the partial last one); otherwise the tile runs the
    // gather algorithm.  Uniform over the launch.
    const int R = table_radius(shl, S, true);
    const bool far = table_radius(shl, S, false) > HALO ||
                     R > min(W - (ntw - 1) * G::TW, H - (nth - 1) * G::TH);
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr[0] = far ? kFarRadius : R;  // for the fix-up
    if (far) {
        // the gather algorithm reads a kRmax-halo tile (at this tile's pitch)
        stage_tile<T, A>(xt, x + ti.bc * HW, H, W, ti.h0, ti.w0, G::TH + 2 * kRmax,
                         G::TW + 2 * kRmax, G::PITCH);
        __syncthreads();
        fwd_gather_tile<T, VEC, 1, ROWS, 1, NTL, TPR, G::PITCH>(
            x, w, S, C, H, W, ti, plane_step, (codes & kCodesSharedW) != 0, U, Z, shl, xt, bd);
        return;
    }
    stage_tile<T, A>(xt, x + ti.bc * HW, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH, HALO);
    lds_zero(mu, G::TILE);  // also used at R = 0 by a (0, 0) mirror row
    lds_zero(mz, G::TILE);
    __syncthreads();

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const int hr = band_row(bd, h < H ? h : ti.h0);  // image row (box tests)
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + HALO) * G::PITCH + tx + HALO;  // pixel k at lc + k*TPR
    const int64_t b = ti.bc / C;
    const bool wsh = (codes & kCodesSharedW) != 0;
    const T* w_bc = w + weight_plane(b, ti.bc - b * C, C, wsh) * HW;  // shift s adds s * wstep
    const int64_t wstep = weight_step(plane_step, C, wsh);

    A xo[VEC], u[VEC], z[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        xo[k] = xt[lc + k * TPR];
        u[k] = z[k] = A(0);
    }
    // Weight prefetch ring.  Loads are unconditional (an idle pixel reads its
    // plane's first element; the tail re-reads plane S-1) so that no load
    // sits behind a branch and the wait counters keep D shifts in flight.
    PixSlot<T, VEC> wb[D];
#pragma unroll
    for (int d = 0; d < D; ++d)
        slot_load_pixels<T, VEC, TPR, NTL>(w_bc + static_cast<int64_t>(min(d, S - 1)) * wstep,
                                           px, wb[d]);

    // One shift: take the ring slot and refill it D shifts ahead, then the
    // forward term into registers and the mirror term scattered into the
    // window at q + s.
    // A wave owns whole tile rows, so scatters of shifts with equal dx never
    // touch another wave's target rows: a barrier is needed only when dx
    // changes (every target word still gets its terms in table order).
    // Branch-free: idle pixels (outside the image) compute and add 0.
    // Interior tiles (every pixel inside the image and every q + s inside it
    // for all rows of the table) need no box test or mirror mask: they run a
    // second, select-free copy of the loop (the masks cost about two thirds
    // of the loop's VALU instructions).
    const int R_all = table_radius(shl, S, false);
    const bool interior = ti.h0 >= R_all && ti.h0 + G::TH + R_all <= H && ti.w0 >= R_all &&
                          ti.w0 + G::TW + R_all <= W &&
                          band_rows_inside(bd, ti.h0, ti.h0 + G::TH - 1, -R_all) &&
                          band_rows_inside(bd, ti.h0, ti.h0 + G::TH - 1, R_all);
    int last_dx = kClamp;
    // Plane of the next refill, w_bc + min(s + D, S - 1) * wstep, advanced
    // one plane per shift (no 64-bit multiply per shift), and the next
    // shift's record, read one shift ahead (off the step's dependency chain).
    const T* wr = w_bc + static_cast<int64_t>(min(D, S - 1)) * wstep;
    ShiftRec rn = read_shift(shl, 0);
    auto run_loop = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        auto step = [&](int s, PixSlot<T, VEC>& slot) {
            const ShiftRec rc = rn;
            rn = read_shift(shl, min(s + 1, S - 1));
            const int op = lc + rc.dx * G::PITCH + rc.dy;  // window index of q + s
            // consume the slot, then refill it D shifts ahead at once
            A wv[VEC];
            slot_get_pixels<T, VEC>(slot, wv);
            slot_load_pixels<T, VEC, TPR, NTL>(wr, px, slot);
            wr += s + D + 1 < S ? wstep : 0;
            if constexpr (!FAST) {
                // Forward box: w_s[q] is dropped where q + s leaves the
                // image.  Only tiles that this shift carries past the image
                // edge test pixels (a uniform branch); the ring registers
                // are selected after it, never read inside it (that would
                // make the compiler wait for every load in flight).
                bool kept[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) kept[k] = true;
                if (rc.fbox &&
                    !tile_inside_band(bd, ti.h0, ti.w0, G::TH, G::TW, H, W, rc.dx, rc.dy)) {
                    const bool frow = in_range(hr + rc.dx, bd.Hg);
#pragma unroll
                    for (int k = 0; k < VEC; ++k)
                        kept[k] = frow && in_range(ti.w0 + tx + k * TPR + rc.dy, W);
                }
#pragma unroll
                for (int k = 0; k < VEC; ++k) wv[k] = kept[k] ? wv[k] : A(0);
            }
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                u[k] = fma_acc(wv[k], xt[op + k * TPR], u[k]);
                z[k] += wv[k];
            }
            if (rc.inv) {
                if (rc.dx != last_dx) {
                    lds_barrier();
                    last_dx = rc.dx;
                }
                // w_s[q] x[q] belongs to output q + s (inside the image, or
                // wrapped for a circular mirror: the fix-up's tile torus)
                if constexpr (FAST) {
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        mu[op + k * TPR] += wv[k] * xo[k];
                        mz[op + k * TPR] += wv[k];
                    }
                } else {
                    const bool rok = rc.per || in_range(hr + rc.dx, bd.Hg);
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        const bool ok = px.act[k] && rok &&
                                        (rc.per || in_range(ti.w0 + tx + k * TPR + rc.dy, W));
                        mu[op + k * TPR] += ok ? wv[k] * xo[k] : A(0);
                        mz[op + k * TPR] += ok ? wv[k] : A(0);
                    }
                }
            }
        };
        // Whole rings first (identical control flow every iteration, so the
        // wait counters keep D - 1 loads in flight), then the remainder.
        const int S_ring = S - S % D;
        for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) step(s0 + d, wb[d]);
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (S_ring + d < S) step(S_ring + d, wb[d]);
    };
    if (interior)
        run_loop(std::true_type{});
    else
        run_loop(std::false_type{});
    A* Ut = U + ti.bc * HW;
    A* Zt = Z + ti.bc * HW;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!px.act[k]) continue;
        Ut[px.own[k]] = u[k] + mu[lc + k * TPR];
        Zt[px.own[k]] = z[k] + mz[lc + k * TPR];
    }
    if (R == 0) return;
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    const int n = spill_count(th, tw, R);
    A* su = spill + t * G::SPILL;
    A* sz = spill + (ntiles + t) * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        const int li = (i + HALO) * G::PITCH + j + HALO;
        su[e] = mu[li];
        sz[e] = mz[li];
    }
}

#define NSH_FWD_SCATTER_PARAMS                                                                  \
    const T *__restrict__ x, const T *__restrict__ w, const int64_t *__restrict__ shifts, int S, \
        int codes, int C, int H, int W, int ntw, int nth, int64_t plane_step,                    \
        acc_t<T> *__restrict__ U, acc_t<T> *__restrict__ Z, int *__restrict__ hdr,              \
        acc_t<T> *__restrict__ spill, int64_t ntiles, Band bd
#define NSH_FWD_SCATTER_ARGS \
    x, w, shifts, S, codes, C, H, W, ntw, nth, plane_step, U, Z, hdr, spill, ntiles, bd

template <typename T, int VEC, int TPR, int ROWS, int D, bool NTL, int WPE, int HALO>
__global__ __launch_bounds__(TPR * ROWS, WPE) void accumulate_uz_fwd_scatter_kernel(
    NSH_FWD_SCATTER_PARAMS) {
    fwd_scatter_tile<T, VEC, TPR, ROWS, D, NTL, HALO>(NSH_FWD_SCATTER_ARGS);
}

// The same kernel held to 80 scalar registers (VCC and the other reserved
// ones included), the most that lets 10 waves share a SIMD.  The 2-pixel
// forward tiles take 44 vector registers and 28 KiB of LDS plus the table,
// so five 512-lane workgroups fit on a CU when the scalar registers do too;
// left to itself the compiler takes 88 + 6 of them (the band and far-table
// tests) and the CU holds four: the 1 M-pixel fp16 forward runs 0.104 ms
// that way and 0.095 ms held to 80 (a few scalar values move to vector
// lanes; a budget of 88 changes nothing).
template <typename T, int VEC, int TPR, int ROWS, int D, bool NTL, int WPE, int HALO>
__global__ __launch_bounds__(TPR * ROWS, WPE) __attribute__((amdgpu_num_sgpr(80))) void
accumulate_uz_fwd_scatter_narrow_kernel(NSH_FWD_SCATTER_PARAMS) {
    fwd_scatter_tile<T, VEC, TPR, ROWS, D, NTL, HALO>(NSH_FWD_SCATTER_ARGS);
}

#undef NSH_FWD_SCATTER_PARAMS
#undef NSH_FWD_SCATTER_ARGS

// The three tiles of the backward (x, gU, gZ) plus their HALO border
// (circular) staged together in the BwdLayout columns: each lane
// issues the loads of a batch of window elements of all three planes before
// it stores any, so one memory latency per batch instead of one per plane
// (c4 backward 7.68 -> 7.60 ms, c2 0.140 -> 0.133 ms).
template <typename T, typename A, typename L, int HALO>
__device__ __forceinline__ void stage3_tile_bwd(A* xl, const T* __restrict__ xp, A* ul,
                                                const A* __restrict__ up, A* zl,
                                                const A* __restrict__ zp, int H, int W, int h0,
                                                int w0, int LH, int LW) {
    constexpr int NB = kStageBatch;
    const bool cheap = H >= LH && W >= LW;  // one conditional wrap suffices
    const int n = LH * LW;
    const int step = static_cast<int>(blockDim.x);
    for (int base = threadIdx.x; base < n; base += step * NB) {
        T xv[NB];
        A uv[NB], zv[NB];
        int li[NB];
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int i = min(base + k * step, n - 1);  // tail: re-load, not stored
            const int r = i / LW;
            const int c = i - r * LW;
            int gh = h0 - HALO + r;
            int gw = w0 - HALO + c;
            if (cheap) {
                gh = wrap1(gh, H);
                gw = wrap1(gw, W);
            } else {
                gh = static_cast<int>(mod_pos(gh, H));
                gw = static_cast<int>(mod_pos(gw, W));
            }
            const uint32_t g = static_cast<uint32_t>(gh) * static_cast<uint32_t>(W) +
                               static_cast<uint32_t>(gw);
            li[k] = r * L::PITCH + L::col(c);
            xv[k] = xp[g];
            uv[k] = up[g];
            zv[k] = zp[g];
        }
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (base + k * step >= n) continue;
            xl[li[k]] = to_acc(xv[k]);
            ul[li[k]] = uv[k];
            zl[li[k]] = zv[k];
        }
    }
}

// Backward, scatter form of the x term: gx[(q+s) mod] += w_s[q] gU[q].
// gw and the mirror term of gx need only aligned w_s[q] and the LDS tiles.
// With a 16-bit T the gx partial sums go to `gxp` (accumulator type) and the
// fix-up rounds once; otherwise they go to gx directly.
// Lane ownership is contiguous here (SGeo<..., false>): the backward writes
// as many bytes as it reads (gw), and one 16-byte load and one 16-byte
// store per lane and shift measured faster than four 4-byte ones; the LDS
// tiles use the de-interleaved columns of BwdLayout so that these lanes'
// LDS accesses are conflict-free.
template <typename T, int VEC, int TPR, int ROWS, int D, bool NTL, int HALO = kRmax>
__global__ __launch_bounds__(TPR * ROWS) void accumulate_uz_bwd_scatter_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const acc_t<T>* __restrict__ gU,
    const acc_t<T>* __restrict__ gZ, const int64_t* __restrict__ shifts, int S, int codes, int C,
    int H, int W, int ntw, int nth, int64_t plane_step, T* __restrict__ gx, acc_t<T>* __restrict__ gxp,
    T* __restrict__ gw, int* __restrict__ hdr, acc_t<T>* __restrict__ spill, int64_t ntiles,
    Band bd) {
    using A = acc_t<T>;
    using G = SGeo<VEC, ROWS, TPR, false, HALO>;
    using L = BwdLayout<VEC, G::LW, G::PITCH>;
    static_assert(G::LH * L::PITCH <= G::TILE, "de-interleaved tile exceeds the LDS plan");
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* ut = xt + G::TILE;
    A* zt = ut + G::TILE;
    A* mg = zt + G::TILE;

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t off = ti.bc * HW;

    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
    // every row scatters its x term: radius within the halo and at most the
    // narrowest tile (the partial last one), else the gather algorithm
    const int R = table_radius(shl, S, false);
    const bool far = R > HALO || R > min(W - (ntw - 1) * G::TW, H - (nth - 1) * G::TH);
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr[0] = far ? kFarRadius : R;  // for the fix-up
    if (far) {
        // the gather algorithm reads row-major kRmax-halo tiles (at this
        // tile's pitch)
        constexpr int GLH = G::TH + 2 * kRmax, GLW = G::TW + 2 * kRmax;
        stage_tile<T, A>(xt, x + off, H, W, ti.h0, ti.w0, GLH, GLW, G::PITCH);
        stage_tile<A, A>(ut, gU + off, H, W, ti.h0, ti.w0, GLH, GLW, G::PITCH);
        stage_tile<A, A>(zt, gZ + off, H, W, ti.h0, ti.w0, GLH, GLW, G::PITCH);
        __syncthreads();
        bwd_gather_tile<T, VEC, 1, ROWS, 1, NTL, TPR, G::PITCH>(
            x, w, gU, gZ, S, C, H, W, ti, plane_step, (codes & kCodesSharedW) != 0, gx, gw, shl,
            xt, ut, zt, bd);
        return;
    }
    stage3_tile_bwd<T, A, L, HALO>(xt, x + off, ut, gU + off, zt, gZ + off, H, W, ti.h0, ti.w0,
                                   G::LH, G::LW);
    lds_zero(mg, G::TILE);
    __syncthreads();

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const int hr = band_row(bd, h < H ? h : ti.h0);  // image row (box tests)
    const int wq = ti.w0 + tx * VEC;
    const bool act = h < H && wq < W;
    const uint32_t own = static_cast<uint32_t>(act ? h : 0) * static_cast<uint32_t>(W) +
                         static_cast<uint32_t>(act ? wq : 0);
    // LDS index of the lane's pixel k displaced by (dx, dy):
    // lb + dx * PITCH + col(HALO + k + dy), the lane's own column folded into
    // lb (col(VEC tx + c) = tx + col(c) for c >= 0)
    const int lb = (ty + HALO) * L::PITCH + (L::DI ? tx : tx * VEC);
    const int64_t b = ti.bc / C;
    const bool wsh = (codes & kCodesSharedW) != 0;
    // planes are addressed as buffers: uniform base, the lane's byte offset
    const uint32_t own_b = own * static_cast<uint32_t>(sizeof(T));
    const T* w_bc = w + weight_plane(b, ti.bc - b * C, C, wsh) * HW;
    const int64_t wstep = weight_step(plane_step, C, wsh);
    T* g_bc = gw + ti.bc * HW;  // the gradient has every channel

    A xo[VEC], uo[VEC], zo[VEC], gxa[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const int i = lb + L::col(HALO + k);
        xo[k] = xt[i];
        uo[k] = ut[i];
        zo[k] = zt[i];
        gxa[k] = A(0);
    }
    // Weight prefetch ring.  Loads are unconditional (an idle lane reads its
    // plane's first vector; the tail re-reads plane S-1) so that no load sits
    // behind a branch and the wait counters can keep D loads in flight.
    SlotRaw<T, VEC> wb[D];
#pragma unroll
    for (int d = 0; d < D; ++d)
        slot_load_at<T, VEC, NTL>(w_bc + static_cast<int64_t>(min(d, S - 1)) * wstep, own_b, wb[d]);

    // One shift: take the ring slot and refill it D shifts ahead, then gw_s[q]
    // (streamed out), the mirror term of gx[q], and the x term of gx
    // scattered into the window at q + s.
    int last_dx = kClamp;  // barrier only when dx changes (see the forward)
    // next refill plane and next record, advanced per shift (see the forward)
    const T* wr = w_bc + static_cast<int64_t>(min(D, S - 1)) * wstep;
    ShiftRec rn = read_shift(shl, 0);
    T* gp = g_bc;  // gw_s plane of this shift
    auto step = [&](int s, SlotRaw<T, VEC>& slot) {
        const ShiftRec rc = rn;
        rn = read_shift(shl, min(s + 1, S - 1));
        // consume the slot, then refill it D shifts ahead at once
        A wv[VEC];
        slot_get<T, VEC>(slot, wv);
        slot_load_at<T, VEC, NTL>(wr, own_b, slot);
        wr += s + D + 1 < S ? wstep : 0;
        if (rc.dx != last_dx) {
            lds_barrier();
            last_dx = rc.dx;
        }
        if (act) {
            const int ob = lb + rc.dx * L::PITCH;
            int oi[VEC];
#pragma unroll
            for (int k = 0; k < VEC; ++k) oi[k] = ob + L::col(HALO + k + rc.dy);
            A xf[VEC], up_[VEC], zp_[VEC], g[VEC];
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                xf[k] = xt[oi[k]];
                up_[k] = ut[oi[k]];
                zp_[k] = zt[oi[k]];
            }
            const bool rok = rc.inv && (rc.per || in_range(hr + rc.dx, bd.Hg));
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const bool okp = rok && (rc.per || in_range(wq + k + rc.dy, W));
                // forward box: a dropped w_s[q] has no gradient and adds no
                // x-gradient term (its mirror is dropped too)
                const bool kept = fwd_kept(rc, hr, wq + k, bd.Hg, W);
                wv[k] = kept ? wv[k] : A(0);
                g[k] = kept ? fma_acc(xf[k], uo[k], zo[k]) : A(0);
                if (okp) {
                    g[k] += fma_acc(xo[k], up_[k], zp_[k]);
                    gxa[k] = fma_acc(wv[k], up_[k], gxa[k]);
                }
            }
            store_acc_at<T, VEC, true>(gp, own_b, g);
#pragma unroll
            for (int k = 0; k < VEC; ++k) mg[oi[k]] += wv[k] * uo[k];
        }
        gp += plane_step;
    };
    const int S_ring = S - S % D;
    for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) step(s0 + d, wb[d]);
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (S_ring + d < S) step(S_ring + d, wb[d]);
    __syncthreads();
    if (act) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) gxa[k] += mg[lb + L::col(HALO + k)];
        if (gxp != nullptr)
            store_out<A, VEC>(gxp + off + own, gxa);
        else
            store_acc<T, VEC>(gx + off + own, gxa, false);
    }
    if (R == 0) return;
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    const int n = spill_count(th, tw, R);
    A* sg = spill + t * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        sg[e] = mg[(i + HALO) * L::PITCH + L::col(j + HALO)];
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
constexpr size_t kLdsLimit = 80 * 1024;  // gather path: two workgroups per CU (160 KB LDS)

struct Dims {
    int S, B, C, H, W;
    int codes = 0;     // kCodesRows / kCodesSharedW (from NSH_SHIFT_CODES, NSH_SHARED_WEIGHTS)
    int halo = kRmax;  // scatter border the table asks for (NSH_WIDE_HALO 16, NSH_WIDER_HALO 24)
    Band band{0, 1};   // image rows of the local rows (whole image: {0, H})
};

// Gather path (no workspace, unaligned buffers, shapes the scatter path does
// not take): tiles of 16 lanes x VEC pixels by 32 rows, one row per lane,
// one shift's weight loads in flight per lane, banded tile order (bands of
// two tile rows, column-major inside a band).  Measured on MI355X, the
// alternatives (2 or 4 rows per lane, 2 or 4 shifts per load chunk, 16 or
// 64 rows, nontemporal loads, row-major order) were no faster; the scatter
// path replaced this one wherever it applies.
constexpr int kGatherRows = 32;
constexpr int kGatherOrder = 2, kGatherBand = 2;

template <typename T, int VEC, bool BWD>
static int launch_gather(const void* x, const void* w, const void* gU, const void* gZ,
                         const int64_t* shifts, const Dims& d, void* o0, void* o1,
                         hipStream_t st) {
    using G = Geo<VEC, 1, kGatherRows>;
    using A = acc_t<T>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    const size_t lds = shift_lds_bytes(d.S) + (BWD ? 3 : 1) * static_cast<size_t>(G::TILE) *
                                                  sizeof(A);
    if constexpr (BWD) {
        hipLaunchKernelGGL((accumulate_uz_bwd_kernel<T, VEC, 1, kGatherRows, 1, false>),
                           dim3(static_cast<unsigned>(tiles)), dim3(G::THREADS), lds, st,
                           static_cast<const T*>(x), static_cast<const T*>(w),
                           static_cast<const A*>(gU), static_cast<const A*>(gZ), shifts, d.S,
                           d.codes, d.C, d.H, d.W, ntw, nth, kGatherOrder, kGatherBand, step,
                           static_cast<T*>(o0), static_cast<T*>(o1), d.band);
        return nsh_host::check_launch("accumulate_uz_backward");
    } else {
        hipLaunchKernelGGL((accumulate_uz_fwd_kernel<T, VEC, 1, kGatherRows, 1, false>),
                           dim3(static_cast<unsigned>(tiles)), dim3(G::THREADS), lds, st,
                           static_cast<const T*>(x), static_cast<const T*>(w), shifts, d.S,
                           d.codes, d.C, d.H, d.W, ntw, nth, kGatherOrder, kGatherBand, step,
                           static_cast<A*>(o0), static_cast<A*>(o1), d.band);
        return nsh_host::check_launch("accumulate_uz_forward");
    }
}

template <int VEC>
static size_t gather_lds(int S, size_t ab, bool bwd) {
    return shift_lds_bytes(S) +
           static_cast<size_t>(bwd ? 3 : 1) * Geo<VEC, 1, kGatherRows>::TILE * ab;
}

// Lanes needed to keep every CU busy: 256 CUs x 32 waves x 64 lanes.
constexpr int64_t kFillLanes = int64_t(1) << 19;

// Widest vector such that every row start is aligned for it, the launch
// still has about kFillLanes lanes (small images trade vector width for
// occupancy) and the LDS budget holds; VEC = 1 handles any shape.
template <typename T>
static int pick_vec(int W, std::initializer_list<const void*> ptrs, int S, bool bwd,
                    int64_t pixels) {
    int maxv = 16 / static_cast<int>(sizeof(T));
    while (maxv > 1 && pixels / maxv < kFillLanes) maxv /= 2;
    const size_t ab = sizeof(acc_t<T>);
    for (int v = maxv; v > 1; v /= 2) {
        if (W % v) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && nsh_host::aligned(p, v * sizeof(T));
        if (!ok) continue;
        size_t lds = 0;
        switch (v) {
            case 8: lds = gather_lds<8>(S, ab, bwd); break;
            case 4: lds = gather_lds<4>(S, ab, bwd); break;
            default: lds = gather_lds<2>(S, ab, bwd); break;
        }
        if (lds <= kLdsLimit) return v;
    }
    return 1;
}

// ---- scatter path -----------------------------------------------------------

// Largest dynamic LDS a scatter plan may ask for (a CU has 160 KB).
constexpr size_t kScatterLdsLimit = 159 * 1024;

// Scatter tile per (type, vector width, pass, variant): TPR lanes x VEC
// pixels across, ROWS rows, weight prefetch depth D (shifts), HALO border.
// Measured on MI355X at 8192^2, S = 85 (fp32, VEC 4):
//  * forward: the weight stream's row segments decide.  128 x 32 tiles of
//    1024 lanes (32 lanes x 4 pixels per row: 512-byte row segments per
//    weight plane; 83 KB of LDS, one workgroup per CU) stream the weights at
//    about 6 TB/s: 4.5 ms, against 4.9 ms for 64 x 64 tiles (256-byte
//    segments, two workgroups per CU) and 4.0-4.4 vs 3.8 ms for the pure
//    stream of a mirror-free table; 256-pixel rows (64 lanes) gain nothing;
//  * backward (four LDS tiles, de-interleaved columns): 128 x 32 tiles of
//    1024 lanes (111 KB of LDS, one workgroup per CU) read and write
//    512-byte row segments: 8.1 ms, against 8.5-8.6 ms for 128 x 16 (two
//    512-lane workgroups per CU, more halo and spill per pixel), 8.5 ms for
//    256 x 16 and 13.4 ms for 256 x 8; prefetch depth 3 or 4: 8.2 ms.
// Variants:
//  * kVarWide: the first choice above (fp32-class types with VEC 4;
//    narrower vectors take 16 x VEC x 32 tiles of 512 lanes, fp64 32 x 16
//    tiles of 256 lanes, twice the workgroups: c3 fp64 forward 0.071 ->
//    0.067 ms, backward 0.173 -> 0.154 ms; 32 x 8 leaves too short a last
//    tile for many heights);
//  * kVarAlt: 64 x 32 tiles (16 lanes x 4 pixels), for images too narrow or
//    short for two tiles of the first choice;
//  * kVarShort: wide backward tiles of half the rows (128 x 16, two
//    workgroups per CU), for problems whose wide tiles would fill the CUs
//    only once (c2 fp16 backward 0.155 -> 0.142 ms);
//  * kVarHalo16: a 16-pixel border for tables of radius 9..16 (fp32-class
//    types with VEC 4): forward 128 x 32 (151 KB of LDS at S = 1024),
//    backward 128 x 16 (one 512-lane workgroup per CU);
//  * kVarHalo24: a 24-pixel border for radius 17..24 (the half-plane up to
//    R = 22, S = 1013): 64 x 32 tiles of 512 lanes in both passes (forward
//    124 KB of LDS, backward 157 KB at S = 1024).
// Prefetch depth 2, except 4 for the 16-bit backward on the wide tiles (c2
// fp16 backward 0.172 -> 0.165 ms; depth 4 made the c3 fp64 passes 7-10%
// slower) and 6 for the passes on the wider borders with one 512-lane
// workgroup per CU, which keep too few loads in flight at depth 2 (4096^2
// fp32: 16-pixel border backward, half-plane R = 15 16.0 -> 11.8 ms, window
// R = 15 30.6 -> 22.5 ms, depths 3, 4 and 8 no better than 2, depth 5 close
// to 6; 24-pixel border forward, R = 22 16.8-17.1 -> 15.5 ms, 15.7 ms at
// depth 4).  Nontemporal weight loads: the wide forward 4.22 -> 4.13 ms at c4,
// the wide fp32 backward 7.97 -> 7.88 ms at c4 and 0.630 -> 0.607 ms at c3,
// the fp64 forward 0.077-0.080 -> 0.071-0.073 ms at c3; the 64-wide
// forward and backward were 2-5% slower with them (c3), the 16-bit (c2) and
// fp64 backwards 1-2% slower.
enum { kVarWide = 0, kVarAlt = 1, kVarShort = 2, kVarHalo16 = 3, kVarHalo24 = 4 };

template <typename T, int VEC, bool BWD, int VAR = kVarWide>
struct ScatterCfg {
    static constexpr bool kFp32Class = sizeof(acc_t<T>) == 4;
    static constexpr bool kWide = kFp32Class && VEC == 4 && VAR != kVarAlt;
    static constexpr bool kBigHalo = VAR == kVarHalo16 || VAR == kVarHalo24;
    static_assert(!kBigHalo || kWide, "the wider borders are built for 4-pixel lanes");
    static constexpr int HALO = VAR == kVarHalo16 ? 16 : (VAR == kVarHalo24 ? 24 : kRmax);
    static constexpr int TPR = (kWide && VAR != kVarHalo24) ? 32 : kTPR;
    static constexpr int ROWS =
        (kWide ? (BWD && (VAR == kVarShort || VAR == kVarHalo16)) : sizeof(T) == 8) ? 16 : 32;
    static constexpr int D = (kWide && kBigHalo && (BWD || VAR == kVarHalo24)) ? 6
                             : (kWide && BWD && sizeof(T) == 2) ? 4 : 2;
    // Register budget (waves per SIMD): the wide forward tile's LDS admits
    // one workgroup per CU, i.e. four waves per SIMD.
    static constexpr int WPE = (kWide && !BWD && TPR * ROWS == 1024) ? 4
                                                                     : kScatterWavesPerEU<TPR * ROWS>;
    static constexpr bool NTL = BWD ? (kWide && sizeof(T) == 4) : (kWide || sizeof(T) == 8);
    // the 2-pixel forward lanes of 16- and 32-bit types (44 vector registers
    // under the budget, so 10 waves per SIMD): held to 80 scalar registers
    // (accumulate_uz_fwd_scatter_narrow_kernel).  Under the same budget the
    // 1-pixel lanes take 49-56 vector registers (no tenth wave) and the
    // 4-pixel ones 74.
    static constexpr bool kSgpr80 = !BWD && !kWide && VEC == 2 && sizeof(T) <= 4;
};

static int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// Workspace layout: [header: table radius, 256 B][spill blocks][16-bit gx
// partial sums (backward only)].
constexpr int64_t kHeaderBytes = 256;

struct SPlan {
    bool ok = false;
    int rows = 0, ntw = 0, nth = 0, spill = 0, halo = kRmax;
    int64_t tiles = 0, spill_bytes = 0, part_bytes = 0, total = 0;
    size_t lds = 0;
};

// Geometry and workspace of the scatter path for a given vector width.
// Eligibility: at least 2 tiles in each direction and every tile at least
// kRmax wide and high, so that a window's border reaches only adjacent tiles
// for any radius up to kRmax (the kernels run the gather form inside the
// launch for a table whose radius exceeds the halo or the narrowest tile).
static SPlan scatter_plan(const Dims& d, int vec, int tpr, int rows, int halo, size_t tsize,
                          size_t asize, bool bwd) {
    SPlan p;
    const int TW = tpr * vec, TH = rows;
    const int LW = TW + 2 * halo;
    // SGeo::TILE: the forward kernel is strided; the backward contiguous,
    // whose de-interleaved rows (VEC 2, 4) take a pitch = 16 mod 32
    const int strided_pitch = LW + ((16 - LW % 32) + 32) % 32;
    const int pitch = !bwd ? strided_pitch
                           : ((vec == 2 || vec == 4) ? std::max(LW + 1, strided_pitch) : LW + 1);
    const size_t tile = static_cast<size_t>(TH + 2 * halo) * pitch * asize;
    p.lds = shift_lds_bytes(d.S) + (bwd ? 4 : 3) * tile;
    p.rows = rows;
    p.halo = halo;
    p.ntw = static_cast<int>(nsh_host::ceil_div(d.W, TW));
    p.nth = static_cast<int>(nsh_host::ceil_div(d.H, TH));
    p.ok = p.lds <= kScatterLdsLimit && p.ntw >= 2 && p.nth >= 2 && TH >= halo &&
           d.W - (p.ntw - 1) * TW >= kRmax && d.H - (p.nth - 1) * TH >= kRmax;
    p.tiles = static_cast<int64_t>(d.B) * d.C * p.ntw * p.nth;
    p.spill = 2 * halo * (TW + 2 * halo) + 2 * halo * TH;
    p.spill_bytes = align256((bwd ? 1 : 2) * p.tiles * p.spill * static_cast<int64_t>(asize));
    p.part_bytes = (bwd && tsize < asize)
                       ? align256(static_cast<int64_t>(d.B) * d.C * d.H * d.W *
                                  static_cast<int64_t>(asize))
                       : 0;
    p.total = kHeaderBytes + p.spill_bytes + p.part_bytes;
    return p;
}

// Vector width of the scatter path from the shape alone (the workspace size
// must not depend on pointer values): the widest vector of at most 4
// elements (2 for fp64) that divides W and still leaves at least the pass's
// fill-lane count.  Measured on MI355X: the c3 fp64 forward (393,216
// pixels) runs 0.112 ms on 1-wide and 0.078 ms on 2-wide lanes, its
// backward 0.179-0.180 ms on 1-wide and 0.173-0.174 ms on 2-wide lanes (so
// fp64 takes the forward's fill count in both passes), the c2 fp16 backward
// (1 M pixels) 0.179 ms on 2-wide and 0.168 ms on 4-wide lanes, the c2 fp16
// forward 0.109 ms on 2-wide and 0.116 ms on 4-wide lanes; the c4 and c3
// fp32 shapes are 4-wide either way.
constexpr int64_t kScatterFillFwd = int64_t(1) << 17;
constexpr int64_t kScatterFillFwd16 = int64_t(1) << 19;
constexpr int64_t kScatterFillBwd = int64_t(1) << 18;

template <typename T>
static int scatter_vec(const Dims& d, bool bwd) {
    const int64_t pixels = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    const int64_t fill = bwd ? (sizeof(T) == 8 ? kScatterFillFwd : kScatterFillBwd)
                             : (sizeof(T) == 2 ? kScatterFillFwd16 : kScatterFillFwd);
    int maxv = sizeof(T) == 8 ? 2 : 4;
    while (maxv > 1 && pixels / maxv < fill) maxv /= 2;
    for (int v = maxv; v > 1; v /= 2)
        if (d.W % v == 0) return v;
    return 1;
}

template <typename T, int VEC, bool BWD, int VAR>
static SPlan scatter_plan_cfg(const Dims& d) {
    using Cfg = ScatterCfg<T, VEC, BWD, VAR>;
    return scatter_plan(d, VEC, Cfg::TPR, Cfg::ROWS, Cfg::HALO, sizeof(T), sizeof(acc_t<T>),
                        BWD);
}

// The backward's wide tiles hold one workgroup per CU (their LDS), so a
// problem of at most one tile per CU (c2: 256 tiles of 128 x 32) leaves each
// CU one workgroup whose waves all meet at every barrier; half-height tiles
// put two independent workgroups on each CU (c2 fp16 backward 0.155 ->
// 0.142 ms; at c3 and c4, many tiles per CU, they cost 3-9% of halo and
// spill, so those keep the full height).  One round is one tile per compute
// unit of the current device (256 on MI355X, also the fallback when no device
// can be queried, e.g. a workspace query from a process without a GPU).
static int64_t one_round_tiles() { return nsh_host::compute_units(); }

// The plan for a shape: with the wide halo asked for, the 16-pixel-border
// tiles where they apply; else the first choice (the half-height backward
// tiles when the full-height ones fill the CUs once), else the second
// choice; *var says which (p.ok false if none applies).
template <typename T, int VEC, bool BWD>
static SPlan scatter_plan_for(const Dims& d, int* var) {
    if constexpr (ScatterCfg<T, VEC, BWD, kVarWide>::kWide) {
        if (d.halo > kRmax) {
            const SPlan q = d.halo > 16 ? scatter_plan_cfg<T, VEC, BWD, kVarHalo24>(d)
                                        : scatter_plan_cfg<T, VEC, BWD, kVarHalo16>(d);
            if (q.ok) {
                *var = d.halo > 16 ? kVarHalo24 : kVarHalo16;
                return q;
            }
        }
    }
    SPlan p = scatter_plan_cfg<T, VEC, BWD, kVarWide>(d);
    *var = kVarWide;
    if constexpr (BWD && ScatterCfg<T, VEC, true, kVarWide>::kWide) {
        if (p.ok && p.tiles <= one_round_tiles()) {
            const SPlan q = scatter_plan_cfg<T, VEC, true, kVarShort>(d);
            if (q.ok) {
                *var = kVarShort;
                return q;
            }
        }
    }
    if (!p.ok) {
        p = scatter_plan_cfg<T, VEC, BWD, kVarAlt>(d);
        *var = kVarAlt;
    }
    return p;
}

template <typename T, bool BWD>
static SPlan scatter_plan_any(const Dims& d, int vec, int* var) {
    switch (vec) {
        case 4: if constexpr (sizeof(T) <= 4) return scatter_plan_for<T, 4, BWD>(d, var); break;
        case 2: return scatter_plan_for<T, 2, BWD>(d, var);
        default: break;
    }
    return scatter_plan_for<T, 1, BWD>(d, var);
}

template <typename T>
static int64_t scatter_workspace(const Dims& d, bool bwd) {
    int var;
    const SPlan p = bwd ? scatter_plan_any<T, true>(d, scatter_vec<T>(d, true), &var)
                        : scatter_plan_any<T, false>(d, scatter_vec<T>(d, false), &var);
    return p.ok ? p.total : 0;
}

// NSH_ACC_SCATTER=0 (read once per process): the gather kernels only, a
// diagnostic switch (same results within the summation-order tolerance).
static bool scatter_disabled() {
    static const bool off = [] {
        const char* e = getenv("NSH_ACC_SCATTER");
        return e != nullptr && e[0] == '0';
    }();
    return off;
}

template <typename T, int VEC, int VAR>
static int launch_fwd_scatter(const void* x, const void* w, const int64_t* sh, const Dims& d,
                              const SPlan& p, void* U, void* Z, void* ws, hipStream_t st) {
    using A = acc_t<T>;
    using Cfg = ScatterCfg<T, VEC, false, VAR>;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    int* hdr = static_cast<int*>(ws);
    A* spill = reinterpret_cast<A*>(static_cast<char*>(ws) + kHeaderBytes);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(p.tiles)),
                           dim3(Cfg::TPR * Cfg::ROWS), p.lds, st, static_cast<const T*>(x),
                           static_cast<const T*>(w), sh, d.S, d.codes, d.C, d.H, d.W, p.ntw,
                           p.nth, step, static_cast<A*>(U), static_cast<A*>(Z), hdr, spill,
                           p.tiles, d.band);
    };
    if constexpr (Cfg::kSgpr80)
        launch(accumulate_uz_fwd_scatter_narrow_kernel<T, VEC, Cfg::TPR, Cfg::ROWS, Cfg::D,
                                                       Cfg::NTL, Cfg::WPE, Cfg::HALO>);
    else
        launch(accumulate_uz_fwd_scatter_kernel<T, VEC, Cfg::TPR, Cfg::ROWS, Cfg::D, Cfg::NTL,
                                                Cfg::WPE, Cfg::HALO>);
    if (int rc = nsh_host::check_launch("accumulate_uz_forward")) return rc;
    hipLaunchKernelGGL((spill_fixup_kernel<A, A, 2, false>),
                       dim3(static_cast<unsigned>(p.tiles)), dim3(256), 0, st, d.H, d.W,
                       Cfg::ROWS, Cfg::TPR * VEC, p.ntw, p.nth, p.spill,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill), p.tiles,
                       static_cast<const A*>(nullptr), static_cast<A*>(U), static_cast<A*>(Z));
    return nsh_host::check_launch("accumulate_uz_forward (fix-up)");
}

template <typename T, int VEC, int VAR>
static int launch_bwd_scatter(const void* x, const void* w, const void* gU, const void* gZ,
                              const int64_t* sh, const Dims& d, const SPlan& p, void* gx,
                              void* gw, void* ws, hipStream_t st) {
    using A = acc_t<T>;
    using Cfg = ScatterCfg<T, VEC, true, VAR>;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    char* base = static_cast<char*>(ws);
    int* hdr = reinterpret_cast<int*>(base);
    A* spill = reinterpret_cast<A*>(base + kHeaderBytes);
    A* part = p.part_bytes ? reinterpret_cast<A*>(base + kHeaderBytes + p.spill_bytes) : nullptr;
    hipLaunchKernelGGL((accumulate_uz_bwd_scatter_kernel<T, VEC, Cfg::TPR, Cfg::ROWS, Cfg::D,
                                                         Cfg::NTL, Cfg::HALO>),
                       dim3(static_cast<unsigned>(p.tiles)), dim3(Cfg::TPR * Cfg::ROWS), p.lds,
                       st, static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<const A*>(gU), static_cast<const A*>(gZ), sh, d.S, d.codes,
                       d.C, d.H, d.W, p.ntw, p.nth, step, static_cast<T*>(gx), part,
                       static_cast<T*>(gw), hdr, spill, p.tiles, d.band);
    if (int rc = nsh_host::check_launch("accumulate_uz_backward")) return rc;
    constexpr bool kPart = sizeof(T) < sizeof(A);
    hipLaunchKernelGGL((spill_fixup_kernel<T, A, 1, kPart>),
                       dim3(static_cast<unsigned>(p.tiles)), dim3(256), 0, st, d.H, d.W,
                       Cfg::ROWS, Cfg::TPR * VEC, p.ntw, p.nth, p.spill,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill), p.tiles,
                       static_cast<const A*>(part), static_cast<T*>(gx), static_cast<T*>(nullptr));
    return nsh_host::check_launch("accumulate_uz_backward (fix-up)");
}

template <typename T, int VEC, bool BWD>
static int launch_scatter_var(int var, const void* x, const void* w, const void* gU,
                              const void* gZ, const int64_t* sh, const Dims& d, const SPlan& p,
                              void* o0, void* o1, void* ws, hipStream_t st) {
    auto go = [&](auto var_tag) {
        constexpr int V = decltype(var_tag)::value;
        if constexpr (BWD)
            return launch_bwd_scatter<T, VEC, V>(x, w, gU, gZ, sh, d, p, o0, o1, ws, st);
        else
            return launch_fwd_scatter<T, VEC, V>(x, w, sh, d, p, o0, o1, ws, st);
    };
    if constexpr (ScatterCfg<T, VEC, BWD, kVarWide>::kWide) {
        if (var == kVarHalo16) return go(std::integral_constant<int, kVarHalo16>{});
        if (var == kVarHalo24) return go(std::integral_constant<int, kVarHalo24>{});
        if constexpr (BWD)
            if (var == kVarShort) return go(std::integral_constant<int, kVarShort>{});
    }
    if (var == kVarAlt) return go(std::integral_constant<int, kVarAlt>{});
    return go(std::integral_constant<int, kVarWide>{});
}

// Try the scatter path; returns -1 when it does not apply (then the gather
// kernels run).
template <typename T, bool BWD>
static int try_scatter(const void* x, const void* w, const void* gU, const void* gZ,
                       const int64_t* sh, const Dims& d, void* o0, void* o1, void* ws,
                       int64_t ws_bytes, hipStream_t st) {
    if (ws == nullptr || scatter_disabled()) return -1;
    const int v = scatter_vec<T>(d, BWD);
    int var = kVarWide;
    const SPlan p = scatter_plan_any<T, BWD>(d, v, &var);
    if (!p.ok || ws_bytes < p.total || !nsh_host::aligned(ws, 256)) return -1;
    const size_t vb = static_cast<size_t>(v) * sizeof(T);
    for (const void* q : {x, w, static_cast<const void*>(o0), static_cast<const void*>(o1)})
        if (!nsh_host::aligned(q, vb)) return -1;
    if (BWD && (!nsh_host::aligned(gU, v * sizeof(acc_t<T>)) ||
                !nsh_host::aligned(gZ, v * sizeof(acc_t<T>))))
        return -1;
    if (!BWD && (!nsh_host::aligned(o0, v * sizeof(acc_t<T>)) ||
                 !nsh_host::aligned(o1, v * sizeof(acc_t<T>))))
        return -1;
    switch (v) {
        case 4:
            if constexpr (sizeof(T) <= 4)
                return launch_scatter_var<T, 4, BWD>(var, x, w, gU, gZ, sh, d, p, o0, o1, ws, st);
            break;
        case 2: return launch_scatter_var<T, 2, BWD>(var, x, w, gU, gZ, sh, d, p, o0, o1, ws, st);
        default: break;
    }
    return launch_scatter_var<T, 1, BWD>(var, x, w, gU, gZ, sh, d, p, o0, o1, ws, st);
}

template <typename T, bool BWD>
static int run(const void* x, const void* w, const void* gU, const void* gZ, const int64_t* sh,
               Dims d, void* o0, void* o1, void* ws, int64_t ws_bytes, hipStream_t st) {
    const int rs = try_scatter<T, BWD>(x, w, gU, gZ, sh, d, o0, o1, ws, ws_bytes, st);
    if (rs >= 0) return rs;
    const int64_t pixels = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    const int v = BWD ? pick_vec<T>(d.W, {x, w, gU, gZ, o0, o1}, d.S, true, pixels)
                      : pick_vec<T>(d.W, {x, w, o0, o1}, d.S, false, pixels);
    switch (v) {
        case 8: if constexpr (sizeof(T) == 2) return launch_gather<T, 8, BWD>(x, w, gU, gZ, sh, d, o0, o1, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return launch_gather<T, 4, BWD>(x, w, gU, gZ, sh, d, o0, o1, st); break;
        case 2: return launch_gather<T, 2, BWD>(x, w, gU, gZ, sh, d, o0, o1, st);
        default: break;
    }
    return launch_gather<T, 1, BWD>(x, w, gU, gZ, sh, d, o0, o1, st);
}

}  // namespace nsh

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using nsh_host::fail;

static int check_acc_dims(const char* op, int64_t S, int64_t B, int64_t C, int64_t H, int64_t W,
                          int dtype, nsh::Dims* d) {
    d->codes = nsh::dtype_codes(dtype);
    d->halo = (dtype & NSH_WIDER_HALO) ? 24 : ((dtype & NSH_WIDE_HALO) ? 16 : nsh::kRmax);
    dtype &= ~NSH_DTYPE_FLAGS;
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
    d->band = nsh::Band{0, d->H};
    return NSH_OK;
}

extern "C" int64_t nsh_accumulate_uz_workspace_bytes(int64_t S, int64_t B, int64_t C, int64_t H,
                                                     int64_t W, int dtype, int backward) {
    nsh::Dims d;
    if (check_acc_dims("accumulate_uz_workspace_bytes", S, B, C, H, W, dtype, &d)) return -1;
    dtype &= ~NSH_DTYPE_FLAGS;
    const bool bwd = backward != 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::scatter_workspace<nsh::f16>(d, bwd);
        case NSH_DTYPE_BFLOAT16: return nsh::scatter_workspace<nsh::bf16>(d, bwd);
        case NSH_DTYPE_FLOAT32: return nsh::scatter_workspace<float>(d, bwd);
        default: return nsh::scatter_workspace<double>(d, bwd);
    }
}

// Optional band: local row h is image row (row_origin + h) mod image_height
// in every box test (nsh::Band).
static int band_dims(const char* op, int64_t row_origin, int64_t image_height, nsh::Dims* d) {
    if (image_height < 1 || image_height > nsh::kClamp || row_origin < -nsh::kClamp ||
        row_origin > nsh::kClamp)
        return fail(NSH_ERR_INVALID,
                    "%s: band rows need 1 <= image_height <= 2^30 and |row_origin| <= 2^30", op);
    d->band = nsh::Band{static_cast<int>(row_origin), static_cast<int>(image_height)};
    return NSH_OK;
}

static int acc_forward(const char* op, const void* x, const void* weights, const int64_t* shifts,
                       int64_t S, int64_t B, int64_t C, int64_t H, int64_t W, int dtype, void* U,
                       void* Z, void* workspace, int64_t workspace_bytes, void* stream,
                       const int64_t* band) {
    nsh::Dims d;
    if (int rc = check_acc_dims(op, S, B, C, H, W, dtype, &d)) return rc;
    if (band)
        if (int rc = band_dims(op, band[0], band[1], &d)) return rc;
    dtype &= ~NSH_DTYPE_FLAGS;
    if (!x || !weights || !shifts || !U || !Z)
        return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = workspace;
    const int64_t wb = workspace_bytes;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            return nsh::run<nsh::f16, false>(x, weights, nullptr, nullptr, shifts, d, U, Z, ws, wb, st);
        case NSH_DTYPE_BFLOAT16:
            return nsh::run<nsh::bf16, false>(x, weights, nullptr, nullptr, shifts, d, U, Z, ws, wb, st);
        case NSH_DTYPE_FLOAT32:
            return nsh::run<float, false>(x, weights, nullptr, nullptr, shifts, d, U, Z, ws, wb, st);
        default:
            return nsh::run<double, false>(x, weights, nullptr, nullptr, shifts, d, U, Z, ws, wb, st);
    }
}

static int acc_backward(const char* op, const void* x, const void* weights, const void* gU,
                        const void* gZ, const int64_t* shifts, int64_t S, int64_t B, int64_t C,
                        int64_t H, int64_t W, int dtype, void* grad_x, void* grad_w,
                        void* workspace, int64_t workspace_bytes, void* stream,
                        const int64_t* band) {
    nsh::Dims d;
    if (int rc = check_acc_dims(op, S, B, C, H, W, dtype, &d)) return rc;
    if (band)
        if (int rc = band_dims(op, band[0], band[1], &d)) return rc;
    dtype &= ~NSH_DTYPE_FLAGS;
    if (!x || !weights || !gU || !gZ || !shifts || !grad_x || !grad_w)
        return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = workspace;
    const int64_t wb = workspace_bytes;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            return nsh::run<nsh::f16, true>(x, weights, gU, gZ, shifts, d, grad_x, grad_w, ws, wb, st);
        case NSH_DTYPE_BFLOAT16:
            return nsh::run<nsh::bf16, true>(x, weights, gU, gZ, shifts, d, grad_x, grad_w, ws, wb, st);
        case NSH_DTYPE_FLOAT32:
            return nsh::run<float, true>(x, weights, gU, gZ, shifts, d, grad_x, grad_w, ws, wb, st);
        default:
            return nsh::run<double, true>(x, weights, gU, gZ, shifts, d, grad_x, grad_w, ws, wb, st);
    }
}

extern "C" int nsh_accumulate_uz_forward(const void* x, const void* weights, const int64_t* shifts,
                                         int64_t S, int64_t B, int64_t C, int64_t H, int64_t W,
                                         int dtype, void* U, void* Z, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
    return acc_forward("accumulate_uz", x, weights, shifts, S, B, C, H, W, dtype, U, Z,
                       workspace, workspace_bytes, stream, nullptr);
}

extern "C" int nsh_accumulate_uz_backward(const void* x, const void* weights, const void* grad_U,
                                          const void* grad_Z, const int64_t* shifts, int64_t S,
                                          int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                                          void* grad_x, void* grad_w, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
    return acc_backward("accumulate_uz_backward", x, weights, grad_U, grad_Z, shifts, S, B, C, H,
                        W, dtype, grad_x, grad_w, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int nsh_accumulate_uz_forward_band(const void* x, const void* weights,
                                              const int64_t* shifts, int64_t S, int64_t B,
                                              int64_t C, int64_t H, int64_t W,
                                              int64_t row_origin, int64_t image_height, int dtype,
                                              void* U, void* Z, void* workspace,
                                              int64_t workspace_bytes, void* stream) {
    const int64_t band[2] = {row_origin, image_height};
    return acc_forward("accumulate_uz_forward_band", x, weights, shifts, S, B, C, H, W, dtype, U,
                       Z, workspace, workspace_bytes, stream, band);
}

extern "C" int nsh_accumulate_uz_backward_band(const void* x, const void* weights,
                                               const void* grad_U, const void* grad_Z,
                                               const int64_t* shifts, int64_t S, int64_t B,
                                               int64_t C, int64_t H, int64_t W,
                                               int64_t row_origin, int64_t image_height,
                                               int dtype, void* grad_x, void* grad_w,
                                               void* workspace, int64_t workspace_bytes,
                                               void* stream) {
    const int64_t band[2] = {row_origin, image_height};
    return acc_backward("accumulate_uz_backward_band", x, weights, grad_U, grad_Z, shifts, S, B,
                        C, H, W, dtype, grad_x, grad_w, workspace, workspace_bytes, stream, band);
}
