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
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include <type_traits>

#include "nsh_common.hpp"

namespace nsh {

// Tile geometry: kTPR lanes x VEC pixels across, ROWS lanes x RPT rows down
// (a lane owns rows ty, ty + ROWS, ... so each ROWS-row pass of the
// workgroup is contiguous); the workgroup has kTPR * ROWS lanes.  LDS tiles
// carry a kRmax halo and an odd row pitch.
template <int VEC, int RPT, int ROWS>
struct Geo {
    static constexpr int THREADS = kTPR * ROWS;
    static constexpr int TW = kTPR * VEC;
    static constexpr int TH = ROWS * RPT;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
    static constexpr int PITCH = LW + 1;
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

// Per-lane pixel block: RPT rows x VEC columns.
template <int VEC, int RPT>
struct Lane {
    int w0;
    int h[RPT];
    bool row_ok[RPT];
    uint32_t own[RPT];  // h*W + w0
    int lc[RPT];        // LDS index of (h, w0)
};

template <int VEC, int RPT, int ROWS>
__device__ __forceinline__ Lane<VEC, RPT> lane_of(const TileIdx& ti, int W, int H) {
    using G = Geo<VEC, RPT, ROWS>;
    Lane<VEC, RPT> L;
    const int tx = threadIdx.x % kTPR;
    const int ty = threadIdx.x / kTPR;
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
template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL>
__global__ __launch_bounds__(kTPR * ROWS) void accumulate_uz_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const int64_t* __restrict__ shifts,
    int S, int C, int H, int W, int ntw, int nth, int order, int band, int64_t plane_step,
    acc_t<T>* __restrict__ U, acc_t<T>* __restrict__ Z) {
    using A = acc_t<T>;
    using G = Geo<VEC, RPT, ROWS>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW, order, band);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;

    stage_shifts(shl, shifts, S, 3, H, W);
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    __syncthreads();

    const Lane<VEC, RPT> L = lane_of<VEC, RPT, ROWS>(ti, W, H);
    if (L.w0 >= W) return;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* w_bc = w + (b * C + c) * HW;  // shift s adds s * plane_step (= B*C*HW)
    const bool full_rows = ti.h0 + G::TH <= H;  // every lane row inside the image

    A u[RPT][VEC], z[RPT][VEC];
#pragma unroll
    for (int r = 0; r < RPT; ++r)
#pragma unroll
        for (int k = 0; k < VEC; ++k) u[r][k] = z[r][k] = A(0);

    for (int s0 = 0; s0 < S; s0 += P) {
        ShiftRec rc[P];
        bool act[P], inside[P];
        const T* wp[P];
        A wv[P][RPT][VEC], wm[P][RPT][VEC];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            act[p] = s0 + p < S;
            rc[p] = read_shift(shl, act[p] ? s0 + p : s0);
            wp[p] = w_bc + static_cast<int64_t>(s0 + p) * plane_step;
            inside[p] = tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, -rc[p].dx, -rc[p].dy);
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
#pragma unroll
                for (int r = 0; r < RPT; ++r) {
                    const bool rok = L.row_ok[r] && in_range(L.h[r] - rc[p].dx, H);
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        const bool ok = rok && in_range(L.w0 + k - rc[p].dy, W);
                        wm[p][r][k] = ok ? to_acc(wp[p][static_cast<int64_t>(L.own[r]) + off + k]) : A(0);
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
            const bool fast = lds && inside[p] && full_rows;
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
                    u[r][k] = __builtin_fma(wv[p][r][k], xv[k], u[r][k]);
                    z[r][k] += wv[p][r][k];
                }
                if (!sr.inv) continue;
                if (fast) {
                    const A* xr = xt + L.lc[r] - sr.dx * G::PITCH - sr.dy;
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        u[r][k] = __builtin_fma(wm[p][r][k], xr[k], u[r][k]);
                        z[r][k] += wm[p][r][k];
                    }
                } else {
                    const bool rok = L.row_ok[r] && in_range(L.h[r] - sr.dx, H);
#pragma unroll
                    for (int k = 0; k < VEC; ++k) {
                        const int ws = L.w0 + k - sr.dy;
                        if (!(rok && in_range(ws, W))) continue;
                        const A xi = lds ? xt[L.lc[r] - sr.dx * G::PITCH - sr.dy + k]
                                         : to_acc(xp[static_cast<uint32_t>(L.h[r] - sr.dx) * W + ws]);
                        u[r][k] = __builtin_fma(wm[p][r][k], xi, u[r][k]);
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

// ---------------------------------------------------------------------------
// Fused backward: one pass over the weight planes produces gw (written once,
// streaming) and gx (register sums).  x, gU and gZ tiles with halo live in
// LDS; weight loads of a chunk of P shifts are issued before any use.
// ---------------------------------------------------------------------------
template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL>
__global__ __launch_bounds__(kTPR * ROWS) void accumulate_uz_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const acc_t<T>* __restrict__ gU,
    const acc_t<T>* __restrict__ gZ, const int64_t* __restrict__ shifts, int S, int C, int H,
    int W, int ntw, int nth, int order, int band, int64_t plane_step, T* __restrict__ gx,
    T* __restrict__ gw) {
    using A = acc_t<T>;
    using G = Geo<VEC, RPT, ROWS>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));
    A* ut = xt + G::TILE;
    A* zt = ut + G::TILE;

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW, order, band);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;
    const A* up = gU + ti.bc * HW;
    const A* zp = gZ + ti.bc * HW;

    stage_shifts(shl, shifts, S, 3, H, W);
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    stage_tile<A, A>(ut, up, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    stage_tile<A, A>(zt, zp, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    __syncthreads();

    const Lane<VEC, RPT> L = lane_of<VEC, RPT, ROWS>(ti, W, H);
    if (L.w0 >= W) return;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* w_bc = w + (b * C + c) * HW;
    T* g_bc = gw + (b * C + c) * HW;

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
            wp[p] = w_bc + static_cast<int64_t>(s0 + p) * plane_step;
            minus_in[p] = tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, -rc[p].dx, -rc[p].dy);
            plus_in[p] = tile_inside(ti.h0, ti.w0, G::TH, G::TW, H, W, rc[p].dx, rc[p].dy);
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
                    const bool rok = plus_in[p] || in_range(L.h[r] + sr.dx, H);
#pragma unroll
                    for (int k = 0; k < VEC; ++k)
                        okp[k] = sr.inv && (plus_in[p] || (rok && in_range(L.w0 + k + sr.dy, W)));
                }
                A g[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    g[k] = __builtin_fma(xf[k], uo[r][k], zo[r][k]);
                    if (okp[k]) g[k] += __builtin_fma(xo[r][k], up_[k], zp_[k]);
                    gxa[r][k] = __builtin_fma(ws[p][r][k], um[k], gxa[r][k]);
                    if (okp[k]) gxa[r][k] = __builtin_fma(wv[p][r][k], up_[k], gxa[r][k]);
                }
                if (L.row_ok[r]) store_acc<T, VEC>(gp + L.own[r], g, true);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPT; ++r)
        if (L.row_ok[r]) store_acc<T, VEC>(gx + ti.bc * HW + L.own[r], gxa[r], false);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int VEC, int RPT, int ROWS>
static size_t acc_lds(int S, size_t acc_bytes, int tiles) {
    return static_cast<size_t>(S) * sizeof(int4) +
           static_cast<size_t>(tiles) * Geo<VEC, RPT, ROWS>::TILE * acc_bytes;
}

constexpr size_t kLdsLimit = 80 * 1024;  // two workgroups per CU (160 KB LDS)

struct Dims {
    int S, B, C, H, W;
};

// Launch configuration: rows per lane, prefetch depth, tile order (0 row-
// major, 2 banded), whether weight loads are nontemporal, the band height in
// tile rows and the lane rows per workgroup (16, 32 or 64, i.e. 256, 512 or
// 1024 lanes).  The defaults were measured on MI355X;
// NSH_ACC_TUNE="rpt,p,order,nt,band,rows" overrides them for both passes.
struct Tune {
    int rpt = 1, p = 1, order = 2, nt = 0, band = 2, rows = 32;
};

static Tune tune_from_env() {
    static const Tune t = [] {
        Tune r;
        if (const char* e = getenv("NSH_ACC_TUNE")) {
            int a, b, c, d, f = 1, g = 16;
            const int n = sscanf(e, "%d,%d,%d,%d,%d,%d", &a, &b, &c, &d, &f, &g);
            if (n >= 4 && (a == 1 || a == 2 || a == 4) && (b == 1 || b == 2 || b == 4) &&
                (c == 0 || c == 2) && (d == 0 || d == 1) && f >= 1 && f <= 64 &&
                (g == 16 || g == 32 || g == 64)) {
                r.rpt = a;
                r.p = b;
                r.order = c;
                r.nt = d;
                r.band = f;
                r.rows = g;
            }
        }
        return r;
    }();
    return t;
}

template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL>
static int launch_fwd(const void* x, const void* w, const int64_t* shifts, Dims d, int order,
                      int band, void* U, void* Z, hipStream_t st) {
    using G = Geo<VEC, RPT, ROWS>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    const size_t lds = acc_lds<VEC, RPT, ROWS>(d.S, sizeof(acc_t<T>), 1);
    hipLaunchKernelGGL((accumulate_uz_fwd_kernel<T, VEC, RPT, ROWS, P, NTL>),
                       dim3(static_cast<unsigned>(tiles)), dim3(G::THREADS), lds, st, static_cast<const T*>(x),
                       static_cast<const T*>(w), shifts, d.S, d.C, d.H, d.W, ntw, nth, order, band, step,
                       static_cast<acc_t<T>*>(U), static_cast<acc_t<T>*>(Z));
    return nsh_host::check_launch("accumulate_uz_forward");
}

template <typename T, int VEC, int RPT, int ROWS, int P, bool NTL>
static int launch_bwd(const void* x, const void* w, const void* gU, const void* gZ,
                      const int64_t* shifts, Dims d, int order, int band, void* gx, void* gw,
                      hipStream_t st) {
    using G = Geo<VEC, RPT, ROWS>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    const size_t lds = acc_lds<VEC, RPT, ROWS>(d.S, sizeof(acc_t<T>), 3);
    hipLaunchKernelGGL((accumulate_uz_bwd_kernel<T, VEC, RPT, ROWS, P, NTL>),
                       dim3(static_cast<unsigned>(tiles)), dim3(G::THREADS), lds, st, static_cast<const T*>(x),
                       static_cast<const T*>(w), static_cast<const acc_t<T>*>(gU),
                       static_cast<const acc_t<T>*>(gZ), shifts, d.S, d.C, d.H, d.W, ntw, nth,
                       order, band, step, static_cast<T*>(gx), static_cast<T*>(gw));
    return nsh_host::check_launch("accumulate_uz_backward");
}

template <int VEC>
static size_t lds_need(int rpt, int rows, int S, size_t ab, bool bwd) {
    const int tiles = bwd ? 3 : 1;
    const int th = rpt * rows + 2 * kRmax;
    (void)acc_lds<VEC, 1, 16>;
    return static_cast<size_t>(S) * sizeof(int4) +
           static_cast<size_t>(tiles) * th * (Geo<VEC, 1, 16>::PITCH) * ab;
}

// Lanes needed to keep every CU busy: 256 CUs x 32 waves x 64 lanes.
constexpr int64_t kFillLanes = int64_t(1) << 19;

// Widest vector such that every row start is aligned for it, the launch
// still has about kFillLanes lanes (small images trade vector width for
// occupancy) and the LDS budget holds; VEC = 1 handles any shape.  Also
// settles rows per lane.
template <typename T>
static int pick_vec(int W, std::initializer_list<const void*> ptrs, int S, bool bwd, int* rpt,
                    int rows, int64_t pixels) {
    int maxv = 16 / static_cast<int>(sizeof(T));
    while (maxv > 1 && pixels / maxv < kFillLanes) maxv /= 2;
    const size_t ab = sizeof(acc_t<T>);
    for (int v = maxv; v >= 1; v /= 2) {
        if (W % v) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && nsh_host::aligned(p, v * sizeof(T));
        if (!ok) continue;
        for (int r = *rpt; r >= 1; r /= 2) {
            size_t lds = 0;
            switch (v) {
                case 8: lds = lds_need<8>(r, rows, S, ab, bwd); break;
                case 4: lds = lds_need<4>(r, rows, S, ab, bwd); break;
                case 2: lds = lds_need<2>(r, rows, S, ab, bwd); break;
                default: lds = lds_need<1>(r, rows, S, ab, bwd); break;
            }
            if (lds <= kLdsLimit) {
                *rpt = r;
                return v;
            }
        }
    }
    *rpt = 1;
    return 1;
}

// Dispatch over (RPT, ROWS, P, NT) for a fixed (T, VEC).  Configurations
// that are not instantiated fall back to the production one.
template <typename T, int VEC, bool BWD>
static int dispatch_cfg(const Tune& t, int rpt, const void* x, const void* w, const void* gU,
                        const void* gZ, const int64_t* sh, Dims d, void* o0, void* o1,
                        hipStream_t st) {
#define NSH_ACC_LAUNCH(R_, W_, P_, N_)                                                            \
    do {                                                                                          \
        if constexpr (BWD)                                                                        \
            return launch_bwd<T, VEC, R_, W_, P_, N_>(x, w, gU, gZ, sh, d, t.order, t.band, o0,   \
                                                      o1, st);                                    \
        else                                                                                      \
            return launch_fwd<T, VEC, R_, W_, P_, N_>(x, w, sh, d, t.order, t.band, o0, o1, st);  \
    } while (0)
#define NSH_ACC_CASE(R_, W_, P_, N_) \
    if (rpt == R_ && t.rows == W_ && t.p == P_ && t.nt == N_) NSH_ACC_LAUNCH(R_, W_, P_, N_);
    if constexpr (std::is_same<T, float>::value && VEC == 4) {
        // measured alternatives for the fp32 production shape
        NSH_ACC_CASE(1, 16, 2, false)
        NSH_ACC_CASE(2, 16, 1, false)
        NSH_ACC_CASE(2, 16, 2, false)
        NSH_ACC_CASE(1, 64, 1, false)
        NSH_ACC_CASE(2, 32, 1, false)
        NSH_ACC_CASE(1, 32, 2, false)
        NSH_ACC_CASE(1, 16, 1, true)
    }
#undef NSH_ACC_CASE
    if (t.rows == 16) NSH_ACC_LAUNCH(1, 16, 1, false);
    NSH_ACC_LAUNCH(1, 32, 1, false);
#undef NSH_ACC_LAUNCH
}

template <typename T, bool BWD>
static int run(const void* x, const void* w, const void* gU, const void* gZ, const int64_t* sh,
               Dims d, void* o0, void* o1, hipStream_t st) {
    const Tune t = tune_from_env();
    int rpt = t.rpt;
    const int64_t pixels = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    const int v = BWD ? pick_vec<T>(d.W, {x, w, gU, gZ, o0, o1}, d.S, true, &rpt, t.rows, pixels)
                      : pick_vec<T>(d.W, {x, w, o0, o1}, d.S, false, &rpt, t.rows, pixels);
    switch (v) {
        case 8: if constexpr (sizeof(T) == 2) return dispatch_cfg<T, 8, BWD>(t, rpt, x, w, gU, gZ, sh, d, o0, o1, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return dispatch_cfg<T, 4, BWD>(t, rpt, x, w, gU, gZ, sh, d, o0, o1, st); break;
        case 2: return dispatch_cfg<T, 2, BWD>(t, rpt, x, w, gU, gZ, sh, d, o0, o1, st);
        default: break;
    }
    return dispatch_cfg<T, 1, BWD>(t, rpt, x, w, gU, gZ, sh, d, o0, o1, st);
}

template <typename T>
static int run_fwd(const void* x, const void* w, const int64_t* shifts, Dims d, void* U, void* Z,
                   hipStream_t st) {
    return run<T, false>(x, w, nullptr, nullptr, shifts, d, U, Z, st);
}

template <typename T>
static int run_bwd(const void* x, const void* w, const void* gU, const void* gZ,
                   const int64_t* shifts, Dims d, void* gx, void* gw, hipStream_t st) {
    return run<T, true>(x, w, gU, gZ, shifts, d, gx, gw, st);
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
