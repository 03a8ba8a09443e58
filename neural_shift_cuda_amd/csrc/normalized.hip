// normalized.hip -- overflow-safe normalized accumulation D = K/C on gfx950.
//
// Semantics (reference GPU kernels csrc/shift_ops_cuda.cu:474-791):
//   terms i of pixel p: forward (w_s[p], x[(p+s) mod]) and, for has_inv rows
//   with box(p-s), mirror (w_s[p-s], x[p-s]).  Keys are the positive weights
//   (log_weights = 0) or the logits (log_weights = 1); w == 0 / l == -inf are
//   masks.  D = sum a_i v_i / sum a_i with a_i = w_i / max w or
//   exp(l_i - max l); log_C = log(max w) + log(sum a) or max l + log(sum a).
//   Empty rows give D = 0, log_C = -inf; a NaN / +inf key, or a negative
//   positive weight, gives NaN in both outputs.
//
// Forward: a single pass over the weight planes as an online softmax.  Each
// lane keeps (m, u, z) per pixel; a term with key k updates
//   k > m : u = u*r + v, z = z*r + 1, m = k      with r = rescale(m -> k)
//   k <= m: u += a v,    z += a                  with a = scale(k -> m)
// where both branches share one transcendental (log mode: exp(-|k - m|)) or
// one division (positive mode: min(k, m) / max(k, m)), so every term costs
// one exp or one divide and the weights are read from HBM exactly once.
//
// Backward (csrc/shift_ops_cuda.cu:655-791), one fused pass per tile:
//   f(v, L) = 0 if lw(v) == -inf or L == -inf else exp(lw(v) - L)
//   gx[q]   = sum_s f(w_s[o], L[o]) gD[o] at o = (q-s) mod
//           + [inv, box(q+s)] f(w_s[q], L[q+s]) gD[q+s]
//   gw_s[q] = 0 for a masked weight, else
//             F(L[q]) score(q, x[(q+s) mod]) + [inv, box(q+s)] F(L[q+s]) score(q+s, x[q])
//   score(o, v) = gD[o] (v - D[o]) + gLogC[o];  F = f (log mode) or exp(-L).
#include <initializer_list>

#include "nsh_common.hpp"

namespace nsh {

template <int VEC>
struct NGeo {
    static constexpr int TW = kTPR * VEC;
    static constexpr int TH = kRows;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
};

template <typename A> struct Lim;
template <> struct Lim<float> {
    static __device__ __forceinline__ float maxv() { return 3.4028234663852886e38f; }
    static __device__ __forceinline__ float inf() { return __builtin_inff(); }
    static __device__ __forceinline__ float nan() { return __builtin_nanf(""); }
    static __device__ __forceinline__ float ex(float v) { return ::expf(v); }
    static __device__ __forceinline__ float lg(float v) { return ::logf(v); }
};
template <> struct Lim<double> {
    static __device__ __forceinline__ double maxv() { return 1.7976931348623157e308; }
    static __device__ __forceinline__ double inf() { return __builtin_inf(); }
    static __device__ __forceinline__ double nan() { return __builtin_nan(""); }
    static __device__ __forceinline__ double ex(double v) { return ::exp(v); }
    static __device__ __forceinline__ double lg(double v) { return ::log(v); }
};

// Per-pixel online-softmax state.
template <typename A>
struct Online {
    A m, u, z;
    bool any, bad;
};

template <typename A, bool LOGW>
__device__ __forceinline__ void online_init(Online<A>& st) {
    st.m = LOGW ? -Lim<A>::maxv() : A(0);
    st.u = A(0);
    st.z = A(0);
    st.any = false;
    st.bad = false;
}

template <typename A, bool LOGW>
__device__ __forceinline__ void online_add(Online<A>& st, A k, A v) {
    bool valid;
    A r, a;
    bool gt;
    if (LOGW) {
        valid = k > -Lim<A>::inf() && k <= Lim<A>::maxv();
        st.bad |= (k != k) || (k > Lim<A>::maxv());  // NaN or +inf
        const A d = k - st.m;
        gt = d > A(0);
        const A t = Lim<A>::ex(-__builtin_fabs(d));
        r = gt ? t : A(1);
        a = gt ? A(1) : t;
    } else {
        valid = k > A(0) && k <= Lim<A>::maxv();
        st.bad |= !(k >= A(0)) || k > Lim<A>::maxv();  // negative, NaN or +inf
        gt = k > st.m;
        const A num = gt ? st.m : k;
        const A den = gt ? k : st.m;
        const A t = num / den;
        r = gt ? t : A(1);
        a = gt ? A(1) : t;
    }
    r = valid ? r : A(1);
    a = valid ? a : A(0);
    st.u = fma_acc(st.u, r, a * v);
    st.z = fma_acc(st.z, r, a);
    st.m = (valid && gt) ? k : st.m;
    st.any |= valid;
}

template <typename A, bool LOGW>
__device__ __forceinline__ void online_final(const Online<A>& st, A& D, A& L) {
    if (st.bad) {
        D = Lim<A>::nan();
        L = Lim<A>::nan();
    } else if (!st.any) {
        D = A(0);
        L = -Lim<A>::inf();
    } else {
        D = st.u / st.z;
        L = (LOGW ? st.m : Lim<A>::lg(st.m)) + Lim<A>::lg(st.z);
    }
}

__device__ __forceinline__ bool tile_inside_n(int h0, int w0, int TH, int TW, int H, int W, int dx,
                                              int dy) {
    const int h1 = (h0 + TH < H ? h0 + TH : H) - 1;
    const int w1 = (w0 + TW < W ? w0 + TW : W) - 1;
    return h0 + dx >= 0 && h1 + dx < H && w0 + dy >= 0 && w1 + dy < W;
}

template <typename T, int VEC, bool LOGW>
__global__ __launch_bounds__(kThreads) void normalized_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const int64_t* __restrict__ shifts, int S,
    int C, int H, int W, int ntw, int nth, int64_t plane_step, acc_t<T>* __restrict__ Dout,
    acc_t<T>* __restrict__ Lout) {
    using A = acc_t<T>;
    using G = NGeo<VEC>;
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
    const int lc = (ty + kRmax) * G::LW + tx * VEC + kRmax;
    const int64_t b = ti.bc / C;
    const int64_t c = ti.bc - b * C;
    const T* wp = w + (b * C + c) * HW;

    Online<A> st[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) online_init<A, LOGW>(st[k]);

    for (int s = 0; s < S; ++s, wp += plane_step) {
        const ShiftRec r = read_shift(shl, s);
        const bool lds = shift_in_lds(r);
        A wv[VEC], xv[VEC];
        load_acc<T, VEC>(wp + own, wv);
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
        for (int k = 0; k < VEC; ++k) online_add<A, LOGW>(st[k], wv[k], xv[k]);

        if (r.inv) {
            const int hs = h - r.dx;
            const bool rok = in_range(hs, H);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const int ws = w0 + k - r.dy;
                if (rok && in_range(ws, W)) {
                    const uint32_t src = static_cast<uint32_t>(hs) * W + ws;
                    const A wi = to_acc(wp[src]);
                    const A xi = lds ? xt[lc - r.dx * G::LW - r.dy + k] : to_acc(xp[src]);
                    online_add<A, LOGW>(st[k], wi, xi);
                }
            }
        }
    }
    A Dv[VEC], Lv[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) online_final<A, LOGW>(st[k], Dv[k], Lv[k]);
    store_out<A, VEC>(Dout + ti.bc * HW + own, Dv);
    store_out<A, VEC>(Lout + ti.bc * HW + own, Lv);
}

// lw(v): the log-weight of a key (positive mode: log v, -inf for 0, NaN < 0).
template <typename A, bool LOGW>
__device__ __forceinline__ A as_log(A v) {
    if (LOGW) return v;
    return v > A(0) ? Lim<A>::lg(v) : (v == A(0) ? -Lim<A>::inf() : Lim<A>::nan());
}

template <typename A>
__device__ __forceinline__ A frac(A lw, A L) {
    return (lw == -Lim<A>::inf() || L == -Lim<A>::inf()) ? A(0) : Lim<A>::ex(lw - L);
}

template <typename T, int VEC, bool LOGW>
__global__ __launch_bounds__(kThreads) void normalized_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const acc_t<T>* __restrict__ Dg,
    const acc_t<T>* __restrict__ Lg, const acc_t<T>* __restrict__ gDg,
    const acc_t<T>* __restrict__ gLg, const int64_t* __restrict__ shifts, int S, int C, int H,
    int W, int ntw, int nth, int64_t plane_step, T* __restrict__ gx, T* __restrict__ gw) {
    using A = acc_t<T>;
    using G = NGeo<VEC>;
    constexpr int LT = G::LH * G::LW;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + static_cast<size_t>(S) * sizeof(int4));
    A* dt = xt + LT;
    A* lt = dt + LT;
    A* gdt = lt + LT;
    A* glt = gdt + LT;

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;
    const A* Dp = Dg + ti.bc * HW;
    const A* Lp = Lg + ti.bc * HW;
    const A* gDp = gDg + ti.bc * HW;
    const A* gLp = gLg + ti.bc * HW;
    stage_shifts(shl, shifts, S, 3, H, W);
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(dt, Dp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(lt, Lp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(gdt, gDp, H, W, ti.h0, ti.w0, G::LH, G::LW);
    stage_tile_acc<A>(glt, gLp, H, W, ti.h0, ti.w0, G::LH, G::LW);
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

    A xo[VEC], Do[VEC], Lo[VEC], gDo[VEC], gLo[VEC], Eo[VEC], gxa[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        xo[k] = xt[lc + k];
        Do[k] = dt[lc + k];
        Lo[k] = lt[lc + k];
        gDo[k] = gdt[lc + k];
        gLo[k] = glt[lc + k];
        Eo[k] = Lim<A>::ex(-Lo[k]);
        gxa[k] = A(0);
    }

    for (int s = 0; s < S; ++s, wp += plane_step, gp += plane_step) {
        const ShiftRec r = read_shift(shl, s);
        const bool lds = shift_in_lds(r);
        // neighbour values at q + s (circular) and q - s (circular)
        A xf[VEC], Dp_[VEC], Lp_[VEC], gDp_[VEC], gLp_[VEC], Lm[VEC], gDm[VEC];
        if (lds) {
            const int op = lc + r.dx * G::LW + r.dy;
            const int om = lc - r.dx * G::LW - r.dy;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                xf[k] = xt[op + k];
                Dp_[k] = dt[op + k];
                Lp_[k] = lt[op + k];
                gDp_[k] = gdt[op + k];
                gLp_[k] = glt[op + k];
                Lm[k] = lt[om + k];
                gDm[k] = gdt[om + k];
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
                Dp_[k] = Dp[ip];
                Lp_[k] = Lp[ip];
                gDp_[k] = gDp[ip];
                gLp_[k] = gLp[ip];
                Lm[k] = Lp[im];
                gDm[k] = gDp[im];
            }
        }
        bool okp[VEC];
        {
            const bool rok = in_range(h + r.dx, H);
#pragma unroll
            for (int k = 0; k < VEC; ++k) okp[k] = r.inv && rok && in_range(w0 + k + r.dy, W);
        }

        A wv[VEC];
        load_acc<T, VEC>(wp + own, wv);
        A g[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const A lw = as_log<A, LOGW>(wv[k]);
            A Fi = A(0), si = A(0);
            if (okp[k]) {
                si = fma_acc(gDp_[k], xo[k] - Dp_[k], gLp_[k]);
                Fi = LOGW ? frac<A>(lw, Lp_[k]) : Lim<A>::ex(-Lp_[k]);
                // gx mirror term: f(w_s[q], L[q+s]) gD[q+s]
                gxa[k] = fma_acc(frac<A>(lw, Lp_[k]), gDp_[k], gxa[k]);
            }
            const A sf = fma_acc(gDo[k], xf[k] - Do[k], gLo[k]);
            const A Ff = LOGW ? frac<A>(lw, Lo[k]) : Eo[k];
            const A gv = fma_acc(Ff, sf, Fi * si);
            g[k] = (lw == -Lim<A>::inf()) ? A(0) : gv;
        }
        store_acc<T, VEC>(gp + own, g, true);

        // gx forward term at o = (q - s) mod
        A ws[VEC];
        if (tile_inside_n(ti.h0, ti.w0, G::TH, G::TW, H, W, -r.dx, -r.dy)) {
            const int off = -(r.dx * W + r.dy);
#pragma unroll
            for (int k = 0; k < VEC; ++k) ws[k] = to_acc(wp[static_cast<int64_t>(own) + off + k]);
        } else {
            int hm = h - r.dxm;
            hm += hm < 0 ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int wm = w0 + k - r.dym;
                wm += wm < 0 ? W : 0;
                ws[k] = to_acc(wp[static_cast<uint32_t>(hm) * W + wm]);
            }
        }
#pragma unroll
        for (int k = 0; k < VEC; ++k)
            gxa[k] = fma_acc(frac<A>(as_log<A, LOGW>(ws[k]), Lm[k]), gDm[k], gxa[k]);
    }
    store_acc<T, VEC>(gx + ti.bc * HW + own, gxa, false);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr size_t kNLdsLimit = 64 * 1024;

template <int VEC>
static size_t nfwd_lds(int S, size_t ab) {
    return static_cast<size_t>(S) * sizeof(int4) + static_cast<size_t>(NGeo<VEC>::LH) * NGeo<VEC>::LW * ab;
}
template <int VEC>
static size_t nbwd_lds(int S, size_t ab) {
    return static_cast<size_t>(S) * sizeof(int4) + 5 * static_cast<size_t>(NGeo<VEC>::LH) * NGeo<VEC>::LW * ab;
}

template <typename T>
static size_t n_lds(int v, int S, bool bwd) {
    const size_t ab = sizeof(acc_t<T>);
    switch (v) {
        case 8: return bwd ? nbwd_lds<8>(S, ab) : nfwd_lds<8>(S, ab);
        case 4: return bwd ? nbwd_lds<4>(S, ab) : nfwd_lds<4>(S, ab);
        case 2: return bwd ? nbwd_lds<2>(S, ab) : nfwd_lds<2>(S, ab);
        default: return bwd ? nbwd_lds<1>(S, ab) : nfwd_lds<1>(S, ab);
    }
}

template <typename T>
static int n_pick_vec(int W, std::initializer_list<const void*> ptrs, int S, bool bwd) {
    for (int v = 16 / static_cast<int>(sizeof(T)); v > 1; v /= 2) {
        if (W % v) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && nsh_host::aligned(p, v * sizeof(T));
        if (ok && n_lds<T>(v, S, bwd) <= kNLdsLimit) return v;
    }
    return 1;
}

struct NDims {
    int S, B, C, H, W;
};

template <typename T, int VEC, bool LOGW>
static int n_launch_fwd(const void* x, const void* w, const int64_t* sh, NDims d, void* D, void* L,
                        hipStream_t st) {
    using G = NGeo<VEC>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    hipLaunchKernelGGL((normalized_fwd_kernel<T, VEC, LOGW>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), n_lds<T>(VEC, d.S, false), st, static_cast<const T*>(x),
                       static_cast<const T*>(w), sh, d.S, d.C, d.H, d.W, ntw, nth, step,
                       static_cast<acc_t<T>*>(D), static_cast<acc_t<T>*>(L));
    return nsh_host::check_launch("normalized_accumulate_uz_forward");
}

template <typename T, int VEC, bool LOGW>
static int n_launch_bwd(const void* x, const void* w, const void* D, const void* L, const void* gD,
                        const void* gL, const int64_t* sh, NDims d, void* gx, void* gw,
                        hipStream_t st) {
    using G = NGeo<VEC>;
    using A = acc_t<T>;
    const int ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    const int64_t tiles = static_cast<int64_t>(d.B) * d.C * ntw * nth;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    hipLaunchKernelGGL((normalized_bwd_kernel<T, VEC, LOGW>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kThreads), n_lds<T>(VEC, d.S, true), st, static_cast<const T*>(x),
                       static_cast<const T*>(w), static_cast<const A*>(D), static_cast<const A*>(L),
                       static_cast<const A*>(gD), static_cast<const A*>(gL), sh, d.S, d.C, d.H, d.W,
                       ntw, nth, step, static_cast<T*>(gx), static_cast<T*>(gw));
    return nsh_host::check_launch("normalized_accumulate_uz_backward");
}

template <typename T, bool LOGW>
static int n_run_fwd(const void* x, const void* w, const int64_t* sh, NDims d, void* D, void* L,
                     hipStream_t st) {
    switch (n_pick_vec<T>(d.W, {x, w, D, L}, d.S, false)) {
        case 8: if constexpr (sizeof(T) == 2) return n_launch_fwd<T, 8, LOGW>(x, w, sh, d, D, L, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return n_launch_fwd<T, 4, LOGW>(x, w, sh, d, D, L, st); break;
        case 2: return n_launch_fwd<T, 2, LOGW>(x, w, sh, d, D, L, st);
        default: break;
    }
    return n_launch_fwd<T, 1, LOGW>(x, w, sh, d, D, L, st);
}

template <typename T, bool LOGW>
static int n_run_bwd(const void* x, const void* w, const void* D, const void* L, const void* gD,
                     const void* gL, const int64_t* sh, NDims d, void* gx, void* gw, hipStream_t st) {
    switch (n_pick_vec<T>(d.W, {x, w, D, L, gD, gL, gx, gw}, d.S, true)) {
        case 8: if constexpr (sizeof(T) == 2) return n_launch_bwd<T, 8, LOGW>(x, w, D, L, gD, gL, sh, d, gx, gw, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return n_launch_bwd<T, 4, LOGW>(x, w, D, L, gD, gL, sh, d, gx, gw, st); break;
        case 2: return n_launch_bwd<T, 2, LOGW>(x, w, D, L, gD, gL, sh, d, gx, gw, st);
        default: break;
    }
    return n_launch_bwd<T, 1, LOGW>(x, w, D, L, gD, gL, sh, d, gx, gw, st);
}

}  // namespace nsh

using nsh_host::fail;

static int n_check(const char* op, int64_t S, int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                   nsh::NDims* d) {
    if (S < 1 || S > 1024)
        return fail(NSH_ERR_INVALID, "%s: tree reduction requires 1 <= S <= 1024", op);
    if (B < 1 || C < 1 || H < 1 || W < 1)
        return fail(NSH_ERR_INVALID, "%s: empty tensor", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (B * C > (int64_t(1) << 24)) return fail(NSH_ERR_INVALID, "%s: B*C too large", op);
    *d = nsh::NDims{static_cast<int>(S), static_cast<int>(B), static_cast<int>(C),
                    static_cast<int>(H), static_cast<int>(W)};
    return NSH_OK;
}

#define NSH_DISPATCH_LOGW(T, FN, ...)                                   \
    (log_weights ? nsh::FN<T, true>(__VA_ARGS__) : nsh::FN<T, false>(__VA_ARGS__))

extern "C" int nsh_normalized_accumulate_uz_forward(const void* x, const void* weights,
                                                    const int64_t* shifts, int64_t S, int64_t B,
                                                    int64_t C, int64_t H, int64_t W, int dtype,
                                                    int log_weights, void* D, void* log_C,
                                                    void* stream) {
    nsh::NDims d;
    if (int rc = n_check("normalized_accumulate_uz", S, B, C, H, W, dtype, &d)) return rc;
    if (!x || !weights || !shifts || !D || !log_C)
        return fail(NSH_ERR_INVALID, "normalized_accumulate_uz: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return NSH_DISPATCH_LOGW(nsh::f16, n_run_fwd, x, weights, shifts, d, D, log_C, st);
        case NSH_DTYPE_BFLOAT16: return NSH_DISPATCH_LOGW(nsh::bf16, n_run_fwd, x, weights, shifts, d, D, log_C, st);
        case NSH_DTYPE_FLOAT32: return NSH_DISPATCH_LOGW(float, n_run_fwd, x, weights, shifts, d, D, log_C, st);
        default: return NSH_DISPATCH_LOGW(double, n_run_fwd, x, weights, shifts, d, D, log_C, st);
    }
}

extern "C" int nsh_normalized_accumulate_uz_backward(const void* x, const void* weights,
                                                     const void* D, const void* log_C,
                                                     const void* grad_D, const void* grad_log_C,
                                                     const int64_t* shifts, int64_t S, int64_t B,
                                                     int64_t C, int64_t H, int64_t W, int dtype,
                                                     int log_weights, void* grad_x, void* grad_w,
                                                     void* stream) {
    nsh::NDims d;
    if (int rc = n_check("normalized_accumulate_uz_backward", S, B, C, H, W, dtype, &d)) return rc;
    if (!x || !weights || !D || !log_C || !grad_D || !grad_log_C || !shifts || !grad_x || !grad_w)
        return fail(NSH_ERR_INVALID, "normalized_accumulate_uz_backward: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            return NSH_DISPATCH_LOGW(nsh::f16, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, st);
        case NSH_DTYPE_BFLOAT16:
            return NSH_DISPATCH_LOGW(nsh::bf16, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, st);
        case NSH_DTYPE_FLOAT32:
            return NSH_DISPATCH_LOGW(float, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, st);
        default:
            return NSH_DISPATCH_LOGW(double, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, st);
    }
}
