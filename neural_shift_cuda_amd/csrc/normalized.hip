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
#include <cstdlib>
#include <initializer_list>

#include <type_traits>

#include "nsh_common.hpp"
#include "scatter.hpp"

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

// Masked key: a term that changes no state.
template <typename A, bool LOGW>
__device__ __forceinline__ A masked_key() {
    return LOGW ? -Lim<A>::inf() : A(0);
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
    int codes, int C, int H, int W, int ntw, int nth, int64_t plane_step,
    acc_t<T>* __restrict__ Dout, acc_t<T>* __restrict__ Lout) {
    using A = acc_t<T>;
    using G = NGeo<VEC>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const T* xp = x + ti.bc * HW;
    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
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
    const bool wsh = (codes & kCodesSharedW) != 0;
    const T* wp = w + weight_plane(b, c, C, wsh) * HW;
    const int64_t wstep = weight_step(plane_step, C, wsh);

    Online<A> st[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) online_init<A, LOGW>(st[k]);

    for (int s = 0; s < S; ++s, wp += wstep) {
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
        for (int k = 0; k < VEC; ++k)
            online_add<A, LOGW>(st[k], fwd_kept(r, h, w0 + k, H, W) ? wv[k]
                                                                    : masked_key<A, LOGW>(),
                                xv[k]);

        if (r.inv) {
            // source (h - dx, w - dy), wrapped for a circular mirror
            const bool rok = r.per || in_range(h - r.dx, H);
            int hs = h - r.dxm;
            hs += hs < 0 ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                if (rok && (r.per || in_range(w0 + k - r.dy, W))) {
                    int ws = w0 + k - r.dym;
                    ws += ws < 0 ? W : 0;
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
    const acc_t<T>* __restrict__ gLg, const int64_t* __restrict__ shifts, int S, int codes, int C,
    int H, int W, int ntw, int nth, int64_t plane_step, T* __restrict__ gx, T* __restrict__ gw) {
    using A = acc_t<T>;
    using G = NGeo<VEC>;
    constexpr int LT = G::LH * G::LW;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
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
    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
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
    const bool wsh = (codes & kCodesSharedW) != 0;
    const T* wp = w + weight_plane(b, c, C, wsh) * HW;
    const int64_t wstep = weight_step(plane_step, C, wsh);
    T* gp = gw + (b * C + c) * HW;  // the gradient has every channel

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

    for (int s = 0; s < S; ++s, wp += wstep, gp += plane_step) {
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
            const bool rok = r.per || in_range(h + r.dx, H);
#pragma unroll
            for (int k = 0; k < VEC; ++k)
                okp[k] = r.inv && rok && (r.per || in_range(w0 + k + r.dy, W));
        }

        A wv[VEC];
        load_acc<T, VEC>(wp + own, wv);
        A g[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            // forward box: a dropped w_s[q] acts as a masked key
            const A lw = fwd_kept(r, h, w0 + k, H, W) ? as_log<A, LOGW>(wv[k]) : -Lim<A>::inf();
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
        for (int k = 0; k < VEC; ++k) {
            const A lw = fwd_kept_src(r, h, w0 + k, H, W) ? as_log<A, LOGW>(ws[k]) : -Lim<A>::inf();
            gxa[k] = fma_acc(frac<A>(lw, Lm[k]), gDm[k], gxa[k]);
        }
    }
    store_acc<T, VEC>(gx + ti.bc * HW + own, gxa, false);
}

// ---------------------------------------------------------------------------
// Scatter form: every weight element is read once, aligned.
//
// The kernels above gather the mirror term of pixel p from w_s[p - s] (and,
// in the backward, the x-gradient term from w_s[(q - s) mod]): reads R rows /
// columns into the neighbouring tile, mostly missed in L2.  The scatter
// kernels below use the lane owning q, which holds w_s[q], for every term
// that weight enters:
//   forward : the mirror term (w_s[q], x[q]) of p = q + s is merged into an
//             LDS window of online-softmax states (m, u, z) at q + s.  The
//             merge of two states is associative, so the window, its border
//             spilled to the workspace, and the lane's own register state
//             combine in any fixed order; normalized_fixup_kernel merges the
//             neighbours' spills into the pixels near a tile edge (whose
//             partial states the main kernel leaves in the workspace) and
//             finishes D and log_C.  A state carries "no valid term" as
//             z == 0 and "bad key" as z = NaN.
//   backward: f(w_s[q], L[q]) gD[q], the x-gradient term of q + s, is added
//             into an LDS window at q + s (circular), as accumulate_uz's
//             backward does; spill_fixup_kernel adds the window borders.
//             Positive weights use E = exp(-L) staged per pixel:
//             f(w, L) = w E, so no transcendental per term.
// Shifts beyond the LDS halo take the gather form in a second loop, so the
// prefetch ring loop issues no conditional loads.  Lane ownership is
// strided (SGeo): LDS accesses are free of bank conflicts.
// ---------------------------------------------------------------------------

// Per-term arithmetic of the scatter kernels.  fp32 uses the hardware exp2
// (v_exp_f32) on x log2(e); its relative error grows like |x| 2^-24, which
// only matters for terms below exp(-87) that fp32 flushes anyway.  fp64
// keeps the library exp.
template <typename A> struct NMath;
template <> struct NMath<float> {
    static __device__ __forceinline__ float ex(float v) {
        return __builtin_amdgcn_exp2f(v * 1.44269504088896341f);
    }
    static __device__ __forceinline__ int fexp(float v) { return __builtin_amdgcn_frexp_expf(v); }
    static __device__ __forceinline__ float ldx(float v, int e) {
        return __builtin_amdgcn_ldexpf(v, e);
    }
};
template <> struct NMath<double> {
    static __device__ __forceinline__ double ex(double v) { return ::exp(v); }
    static __device__ __forceinline__ int fexp(double v) { return __builtin_amdgcn_frexp_exp(v); }
    static __device__ __forceinline__ double ldx(double v, int e) {
        return __builtin_amdgcn_ldexp(v, e);
    }
};

// Online-softmax state (m, u, z): u = sum a_i v_i and z = sum a_i over the
// terms seen so far, with a_i = exp(l_i - m), m the largest logit (log
// weights), or a_i = w_i 2^-m, m the binary exponent of the largest weight
// (positive weights: power-of-two scaling is exact and needs no divide; the
// largest term has a >= 1/2, so z cannot overflow).  z == 0: no valid
// term; z = NaN: a bad key (NaN / +inf logit; negative, NaN or +inf weight).
// Initial state: (empty_m, 0, 0).
template <typename A, bool LOGW>
__device__ __forceinline__ A empty_m() {
    // below every binary exponent of a nonzero value (fp32 >= -148, fp64 >= -1073)
    return LOGW ? -Lim<A>::maxv() : A(sizeof(A) == 8 ? -2000 : -1000);
}

template <typename A, bool LOGW>
__device__ __forceinline__ void term_add(A& m, A& u, A& z, A k, A v) {
    using M = NMath<A>;
    if (LOGW) {
        // -inf (mask) changes nothing below.  A NaN key makes a and hence u
        // and z NaN.  A +inf key (bad) sets m = +inf: every later key or
        // merge then forms exp(inf - inf) = NaN, and state_final reports a
        // state still at m = +inf as NaN, so no per-term test is needed.
        const A d = k - m;
        const bool gt = d > A(0);
        const A t = M::ex(-__builtin_fabs(d));
        const A r = gt ? t : A(1);
        const A a = gt ? A(1) : t;
        u = fma_acc(u, r, a * v);
        z = fma_acc(z, r, a);
        m = gt ? k : m;
    } else {
        const bool bad = !(k >= A(0)) || k > Lim<A>::maxv();
        const int me = static_cast<int>(m);
        const int e = k > A(0) ? M::fexp(k) : static_cast<int>(empty_m<A, false>());
        const int dd = me - e < 0 ? me - e : 0;  // rescale when the maximum grows
        const int mn = me > e ? me : e;
        const A a = M::ldx(k, -mn);
        u = fma_acc(a, v, M::ldx(u, dd));
        z = M::ldx(z, dd) + a;
        z = bad ? Lim<A>::nan() : z;
        m = static_cast<A>(mn);
    }
}

// term_add with a lazy reference point.  m need not be the largest key: a
// term may weigh up to e^kLazyLog (log weights) or 2^kLazyExp (positive
// weights) relative to m, and m moves (u and z rescaled) only when a key
// exceeds that, in practice at a state's first term.  The common term is
// then one exp (or one ldexp), one compare and two adds, and the rare one
// takes a branch that a wave skips when none of its lanes needs it.  Any
// (m, u, z) with a = weight relative to m is a valid state for term_add,
// state_merge and state_final, so the two forms mix freely.  Range: u and z
// stay below 2^11 (at most 2048 terms) times e^16 resp. 2^24 (times max |v|
// for u), far inside the accumulator range for image values.
constexpr float kLazyLog = 16.0f;
constexpr int kLazyExp = 24;

template <typename A>
__device__ __forceinline__ bool below_lazy_bound(A a) {
    // a in [+0, 2^kLazyExp): one unsigned compare of the bit pattern (a
    // negative value, -0, NaN and +inf all compare above the bound)
    if constexpr (sizeof(A) == 4)
        return __float_as_uint(a) < __float_as_uint(static_cast<float>(1 << kLazyExp));
    else
        return static_cast<uint64_t>(__double_as_longlong(a)) <
               static_cast<uint64_t>(__double_as_longlong(static_cast<double>(1 << kLazyExp)));
}

template <typename A, bool LOGW>
__device__ __forceinline__ void term_add_lazy(A& m, A& u, A& z, A k, A v) {
    using M = NMath<A>;
    if (LOGW) {
        // k - m > bound: move m to k (also for a +inf key, whose a is then
        // exp(inf - inf) = NaN: bad).  A NaN key gives a = NaN, a -inf
        // (masked) key a = 0.  The empty state (m = -maxv) takes the branch
        // with any finite key and rescales its zeros.
        if (__builtin_expect(k - m > A(kLazyLog), 0)) {
            const A r = M::ex(m - k);
            u *= r;
            z *= r;
            m = k;
        }
        const A a = M::ex(k - m);
        u = fma_acc(a, v, u);
        z += a;
    } else {
        const A a = M::ldx(k, -static_cast<int>(m));
        if (__builtin_expect(below_lazy_bound(a), 1)) {
            u = fma_acc(a, v, u);
            z += a;
        } else {
            // a bad key (negative, NaN, +inf) or one far above 2^m: the
            // exact update (it moves m to the key's exponent, or sets NaN)
            term_add<A, false>(m, u, z, k, v);
        }
    }
}

// term_add_lazy for the VEC pixels of a lane at once: the rare rescale is
// one branch for all of them (taken by a wave when any lane needs it), not
// one per pixel; the same arithmetic per pixel as term_add_lazy.
template <typename A, bool LOGW, int VEC>
__device__ __forceinline__ void terms_add_lazy(A (&m)[VEC], A (&u)[VEC], A (&z)[VEC],
                                               const A (&k)[VEC], const A (&v)[VEC]) {
    using M = NMath<A>;
    if constexpr (LOGW) {
        bool far = false;
#pragma unroll
        for (int i = 0; i < VEC; ++i) far |= k[i] - m[i] > A(kLazyLog);
        if (__builtin_expect(far, 0)) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                if (k[i] - m[i] > A(kLazyLog)) {
                    const A r = M::ex(m[i] - k[i]);
                    u[i] *= r;
                    z[i] *= r;
                    m[i] = k[i];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            const A a = M::ex(k[i] - m[i]);
            u[i] = fma_acc(a, v[i], u[i]);
            z[i] += a;
        }
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) term_add_lazy<A, false>(m[i], u[i], z[i], k[i], v[i]);
    }
}

// (m, u, z) := (m, u, z) merged with (m2, u2, z2).
template <typename A, bool LOGW>
__device__ __forceinline__ void state_merge(A& m, A& u, A& z, A m2, A u2, A z2) {
    using M = NMath<A>;
    if (LOGW) {
        const bool e1 = z == A(0), e2 = z2 == A(0);  // NaN (bad) is not empty
        const A mm = e1 ? m2 : (e2 ? m : (m > m2 ? m : m2));
        const A r1 = e1 ? A(0) : M::ex(m - mm);
        const A r2 = e2 ? A(0) : M::ex(m2 - mm);
        u = u * r1 + u2 * r2;
        z = z * r1 + z2 * r2;
        m = mm;
    } else {
        const int e1 = static_cast<int>(m), e2 = static_cast<int>(m2);
        const int mm = e1 > e2 ? e1 : e2;
        u = M::ldx(u, e1 - mm) + M::ldx(u2, e2 - mm);
        z = M::ldx(z, e1 - mm) + M::ldx(z2, e2 - mm);
        m = static_cast<A>(mm);
    }
}

template <typename A, bool LOGW>
__device__ __forceinline__ void state_final(A m, A u, A z, A& D, A& L) {
    if (z != z || (LOGW && m == Lim<A>::inf())) {  // bad key (NaN, or a +inf logit)
        D = Lim<A>::nan();
        L = Lim<A>::nan();
    } else if (z == A(0)) {
        D = A(0);
        L = -Lim<A>::inf();
    } else {
        D = u / z;
        // log C = m + log z, or (binary exponent m) m ln 2 + log z
        L = (LOGW ? m : m * A(0.693147180559945309)) + Lim<A>::lg(z);
    }
}

// Largest max(|dx|, |dy|) over the rows (only has_inverse rows when
// `only_inv`) that stay within the LDS halo; uniform across the workgroup.
template <int HALO = kRmax>
__device__ __forceinline__ int near_radius(const int4* shl, int S, bool only_inv) {
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

// Nontemporal weight loads: the fp64 forward 4-7% faster (c3 0.090 ->
// 0.085-0.087 ms), the fp32 backward on its 128-wide tiles 3% (c3 positive
// 0.642 -> 0.621 ms), the fp32 forward on 128-wide tiles 2% (on 64-wide
// tiles 13% slower: c3 0.326 -> 0.368 ms); the 16-bit forward 2% slower,
// the fp16 and fp64 backwards within the run-to-run spread (+-2%).  So:
// nontemporal in the fp32 and fp64 forwards and the fp32 backward.
template <typename T>
constexpr bool kNormFwdNT = sizeof(T) >= 4;
template <typename T>
constexpr bool kNormBwdNT = sizeof(T) == 4;
// The weight of pixel p for channel c from NH head planes: NH = 1 reads the
// plane as it is; NH > 1 forms sum_j mix[c][j] w_j[p] (the head-mixing
// product of the attention installers, applied where the weights are
// consumed, so no (S, B, C, H, W) stack is written and read).
template <typename T, int VEC, int NH, typename A>
__device__ __forceinline__ void mixed_pixels(PixSlot<T, VEC> (&slot)[NH], const A (&mixc)[NH],
                                             A (&wv)[VEC]) {
    slot_get_pixels<T, VEC>(slot[0], wv);
    if constexpr (NH > 1) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) wv[k] *= mixc[0];
#pragma unroll
        for (int j = 1; j < NH; ++j) {
            A t[VEC];
            slot_get_pixels<T, VEC>(slot[j], t);
#pragma unroll
            for (int k = 0; k < VEC; ++k) wv[k] = fma_acc(mixc[j], t[k], wv[k]);
        }
    }
}

// NH > 1: w is the head stack (S*B, NH, H, W), plane_step = B * NH * H * W,
// and mix the (C, NH) mixing matrix in the accumulator type.
template <typename T, int VEC, int TPR, int ROWS, int D, bool LOGW,
          int WPE = kScatterWavesPerEU<TPR * ROWS>, int NH = 1>
__global__ __launch_bounds__(TPR * ROWS, WPE) void
normalized_fwd_scatter_kernel(const T* __restrict__ x, const T* __restrict__ w,
                              const int64_t* __restrict__ shifts, int S, int codes, int C, int H,
                              int W, int ntw, int nth, int64_t plane_step, acc_t<T>* __restrict__ Dout,
                              acc_t<T>* __restrict__ Lout, int* __restrict__ hdr,
                              acc_t<T>* __restrict__ spill, acc_t<T>* __restrict__ part,
                              int ring_stride, int64_t ntiles,
                              const acc_t<T>* __restrict__ mix) {
    using A = acc_t<T>;
    using G = SGeo<VEC, ROWS, TPR>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* wm = xt + G::TILE;  // window of states (m, u, z)
    A* wu = wm + G::TILE;
    A* wz = wu + G::TILE;

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t off = ti.bc * HW;
    const T* xp = x + off;
    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    const int R = near_radius(shl, S, true);
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr[0] = R;  // for the fix-up
    const A m0 = empty_m<A, LOGW>();
    // the window is also used at R = 0 by a (0, 0) mirror row
    for (int i = threadIdx.x; i < G::TILE; i += blockDim.x) {
        wm[i] = m0;
        wu[i] = A(0);
        wz[i] = A(0);
    }
    __syncthreads();

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + kRmax) * G::PITCH + tx + kRmax;  // pixel k at lc + k*TPR
    const int64_t b = ti.bc / C;
    const int64_t ch = ti.bc - b * C;
    const bool wsh = (codes & kCodesSharedW) != 0;
    // shift s adds s * wstep; head j of a mixed stack sits j planes further
    const T* w_bc = NH > 1 ? w + b * NH * HW : w + weight_plane(b, ch, C, wsh) * HW;
    const int64_t wstep = NH > 1 ? plane_step : weight_step(plane_step, C, wsh);
    A mixc[NH];
#pragma unroll
    for (int j = 0; j < NH; ++j) mixc[j] = NH > 1 ? mix[ch * NH + j] : A(1);

    A xo[VEC], sm[VEC], su[VEC], sz[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        xo[k] = xt[lc + k * TPR];
        sm[k] = m0;
        su[k] = A(0);
        sz[k] = A(0);
    }
    // Weight prefetch ring (raw slots, promoted where consumed); the plane
    // of the next refill advances one plane per shift and the next shift's
    // record is read one shift ahead.
    PixSlot<T, VEC> wb[D][NH];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int j = 0; j < NH; ++j)
            slot_load_pixels<T, VEC, TPR, kNormFwdNT<T>>(
                w_bc + j * HW + static_cast<int64_t>(min(d, S - 1)) * wstep, px, wb[d][j]);
    const T* wr = w_bc + static_cast<int64_t>(min(D, S - 1)) * wstep;
    ShiftRec rn = read_shift(shl, 0);

    // Interior tiles (every pixel inside the image and every q + s inside
    // it for all rows of the table) need no forward-box test and no mirror
    // mask: they run a select-free copy of the loop.
    const int R_all = table_radius(shl, S, false);
    const bool interior = ti.h0 >= R_all && ti.h0 + G::TH + R_all <= H && ti.w0 >= R_all &&
                          ti.w0 + G::TW + R_all <= W;
    int last_dx = kClamp;
    // MODE 0: interior tile; 1: masks; 2: masks and forward-box rows
    auto step = [&](int s, PixSlot<T, VEC> (&slot)[NH], auto mode_tag) {
        constexpr int MODE = decltype(mode_tag)::value;
        const ShiftRec rc = rn;
        rn = read_shift(shl, min(s + 1, S - 1));
        A wv[VEC];
        mixed_pixels<T, VEC, NH, A>(slot, mixc, wv);
#pragma unroll
        for (int j = 0; j < NH; ++j)
            slot_load_pixels<T, VEC, TPR, kNormFwdNT<T>>(wr + j * HW, px, slot[j]);
        wr += s + D + 1 < S ? wstep : 0;
        if (shift_in_lds(rc)) {
            const int op = lc + rc.dx * G::PITCH + rc.dy;  // window index of q + s
            if constexpr (MODE == 2) {
                // Forward box: a w_s[q] whose q + s leaves the image is a
                // masked key.  Only tiles this shift carries past the edge
                // test pixels.
                bool kept[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) kept[k] = true;
                if (rc.fbox && !tile_inside_n(ti.h0, ti.w0, G::TH, G::TW, H, W, rc.dx, rc.dy)) {
                    const bool frow = in_range(h + rc.dx, H);
#pragma unroll
                    for (int k = 0; k < VEC; ++k)
                        kept[k] = frow && in_range(ti.w0 + tx + k * TPR + rc.dy, W);
                }
#pragma unroll
                for (int k = 0; k < VEC; ++k) wv[k] = kept[k] ? wv[k] : masked_key<A, LOGW>();
            }
            {
                A xv[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) xv[k] = xt[op + k * TPR];
                terms_add_lazy<A, LOGW, VEC>(sm, su, sz, wv, xv);
            }
            if (rc.inv) {
                // Same dx: the wave's targets are its own rows shifted by dx,
                // disjoint from every other wave's; barrier only on a new dx.
                // Every lane merges (a masked key for a pixel outside the
                // image or a target outside the box changes nothing).  The
                // lane's VEC window states are read before any is written
                // (one LDS round trip per shift, not one per pixel).
                if (rc.dx != last_dx) {
                    lds_barrier();
                    last_dx = rc.dx;
                }
                const bool rok = rc.per || in_range(h + rc.dx, H);
                A m[VEC], u[VEC], z[VEC], kk[VEC], vv[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const int i = op + k * TPR;
                    m[k] = wm[i];
                    u[k] = wu[i];
                    z[k] = wz[i];
                    if constexpr (MODE == 0) {
                        kk[k] = wv[k];
                        vv[k] = xo[k];
                    } else {
                        const bool ok = px.act[k] && rok &&
                                        (rc.per || in_range(ti.w0 + tx + k * TPR + rc.dy, W));
                        kk[k] = ok ? wv[k] : masked_key<A, LOGW>();
                        vv[k] = ok ? xo[k] : A(0);
                    }
                }
                terms_add_lazy<A, LOGW, VEC>(m, u, z, kk, vv);
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const int i = op + k * TPR;
                    wm[i] = m[k];
                    wu[i] = u[k];
                    wz[i] = z[k];
                }
            }
        }
    };
    auto ring = [&](auto mode_tag) {
        const int S_ring = S - S % D;
        for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) step(s0 + d, wb[d], mode_tag);
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (S_ring + d < S) step(S_ring + d, wb[d], mode_tag);
    };
    if (interior)
        ring(std::integral_constant<int, 0>{});
    else if (table_any_fbox(shl, S))
        ring(std::integral_constant<int, 2>{});
    else
        ring(std::integral_constant<int, 1>{});
    // Shifts beyond the halo: gather form (forward x and mirror terms read
    // from HBM), kept out of the ring loop.
    auto weight_at = [&](const T* wp, uint32_t i) {
        A v = to_acc(wp[i]);
        if constexpr (NH > 1) {
            v *= mixc[0];
#pragma unroll
            for (int j = 1; j < NH; ++j) v = fma_acc(mixc[j], to_acc(wp[j * HW + i]), v);
        }
        return v;
    };
    for (int s = 0; s < S && px.any; ++s) {
        const ShiftRec rc = read_shift(shl, s);
        if (shift_in_lds(rc)) continue;
        const T* wp = w_bc + static_cast<int64_t>(s) * wstep;
        int hp = h + rc.dxm;
        hp -= hp >= H ? H : 0;
        int hm = h - rc.dxm;
        hm += hm < 0 ? H : 0;
        const bool irow = rc.per || in_range(h - rc.dx, H);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            if (!px.act[k]) continue;
            const int wq = ti.w0 + tx + k * TPR;
            int wj = wq + rc.dym;
            wj -= wj >= W ? W : 0;
            const A wq_ = weight_at(wp, px.own[k]);
            term_add<A, LOGW>(sm[k], su[k], sz[k],
                              fwd_kept(rc, h, wq, H, W) ? wq_ : masked_key<A, LOGW>(),
                              to_acc(xp[static_cast<uint32_t>(hp) * W + wj]));
            if (rc.inv && irow && (rc.per || in_range(wq - rc.dy, W))) {
                int wm_ = wq - rc.dym;
                wm_ += wm_ < 0 ? W : 0;
                const uint32_t src = static_cast<uint32_t>(hm) * W + wm_;
                term_add<A, LOGW>(sm[k], su[k], sz[k], weight_at(wp, src), to_acc(xp[src]));
            }
        }
    }

    __syncthreads();
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    A* pm = part + 3 * t * ring_stride;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!px.act[k]) continue;
        const int i = lc + k * TPR;
        state_merge<A, LOGW>(sm[k], su[k], sz[k], wm[i], wu[i], wz[i]);
        if (R > 0) {
            const int slot = ring_slot(ty, tx + k * TPR, th, tw, R);
            if (slot >= 0) {  // finished by the fix-up
                pm[slot] = sm[k];
                pm[ring_stride + slot] = su[k];
                pm[2 * ring_stride + slot] = sz[k];
                continue;
            }
        }
        A Dv, Lv;
        state_final<A, LOGW>(sm[k], su[k], sz[k], Dv, Lv);
        Dout[off + px.own[k]] = Dv;
        Lout[off + px.own[k]] = Lv;
    }
    if (R == 0) return;
    const int n = spill_count(th, tw, R);
    A* s0p = spill + t * G::SPILL;
    A* s1p = spill + (ntiles + t) * G::SPILL;
    A* s2p = spill + (2 * ntiles + t) * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        const int li = (i + kRmax) * G::PITCH + j + kRmax;
        s0p[e] = wm[li];
        s1p[e] = wu[li];
        s2p[e] = wz[li];
    }
}

// Finishes the ring pixels of the forward: own partial state merged with
// the neighbouring tiles' spilled window states (fixed order), then D and
// log_C.
template <typename A, bool LOGW>
__global__ __launch_bounds__(256) void normalized_fixup_kernel(
    int H, int W, int TH, int TW, int ntw, int nth, int spill_stride, int ring_stride,
    const int* __restrict__ hdr, const A* __restrict__ spill, const A* __restrict__ part,
    int64_t ntiles, A* __restrict__ Dout, A* __restrict__ Lout) {
    const int R = __builtin_amdgcn_readfirstlane(hdr[0]);
    if (R == 0) return;
    const FixTile f = fix_tile(blockIdx.x, H, W, TH, TW, ntw, nth);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const A* pm = part + 3 * static_cast<int64_t>(blockIdx.x) * ring_stride;
    int lg;
    if (fix_slots_ok(f, R, TW, false, lg)) {
        // ring tiles: the slot enumeration, kFixBatch slots per lane with
        // all their loads issued before any merge
        const FixRing g = fix_ring<false>(f, R, lg, HW, W, spill_stride);
        const int64_t qstride = ntiles * spill_stride;
        const int step = static_cast<int>(blockDim.x);
        for (int s0 = threadIdx.x; s0 < g.n; s0 += step * kFixBatch) {
            int lr[kFixBatch], lc[kFixBatch];
            bool act[kFixBatch];
            uint32_t pp[kFixBatch];
            int64_t e[kFixBatch][3];
            A st[kFixBatch][3], sv[kFixBatch][3][3];
#pragma unroll
            for (int k = 0; k < kFixBatch; ++k) {
                fix_slot<false>(f, g, s0 + k * step, W, lr[k], lc[k], act[k], pp[k], e[k]);
                const int ri = ring_slot(lr[k], lc[k], f.th, f.tw, R);
#pragma unroll
                for (int q = 0; q < 3; ++q) {
                    st[k][q] = pm[q * ring_stride + ri];
#pragma unroll
                    for (int c = 0; c < 3; ++c)
                        sv[k][q][c] = spill[e[k][c] >= 0 ? q * qstride + e[k][c] : 0];
                }
            }
#pragma unroll
            for (int k = 0; k < kFixBatch; ++k) {
                if (!act[k]) continue;
                A m = st[k][0], u = st[k][1], z = st[k][2];
#pragma unroll
                for (int c = 0; c < 3; ++c)
                    if (e[k][c] >= 0)
                        state_merge<A, LOGW>(m, u, z, sv[k][0][c], sv[k][1][c], sv[k][2][c]);
                A Dv, Lv;
                state_final<A, LOGW>(m, u, z, Dv, Lv);
                Dout[g.pb + pp[k]] = Dv;
                Lout[g.pb + pp[k]] = Lv;
            }
        }
        return;
    }
    const int n = ring_count(f.th, f.tw, R);
    for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
        int lr, lc;
        ring_pixel(idx, f.th, f.tw, R, lr, lc);
        A m = pm[idx], u = pm[ring_stride + idx], z = pm[2 * ring_stride + idx];
        spill_visit(f, R, lr, lc, [&](int64_t tn, int e) {
            state_merge<A, LOGW>(m, u, z, spill[tn * spill_stride + e],
                                 spill[(ntiles + tn) * spill_stride + e],
                                 spill[(2 * ntiles + tn) * spill_stride + e]);
        });
        A Dv, Lv;
        state_final<A, LOGW>(m, u, z, Dv, Lv);
        const int64_t p = f.bc * HW + static_cast<int64_t>(f.h0 + lr) * W + (f.w0 + lc);
        Dout[p] = Dv;
        Lout[p] = Lv;
    }
}

// Backward.  LDS: x; L (log weights) or E = exp(-L) (positive weights);
// alpha = gD; beta = gLogC - gD D (so score(o, v) = alpha[o] v + beta[o]);
// and the x-gradient window.  With a 16-bit T the gx partial sums go to
// `gxp` (accumulator type) and the fix-up rounds once.
template <typename A, bool LOGW>
__device__ __forceinline__ A frac_tile(A w, A l) {
    // f(w, L): log weights exp(w - L); positive weights w E with l = E = exp(-L)
    if (LOGW) return (w == -Lim<A>::inf() || l == -Lim<A>::inf()) ? A(0) : Lim<A>::ex(w - l);
    return (w == A(0) || l == Lim<A>::inf()) ? A(0) : w * l;
}

// Log keys of the backward's fractions f = exp(l - L): the staged L is
// log_key(L) = L log2(e) (fp32; fp64 keeps natural units), with an empty
// row's L = -inf staged as +inf, and a term's logit enters as
// log_scale(l) = l log2(e); then f = exp2(log_scale(l) - log_key(L)) is 0
// for an empty row without a test (exp2(-inf)), and a masked logit (-inf) is
// tested once by the caller.  One multiply per term serves both fractions
// of a term (own and mirror output).
template <typename A>
__device__ __forceinline__ A log_scale(A l) {
    if constexpr (sizeof(A) == 4) return l * 1.44269504088896341f;
    return l;
}
template <typename A>
__device__ __forceinline__ A log_key(A L) {
    return L == -Lim<A>::inf() ? Lim<A>::inf() : log_scale<A>(L);
}
template <typename A>
__device__ __forceinline__ A frac_log(A kw, A key) {
    if constexpr (sizeof(A) == 4) return __builtin_amdgcn_exp2f(kw - key);
    return Lim<A>::ex(kw - key);
}

// Tile geometry of the backward with a HALO border: SGeo's, or for the
// narrow border (fp64, tables within it: the NSH_NARROW_HALO hint) rows at the
// plain LW pitch -- its 8-byte elements are read as 16-lane rows of 128 bytes,
// which cover every bank at any pitch -- so that three 256-lane workgroups
// share a CU.
template <int VEC, int ROWS, int TPR, int HALO>
struct NTileGeo : SGeo<VEC, ROWS, TPR, true, HALO> {
    using Base = SGeo<VEC, ROWS, TPR, true, HALO>;
    static constexpr int PITCH = HALO == kRmax ? Base::PITCH : Base::LW;
    static constexpr int TILE = Base::LH * PITCH;
};

// CONTIG (VEC = 4, W a multiple of 4, 16-byte aligned tensors): lane tx owns
// the four consecutive pixels 4 tx .. 4 tx + 3 of its row, moved with one
// 16-byte load or store per shift, and the LDS tiles use the de-interleaved
// columns of BwdLayout (conflict-free for these lanes).  Otherwise the lanes
// are strided (pixels tx, tx + TPR, ...) with row-major tiles.
template <typename T, int VEC, int TPR, int ROWS, int D, bool LOGW, bool CONTIG,
          int WPE = kScatterWavesPerEU<TPR * ROWS>, int HALO = kRmax>
__global__ __launch_bounds__(TPR * ROWS, WPE) void
normalized_bwd_scatter_kernel(const T* __restrict__ x, const T* __restrict__ w,
                              const acc_t<T>* __restrict__ Dg, const acc_t<T>* __restrict__ Lg,
                              const acc_t<T>* __restrict__ gDg, const acc_t<T>* __restrict__ gLg,
                              const int64_t* __restrict__ shifts, int S, int codes, int C, int H,
                              int W, int ntw, int nth, int64_t plane_step, T* __restrict__ gx,
                              acc_t<T>* __restrict__ gxp, T* __restrict__ gw,
                              int* __restrict__ hdr, acc_t<T>* __restrict__ spill) {
    using A = acc_t<T>;
    using G = NTileGeo<VEC, ROWS, TPR, HALO>;
    static_assert(HALO == kRmax || !CONTIG, "the narrow border is built for strided lanes");
    static_assert(!CONTIG || VEC == 4, "the contiguous form moves 4-pixel vectors");
    // Column offset within a row: de-interleaved for the contiguous lanes
    // (the strided SGeo pitch is the BwdLayout pitch), row-major otherwise.
    using L = BwdLayout<VEC, G::LW, G::PITCH>;
    auto colm = [](int j) { return CONTIG ? L::col(j) : j; };
    static_assert(!CONTIG || L::PITCH == G::PITCH, "de-interleaved rows use the strided pitch");
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* lt = xt + G::TILE;
    A* at = lt + G::TILE;
    A* bt = at + G::TILE;
    A* mg = bt + G::TILE;

    const int64_t t = xcd_tile(blockIdx.x, gridDim.x);
    const TileIdx ti = tile_of(t, ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t off = ti.bc * HW;
    const T* xp = x + off;
    const A* Dp = Dg + off;
    const A* Lp = Lg + off;
    const A* gDp = gDg + off;
    const A* gLp = gLg + off;
    stage_shifts(shl, shifts, S, 3, H, W, (codes & kCodesRows) != 0);
    {
        const bool cheap = H >= G::LH && W >= G::LW;
        for (int i = threadIdx.x; i < G::LH * G::LW; i += blockDim.x) {
            const int r = i / G::LW;
            const int cc = i - r * G::LW;
            int gh = ti.h0 - HALO + r;
            int gw_ = ti.w0 - HALO + cc;
            if (cheap) {
                gh = wrap1(gh, H);
                gw_ = wrap1(gw_, W);
            } else {
                gh = static_cast<int>(mod_pos(gh, H));
                gw_ = static_cast<int>(mod_pos(gw_, W));
            }
            const uint32_t g = static_cast<uint32_t>(gh) * static_cast<uint32_t>(W) +
                               static_cast<uint32_t>(gw_);
            const int li = r * G::PITCH + colm(cc);
            const A gd = gDp[g];
            xt[li] = to_acc(xp[g]);
            lt[li] = LOGW ? log_key<A>(Lp[g]) : Lim<A>::ex(-Lp[g]);
            at[li] = gd;
            bt[li] = gLp[g] - gd * Dp[g];
        }
    }
    const int R = near_radius<HALO>(shl, S, false);
    if (blockIdx.x == 0 && threadIdx.x == 0) hdr[0] = R;  // for the fix-up
    lds_zero(mg, G::TILE);
    __syncthreads();

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    // The lane's pixels: column, activity and in-plane offset of pixel k,
    // and its LDS index displaced by (dx, dy).
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);  // strided form
    const int wq0 = ti.w0 + tx * VEC;                                          // contiguous form
    const bool cact = h < H && wq0 < W;
    const uint32_t cown = static_cast<uint32_t>(cact ? h : 0) * static_cast<uint32_t>(W) +
                          static_cast<uint32_t>(cact ? wq0 : 0);
    auto pcol = [&](int k) { return CONTIG ? wq0 + k : ti.w0 + tx + k * TPR; };
    auto pact = [&](int k) { return CONTIG ? cact : px.act[k]; };
    auto pown = [&](int k) { return CONTIG ? cown + k : px.own[k]; };
    const int lrow = (ty + HALO) * G::PITCH + (CONTIG ? tx : 0);
    auto lidx = [&](int k, int dx, int dy) {
        return lrow + dx * G::PITCH + (CONTIG ? colm(HALO + k + dy) : tx + HALO + k * TPR + dy);
    };
    const int64_t b = ti.bc / C;
    const bool wsh = (codes & kCodesSharedW) != 0;
    const T* w_bc = w + weight_plane(b, ti.bc - b * C, C, wsh) * HW;
    const int64_t wstep = weight_step(plane_step, C, wsh);
    T* g_bc = gw + ti.bc * HW;  // the gradient has every channel
    // Weight prefetch ring: raw slots (promoted where consumed), one vector
    // per lane (contiguous) or one element per pixel (strided).
    using Slot = std::conditional_t<CONTIG, SlotRaw<T, VEC>, PixSlot<T, VEC>>;
    auto slot_fill = [&](const T* wp, Slot& sl) {
        if constexpr (CONTIG)
            slot_load_at<T, VEC, kNormBwdNT<T>>(wp, cown * static_cast<uint32_t>(sizeof(T)),
                                                       sl);
        else
            slot_load_pixels<T, VEC, TPR, kNormBwdNT<T>>(wp, px, sl);
    };
    auto slot_take = [&](const Slot& sl, A (&wv)[VEC]) {
        if constexpr (CONTIG)
            slot_get<T, VEC>(sl, wv);
        else
            slot_get_pixels<T, VEC>(sl, wv);
    };

    A xo[VEC], lo[VEC], ao[VEC], bo[VEC], gxa[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const int i = lidx(k, 0, 0);
        xo[k] = xt[i];
        lo[k] = lt[i];
        ao[k] = at[i];
        bo[k] = bt[i];
        gxa[k] = A(0);
    }
    Slot wb[D];
#pragma unroll
    for (int d = 0; d < D; ++d) slot_fill(w_bc + static_cast<int64_t>(min(d, S - 1)) * wstep, wb[d]);
    // the next refill's plane and the next shift's record, advanced per
    // shift; the gw plane of the current shift
    const T* wr = w_bc + static_cast<int64_t>(min(D, S - 1)) * wstep;
    ShiftRec rn = read_shift(shl, 0);
    T* gs = g_bc;

    // gw_s[q] for one pixel given the neighbour values at q + s.  Log
    // weights: the staged L are log keys (log_key), so both fractions are
    // exp of one difference of the scaled logit (frac_log), with a single
    // test of the mask.
    auto grad_w = [&](int k, A wv, A xf, A lp, A ap, A bp, bool okp, A& fo) -> A {
        const bool masked = LOGW ? wv == -Lim<A>::inf() : wv == A(0);
        A Ff, Fi;
        if constexpr (LOGW) {
            const A kw = log_scale<A>(wv);
            fo = masked ? A(0) : frac_log<A>(kw, lo[k]);  // f(w_s[q], L[q])
            Ff = fo;
            Fi = masked ? A(0) : frac_log<A>(kw, lp);     // f(w_s[q], L[q+s])
        } else {
            fo = frac_tile<A, LOGW>(wv, lo[k]);  // f(w_s[q], L[q])
            Ff = lo[k];                          // F(L[q])
            Fi = lp;
        }
        const A sf = fma_acc(ao[k], xf, bo[k]);   // score(q, x[q+s])
        const A si = fma_acc(ap, xo[k], bp);      // score(q+s, x[q])
        const A gv = fma_acc(Ff, sf, okp ? Fi * si : A(0));
        if (okp) gxa[k] = fma_acc(LOGW ? Fi : frac_tile<A, LOGW>(wv, lp), ap, gxa[k]);
        return masked ? A(0) : gv;
    };

    // Interior tiles (every pixel and every q + s inside the image for all
    // rows of the table): no forward-box test and no mirror mask.
    const int R_all = table_radius(shl, S, false);
    const bool interior = ti.h0 >= R_all && ti.h0 + G::TH + R_all <= H && ti.w0 >= R_all &&
                          ti.w0 + G::TW + R_all <= W;
    int last_dx = kClamp;
    auto step = [&](int s, Slot& slot, auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        const ShiftRec rc = rn;
        rn = read_shift(shl, min(s + 1, S - 1));
        A wv[VEC];
        slot_take(slot, wv);
        slot_fill(wr, slot);
        wr += s + D + 1 < S ? wstep : 0;
        if (shift_in_lds<HALO>(rc)) {
            if (rc.dx != last_dx) {
                lds_barrier();
                last_dx = rc.dx;
            }
            const bool rok = rc.inv && (rc.per || in_range(h + rc.dx, H));
            A gv[VEC];
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                const int i = lidx(k, rc.dx, rc.dy);
                A fo;
                if constexpr (FAST) {
                    gv[k] = grad_w(k, wv[k], xt[i], lt[i], at[i], bt[i], rc.inv, fo);
                    if constexpr (!CONTIG)
                        store_elem_at<T, true>(gs, px.own[k] * static_cast<uint32_t>(sizeof(T)),
                                               from_acc<T>(gv[k]));
                    mg[i] += fo * ao[k];
                } else {
                    const bool okp = rok && (rc.per || in_range(pcol(k) + rc.dy, W));
                    const A wk = fwd_kept(rc, h, pcol(k), H, W) ? wv[k] : masked_key<A, LOGW>();
                    gv[k] = grad_w(k, wk, xt[i], lt[i], at[i], bt[i], okp, fo);
                    if constexpr (!CONTIG)
                        if (px.act[k])
                            store_elem_at<T, true>(
                                gs, px.own[k] * static_cast<uint32_t>(sizeof(T)), from_acc<T>(gv[k]));
                    // x-gradient term of q + s: f(w_s[q], L[q]) gD[q]
                    mg[i] += pact(k) ? fo * ao[k] : A(0);
                }
            }
            if constexpr (CONTIG)
                if (FAST || cact)
                    store_acc_at<T, VEC, true>(gs, cown * static_cast<uint32_t>(sizeof(T)), gv);
        }
        gs += plane_step;
    };
    auto ring = [&](auto fast_tag) {
        const int S_ring = S - S % D;
        for (int s0 = 0; s0 < S_ring; s0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) step(s0 + d, wb[d], fast_tag);
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (S_ring + d < S) step(S_ring + d, wb[d], fast_tag);
    };
    if (interior)
        ring(std::true_type{});
    else
        ring(std::false_type{});
    // Shifts beyond the halo: gather form, neighbour values from HBM.
    for (int s = 0; s < S && (CONTIG ? cact : px.any); ++s) {
        const ShiftRec rc = read_shift(shl, s);
        if (shift_in_lds<HALO>(rc)) continue;
        const T* wp = w_bc + static_cast<int64_t>(s) * wstep;
        T* gs = g_bc + static_cast<int64_t>(s) * plane_step;
        int hp = h + rc.dxm;
        hp -= hp >= H ? H : 0;
        int hm = h - rc.dxm;
        hm += hm < 0 ? H : 0;
        const bool rok = rc.inv && (rc.per || in_range(h + rc.dx, H));
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            if (!pact(k)) continue;
            const int wq = pcol(k);
            int wj = wq + rc.dym;
            wj -= wj >= W ? W : 0;
            int wm = wq - rc.dym;
            wm += wm < 0 ? W : 0;
            const uint32_t ip = static_cast<uint32_t>(hp) * W + wj;
            const uint32_t im = static_cast<uint32_t>(hm) * W + wm;
            const bool okp = rok && (rc.per || in_range(wq + rc.dy, W));
            const A lp = LOGW ? log_key<A>(Lp[ip]) : Lim<A>::ex(-Lp[ip]);
            const A gdp = gDp[ip];
            A fo;
            const A wk = fwd_kept(rc, h, wq, H, W) ? to_acc(*elem_ptr(wp, pown(k)))
                                                   : masked_key<A, LOGW>();
            const A g = grad_w(k, wk, to_acc(xp[ip]), lp, gdp, gLp[ip] - gdp * Dp[ip], okp, fo);
            store_elem_nt<T>(elem_ptr(gs, pown(k)), from_acc<T>(g));
            // x-gradient term from o = (q - s) mod: f(w_s[o], L[o]) gD[o]
            const A lm = LOGW ? Lp[im] : Lim<A>::ex(-Lp[im]);
            const A wo = fwd_kept_src(rc, h, wq, H, W) ? to_acc(wp[im]) : masked_key<A, LOGW>();
            gxa[k] = fma_acc(frac_tile<A, LOGW>(wo, lm), gDp[im], gxa[k]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!pact(k)) continue;
        const A v = gxa[k] + mg[lidx(k, 0, 0)];
        if (gxp != nullptr)
            gxp[off + pown(k)] = v;
        else
            gx[off + pown(k)] = from_acc<T>(v);
    }
    if (R == 0) return;
    const int th = min(G::TH, H - ti.h0);
    const int tw = min(G::TW, W - ti.w0);
    const int n = spill_count(th, tw, R);
    A* sg = spill + t * G::SPILL;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        int i, j;
        spill_coords(e, th, tw, R, i, j);
        sg[e] = mg[(i + HALO) * G::PITCH + colm(j + HALO)];
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr size_t kNLdsLimit = 64 * 1024;

template <int VEC>
static size_t nfwd_lds(int S, size_t ab) {
    return shift_lds_bytes(S) + static_cast<size_t>(NGeo<VEC>::LH) * NGeo<VEC>::LW * ab;
}
template <int VEC>
static size_t nbwd_lds(int S, size_t ab) {
    return shift_lds_bytes(S) + 5 * static_cast<size_t>(NGeo<VEC>::LH) * NGeo<VEC>::LW * ab;
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
    int codes = 0;  // kCodesRows / kCodesSharedW (from NSH_SHIFT_CODES, NSH_SHARED_WEIGHTS)
    bool narrow = false;  // NSH_NARROW_HALO: every row within 6 pixels (a hint)
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
                       static_cast<const T*>(w), sh, d.S, d.codes, d.C, d.H, d.W, ntw, nth, step,
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
                       static_cast<const A*>(gD), static_cast<const A*>(gL), sh, d.S, d.codes, d.C, d.H,
                       d.W, ntw, nth, step, static_cast<T*>(gx), static_cast<T*>(gw));
    return nsh_host::check_launch("normalized_accumulate_uz_backward");
}

// ---- scatter path -------------------------------------------------------
// Tiles of 16 lanes x VEC pixels (4; 2 for fp64) across, 32 rows down
// (512-lane workgroups; the fp32 passes take 32 lanes, 128 x 32 tiles): the
// forward keeps four LDS arrays (x and the three state windows), the
// backward five (x, L or E, alpha, beta, window).  Weight prefetch depth 2,
// except the fp64 backward: four shifts in flight (c3 fp64 0.226 -> 0.213
// ms); depth 3 or 4 makes the fp32 passes and every forward 1-3% slower.
// fp32 forward: 128 x 32 tiles with nontemporal weight loads, c3 positive
// 0.329 -> 0.322 ms; the 16-bit forward stays on 64 x 32 tiles with plain
// loads (c2 logits 0.150 ms against 0.154 ms wide, 0.159 ms wide and
// nontemporal).  fp32 backward: 32 lanes per row (128 x 32 tiles, one
// workgroup per CU): c3 positive 0.690 -> 0.666 ms; the 16-bit backward
// stays at 16 (c2 logits 0.236 ms against 0.254 ms on the wide tiles).
template <typename T, bool BWD, bool NARROW = false>
struct NScatterCfg {
    static_assert(!NARROW || (BWD && sizeof(T) == 8), "the narrow border serves the fp64 backward");
    static constexpr bool kWide = sizeof(T) != 8;
    static constexpr int VEC = sizeof(T) == 8 ? 2 : 4;
    static constexpr int TPR = (kWide && sizeof(T) == 4) ? 32 : kTPR;
    // fp64 forward: 32 x 16 tiles (twice the workgroups; c3 0.083 -> 0.080
    // ms).  fp64 backward: 32 x 32 tiles, or on the narrow border 32 x 16
    // (three 256-lane workgroups per CU: the c3 fp64 shape's 768 tiles in one
    // round); 32 x 16 on the 8-pixel border (two workgroups per CU, 1.5
    // rounds) measured no faster.
    static constexpr int ROWS = ((!BWD || NARROW) && sizeof(T) == 8) ? 16 : 32;
    static constexpr int HALO = NARROW ? 6 : kRmax;
    // prefetch depth: 4 for the fp64 backward on the 8-pixel border, 2 on
    // the narrow one (c3 fp64 0.189 ms at 4, 0.181 at 2, 0.191 at 6)
    static constexpr int D = (BWD && sizeof(T) == 8 && !NARROW) ? 4 : 2;
    // register budget: a 1024-lane workgroup holds a CU alone (its LDS), so
    // four waves per SIMD; smaller ones two workgroups per CU, the narrow
    // border's three (1-pixel lanes there, 32 per row and 24 waves per CU:
    // no faster)
    static constexpr int WPE = NARROW ? 3
                                      : (TPR * ROWS >= 1024 ? 4 : kScatterWavesPerEU<TPR * ROWS>);
    using G = NTileGeo<VEC, ROWS, TPR, HALO>;
};

constexpr size_t kNScatterLds = 160 * 1024 - 1024;
constexpr int64_t kNHeader = 256;

struct NPlan {
    bool ok = false;
    bool narrow = false;  // the backward on the narrow border (NScatterCfg<T, true, true>)
    int ntw = 0, nth = 0, spill = 0, ring = 0;
    int64_t tiles = 0, spill_bytes = 0, part_bytes = 0, total = 0;
    size_t lds = 0;
};

static int64_t n_align256(int64_t b) { return (b + 255) / 256 * 256; }

template <typename T, bool BWD, bool NARROW = false>
static NPlan n_plan_cfg(const NDims& d) {
    using Cfg = NScatterCfg<T, BWD, NARROW>;
    using G = typename Cfg::G;
    constexpr bool bwd = BWD;
    const int64_t ab = sizeof(acc_t<T>);
    NPlan p;
    p.narrow = NARROW;
    p.ntw = static_cast<int>(nsh_host::ceil_div(d.W, G::TW));
    p.nth = static_cast<int>(nsh_host::ceil_div(d.H, G::TH));
    p.tiles = static_cast<int64_t>(d.B) * d.C * p.ntw * p.nth;
    p.lds = shift_lds_bytes(d.S) +
            (bwd ? 5 : 4) * static_cast<size_t>(G::TILE) * ab;
    p.spill = G::SPILL;
    p.ring = G::RING;
    p.ok = p.ntw >= 2 && p.nth >= 2 && d.W - (p.ntw - 1) * G::TW >= kRmax &&
           d.H - (p.nth - 1) * G::TH >= kRmax && p.lds <= kNScatterLds;
    p.spill_bytes = n_align256((bwd ? 1 : 3) * p.tiles * p.spill * ab);
    if (bwd)
        p.part_bytes = sizeof(T) < sizeof(acc_t<T>)
                           ? n_align256(static_cast<int64_t>(d.B) * d.C * d.H * d.W * ab)
                           : 0;
    else
        p.part_bytes = n_align256(3 * p.tiles * p.ring * ab);
    p.total = kNHeader + p.spill_bytes + p.part_bytes;
    return p;
}

// The plan; the fp64 backward on the narrow border when the caller's hint
// asks for it (d.narrow) and `narrow` allows it.
template <typename T>
static NPlan n_plan(const NDims& d, bool bwd, bool narrow = true) {
    if constexpr (sizeof(T) == 8) {
        if (bwd && narrow && d.narrow) {
            const NPlan p = n_plan_cfg<T, true, true>(d);
            if (p.ok) return p;
        }
    }
    return bwd ? n_plan_cfg<T, true>(d) : n_plan_cfg<T, false>(d);
}

static bool n_scatter_disabled() {
    static const bool off = [] {
        const char* e = getenv("NSH_NORM_SCATTER");
        return e != nullptr && e[0] == '0';
    }();
    return off;
}

template <typename T>
static bool n_use_scatter(const NPlan& p, void* ws, int64_t ws_bytes) {
    return ws != nullptr && !n_scatter_disabled() && p.ok && ws_bytes >= p.total &&
           nsh_host::aligned(ws, 256);
}

// NH > 1: w is a head stack (S*B, NH, H, W) mixed by mix (C, NH) in the
// kernel's weight load.
template <typename T, bool LOGW, int NH = 1>
static int n_scatter_fwd(const void* x, const void* w, const int64_t* sh, NDims d, void* D,
                         void* L, const NPlan& p, void* ws, hipStream_t st,
                         const acc_t<T>* mix = nullptr) {
    using Cfg = NScatterCfg<T, false>;
    using A = acc_t<T>;
    constexpr int V = Cfg::VEC, TPR = Cfg::TPR, RW = Cfg::ROWS;
    char* base = static_cast<char*>(ws);
    int* hdr = reinterpret_cast<int*>(base);
    A* spill = reinterpret_cast<A*>(base + kNHeader);
    A* part = reinterpret_cast<A*>(base + kNHeader + p.spill_bytes);
    const int64_t step = static_cast<int64_t>(d.B) * (NH > 1 ? NH : d.C) * d.H * d.W;
    hipLaunchKernelGGL((normalized_fwd_scatter_kernel<T, V, TPR, RW, Cfg::D, LOGW, Cfg::WPE, NH>),
                       dim3(static_cast<unsigned>(p.tiles)), dim3(TPR * RW), p.lds, st,
                       static_cast<const T*>(x), static_cast<const T*>(w), sh, d.S, d.codes, d.C, d.H, d.W,
                       p.ntw, p.nth, step, static_cast<A*>(D), static_cast<A*>(L), hdr, spill, part,
                       p.ring, p.tiles, mix);
    if (int rc = nsh_host::check_launch("normalized_accumulate_uz_forward")) return rc;
    hipLaunchKernelGGL((normalized_fixup_kernel<A, LOGW>), dim3(static_cast<unsigned>(p.tiles)),
                       dim3(256), 0, st, d.H, d.W, RW, TPR * V, p.ntw, p.nth, p.spill, p.ring,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill),
                       static_cast<const A*>(part), p.tiles, static_cast<A*>(D),
                       static_cast<A*>(L));
    return nsh_host::check_launch("normalized_accumulate_uz_forward (fix-up)");
}

template <typename T, bool LOGW, bool NARROW>
static int n_scatter_bwd_cfg(const void* x, const void* w, const void* D, const void* L,
                             const void* gD, const void* gL, const int64_t* sh, NDims d, void* gx,
                             void* gw, const NPlan& p, void* ws, hipStream_t st) {
    using Cfg = NScatterCfg<T, true, NARROW>;
    using A = acc_t<T>;
    constexpr int V = Cfg::VEC, TPR = Cfg::TPR, RW = Cfg::ROWS;
    char* base = static_cast<char*>(ws);
    int* hdr = reinterpret_cast<int*>(base);
    A* spill = reinterpret_cast<A*>(base + kNHeader);
    A* part = p.part_bytes ? reinterpret_cast<A*>(base + kNHeader + p.spill_bytes) : nullptr;
    const int64_t step = static_cast<int64_t>(d.B) * d.C * d.H * d.W;
    // Contiguous 16-byte lanes where the row length and the pointers allow.
    const size_t vb = static_cast<size_t>(V) * sizeof(T);
    const bool contig = V == 4 && d.W % V == 0 && nsh_host::aligned(x, vb) &&
                        nsh_host::aligned(w, vb) && nsh_host::aligned(gw, vb);
#define NSH_NBWD_LAUNCH(CT_)                                                                    \
    hipLaunchKernelGGL((normalized_bwd_scatter_kernel<T, V, TPR, RW, Cfg::D, LOGW, CT_,      \
                                                      Cfg::WPE, Cfg::HALO>),                    \
                       dim3(static_cast<unsigned>(p.tiles)), dim3(TPR * RW), p.lds, st,         \
                       static_cast<const T*>(x), static_cast<const T*>(w),                      \
                       static_cast<const A*>(D), static_cast<const A*>(L),                      \
                       static_cast<const A*>(gD), static_cast<const A*>(gL), sh, d.S, d.codes,  \
                       d.C, d.H, d.W, p.ntw, p.nth, step, static_cast<T*>(gx), part,            \
                       static_cast<T*>(gw),                                                     \
                       hdr, spill)
    if constexpr (V == 4) {
        if (contig)
            NSH_NBWD_LAUNCH(true);
        else
            NSH_NBWD_LAUNCH(false);
    } else {
        NSH_NBWD_LAUNCH(false);
    }
#undef NSH_NBWD_LAUNCH
    if (int rc = nsh_host::check_launch("normalized_accumulate_uz_backward")) return rc;
    constexpr bool kPart = sizeof(T) < sizeof(A);
    hipLaunchKernelGGL((spill_fixup_kernel<T, A, 1, kPart>), dim3(static_cast<unsigned>(p.tiles)),
                       dim3(256), 0, st, d.H, d.W, RW, TPR * V, p.ntw, p.nth, p.spill,
                       static_cast<const int*>(hdr), static_cast<const A*>(spill), p.tiles,
                       static_cast<const A*>(part), static_cast<T*>(gx), static_cast<T*>(nullptr));
    return nsh_host::check_launch("normalized_accumulate_uz_backward (fix-up)");
}

template <typename T, bool LOGW>
static int n_scatter_bwd(const void* x, const void* w, const void* D, const void* L,
                         const void* gD, const void* gL, const int64_t* sh, NDims d, void* gx,
                         void* gw, const NPlan& p, void* ws, hipStream_t st) {
    if constexpr (sizeof(T) == 8) {
        if (p.narrow)
            return n_scatter_bwd_cfg<T, LOGW, true>(x, w, D, L, gD, gL, sh, d, gx, gw, p, ws, st);
    }
    return n_scatter_bwd_cfg<T, LOGW, false>(x, w, D, L, gD, gL, sh, d, gx, gw, p, ws, st);
}

// Either plan may run (n_run_bwd takes the 8-pixel border when the workspace
// is too small for the narrow one): the larger of the two.
template <typename T>
static int64_t n_workspace(const NDims& d, bool bwd) {
    const NPlan p = n_plan<T>(d, bwd, false);
    const NPlan q = n_plan<T>(d, bwd);
    return std::max(p.ok ? p.total : 0, q.ok ? q.total : 0);
}

template <typename T, bool LOGW>
static int n_run_fwd(const void* x, const void* w, const int64_t* sh, NDims d, void* D, void* L,
                     void* ws, int64_t ws_bytes, hipStream_t st) {
    const NPlan p = n_plan<T>(d, false);
    if (n_use_scatter<T>(p, ws, ws_bytes))
        return n_scatter_fwd<T, LOGW>(x, w, sh, d, D, L, p, ws, st);
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
                     const void* gL, const int64_t* sh, NDims d, void* gx, void* gw, void* ws,
                     int64_t ws_bytes, hipStream_t st) {
    NPlan p = n_plan<T>(d, true);
    if (p.narrow && !n_use_scatter<T>(p, ws, ws_bytes)) p = n_plan<T>(d, true, false);
    if (n_use_scatter<T>(p, ws, ws_bytes))
        return n_scatter_bwd<T, LOGW>(x, w, D, L, gD, gL, sh, d, gx, gw, p, ws, st);
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
    const int codes = nsh::dtype_codes(dtype);
    const bool narrow = (dtype & NSH_NARROW_HALO) != 0;
    dtype &= ~NSH_DTYPE_FLAGS;
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
                    static_cast<int>(H), static_cast<int>(W), codes, narrow};
    return NSH_OK;
}

#define NSH_DISPATCH_LOGW(T, FN, ...)                                   \
    (log_weights ? nsh::FN<T, true>(__VA_ARGS__) : nsh::FN<T, false>(__VA_ARGS__))

extern "C" int64_t nsh_normalized_workspace_bytes(int64_t S, int64_t B, int64_t C, int64_t H,
                                                  int64_t W, int dtype, int backward) {
    nsh::NDims d;
    if (n_check("normalized_accumulate_uz", S, B, C, H, W, dtype, &d) != NSH_OK) return -1;
    dtype &= ~NSH_DTYPE_FLAGS;
    const bool bwd = backward != 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::n_workspace<nsh::f16>(d, bwd);
        case NSH_DTYPE_BFLOAT16: return nsh::n_workspace<nsh::bf16>(d, bwd);
        case NSH_DTYPE_FLOAT32: return nsh::n_workspace<float>(d, bwd);
        default: return nsh::n_workspace<double>(d, bwd);
    }
}

extern "C" int nsh_normalized_accumulate_uz_forward(const void* x, const void* weights,
                                                    const int64_t* shifts, int64_t S, int64_t B,
                                                    int64_t C, int64_t H, int64_t W, int dtype,
                                                    int log_weights, void* D, void* log_C,
                                                    void* workspace, int64_t workspace_bytes,
                                                    void* stream) {
    nsh::NDims d;
    if (int rc = n_check("normalized_accumulate_uz", S, B, C, H, W, dtype, &d)) return rc;
    dtype &= ~NSH_DTYPE_FLAGS;
    if (!x || !weights || !shifts || !D || !log_C)
        return fail(NSH_ERR_INVALID, "normalized_accumulate_uz: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = workspace;
    const int64_t nws = workspace ? workspace_bytes : 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return NSH_DISPATCH_LOGW(nsh::f16, n_run_fwd, x, weights, shifts, d, D, log_C, ws, nws, st);
        case NSH_DTYPE_BFLOAT16: return NSH_DISPATCH_LOGW(nsh::bf16, n_run_fwd, x, weights, shifts, d, D, log_C, ws, nws, st);
        case NSH_DTYPE_FLOAT32: return NSH_DISPATCH_LOGW(float, n_run_fwd, x, weights, shifts, d, D, log_C, ws, nws, st);
        default: return NSH_DISPATCH_LOGW(double, n_run_fwd, x, weights, shifts, d, D, log_C, ws, nws, st);
    }
}

// Head mixing in the weight load: with a (C, heads) mix the scatter path
// only (the shapes the workspace plan serves), positive weights, no grad.
template <typename T>
static int n_run_fwd_mixed(const void* x, const void* hw, const void* mix, const int64_t* sh,
                           nsh::NDims d, int heads, void* D, void* L, void* ws, int64_t nws,
                           hipStream_t st) {
    using A = nsh::acc_t<T>;
    const nsh::NPlan p = nsh::n_plan<T>(d, false);
    if (!nsh::n_use_scatter<T>(p, ws, nws))
        return fail(NSH_ERR_UNSUPPORTED,
                    "normalized_accumulate_uz_forward_mixed: shape or workspace not served by "
                    "the scatter path");
    const A* m = static_cast<const A*>(mix);
    switch (heads) {
        case 2: return nsh::n_scatter_fwd<T, false, 2>(x, hw, sh, d, D, L, p, ws, st, m);
        case 3: return nsh::n_scatter_fwd<T, false, 3>(x, hw, sh, d, D, L, p, ws, st, m);
        default: return nsh::n_scatter_fwd<T, false, 4>(x, hw, sh, d, D, L, p, ws, st, m);
    }
}

extern "C" int nsh_normalized_accumulate_uz_forward_mixed(
    const void* x, const void* head_weights, const void* mix, const int64_t* shifts, int64_t S,
    int64_t B, int64_t C, int64_t H, int64_t W, int64_t heads, int dtype, void* D, void* log_C,
    void* workspace, int64_t workspace_bytes, void* stream) {
    nsh::NDims d;
    if (int rc = n_check("normalized_accumulate_uz_forward_mixed", S, B, C, H, W, dtype, &d))
        return rc;
    if (dtype & NSH_SHARED_WEIGHTS)
        return fail(NSH_ERR_INVALID,
                    "normalized_accumulate_uz_forward_mixed: shared weights do not apply to a "
                    "head stack");
    dtype &= ~NSH_DTYPE_FLAGS;
    if (!x || !head_weights || !mix || !shifts || !D || !log_C)
        return fail(NSH_ERR_INVALID, "normalized_accumulate_uz_forward_mixed: null pointer argument");
    if (heads < 2 || heads > 4)
        return fail(NSH_ERR_UNSUPPORTED,
                    "normalized_accumulate_uz_forward_mixed: %lld heads (2..4 are served)",
                    static_cast<long long>(heads));
    if (B * heads > (int64_t(1) << 24))
        return fail(NSH_ERR_INVALID, "normalized_accumulate_uz_forward_mixed: B*heads too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t nws = workspace ? workspace_bytes : 0;
    const int h = static_cast<int>(heads);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return n_run_fwd_mixed<nsh::f16>(x, head_weights, mix, shifts, d, h, D, log_C, workspace, nws, st);
        case NSH_DTYPE_BFLOAT16: return n_run_fwd_mixed<nsh::bf16>(x, head_weights, mix, shifts, d, h, D, log_C, workspace, nws, st);
        case NSH_DTYPE_FLOAT32: return n_run_fwd_mixed<float>(x, head_weights, mix, shifts, d, h, D, log_C, workspace, nws, st);
        default: return n_run_fwd_mixed<double>(x, head_weights, mix, shifts, d, h, D, log_C, workspace, nws, st);
    }
}

extern "C" int nsh_normalized_accumulate_uz_backward(const void* x, const void* weights,
                                                     const void* D, const void* log_C,
                                                     const void* grad_D, const void* grad_log_C,
                                                     const int64_t* shifts, int64_t S, int64_t B,
                                                     int64_t C, int64_t H, int64_t W, int dtype,
                                                     int log_weights, void* grad_x, void* grad_w,
                                                     void* workspace, int64_t workspace_bytes,
                                                     void* stream) {
    nsh::NDims d;
    if (int rc = n_check("normalized_accumulate_uz_backward", S, B, C, H, W, dtype, &d)) return rc;
    dtype &= ~NSH_DTYPE_FLAGS;
    if (!x || !weights || !D || !log_C || !grad_D || !grad_log_C || !shifts || !grad_x || !grad_w)
        return fail(NSH_ERR_INVALID, "normalized_accumulate_uz_backward: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = workspace;
    const int64_t nws = workspace ? workspace_bytes : 0;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            return NSH_DISPATCH_LOGW(nsh::f16, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, ws, nws, st);
        case NSH_DTYPE_BFLOAT16:
            return NSH_DISPATCH_LOGW(nsh::bf16, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, ws, nws, st);
        case NSH_DTYPE_FLOAT32:
            return NSH_DISPATCH_LOGW(float, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, ws, nws, st);
        default:
            return NSH_DISPATCH_LOGW(double, n_run_bwd, x, weights, D, log_C, grad_D, grad_log_C, shifts, d, grad_x, grad_w, ws, nws, st);
    }
}
