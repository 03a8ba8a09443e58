// gather.hip -- shift_gather / pair_gather forward and backward on gfx950.
//
// Semantics (reference csrc/shift_ops_cuda.cu:61-246, ops.py:95-154):
//   gs[s*B+b, c, h, w]   = guide[b, c, (h+dx) mod H, (w+dy) mod W]
//   mask[s*B+b, 0, h, w] = box(h+dx, w+dy)           (in the guide dtype)
//   pair[s*B+b]          = cat(guide[b], gs[s*B+b]) on channels
//   backward: grad_guide[b,c,q] = sum_s g[s*B+b, c, (q-s) mod]  (+ centre half)
//
// The forward is write-bound: one workgroup fills a run of 16-byte output
// vectors of one output plane (every dtype is copied bit-exactly, no
// conversion), reading the small guide plane through L2.  When dy is a
// multiple of the vector width the source vector is contiguous and aligned
// and moves with one load; otherwise its elements are gathered one by one.
// The mask plane (s, b) is written by the c == 0 workgroups of that plane.
// The backward is gather-form: every lane owns VEC output elements, walks
// the S shifted planes and sums in the accumulator type, so it is
// deterministic and atomic-free (the reference pair backward used
// atomicAdd).
#include <initializer_list>
#include <type_traits>

#include "nsh_common.hpp"

namespace nsh {

constexpr int kGIter = 4;  // vectors per lane per workgroup

// Storage-type-agnostic element carrier for bit-exact copies.
template <int ES> struct Bits;
template <> struct Bits<2> { using type = uint16_t; };
template <> struct Bits<4> { using type = uint32_t; };
template <> struct Bits<8> { using type = uint64_t; };

template <int ES, int VEC, bool PAIR>
__global__ __launch_bounds__(kThreads) void gather_fwd_kernel(
    const typename Bits<ES>::type* __restrict__ guide, const int64_t* __restrict__ shifts,
    int cols, int B, int C, int H, int W, int64_t chunks, typename Bits<ES>::type* __restrict__ out,
    typename Bits<ES>::type* __restrict__ mask, typename Bits<ES>::type one) {
    using E = typename Bits<ES>::type;
    const int Cout = PAIR ? 2 * C : C;
    const int64_t plane = blockIdx.x / chunks;  // output plane (s*B+b)*Cout + co
    const int64_t chunk = blockIdx.x - plane * chunks;
    const int64_t sb = plane / Cout;
    const int co = static_cast<int>(plane - sb * Cout);
    const int64_t s = sb / B;
    const int64_t b = sb - s * B;
    const bool centre = PAIR && co < C;
    const int c = PAIR ? (co < C ? co : co - C) : co;

    const int64_t dx64 = shifts[s * cols + 0];
    const int64_t dy64 = shifts[s * cols + 1];
    const int dxm = static_cast<int>(mod_pos(dx64, H));
    const int dym = static_cast<int>(mod_pos(dy64, W));
    const int dxc = clamp_shift(dx64);
    const int dyc = clamp_shift(dy64);
    const int sx = centre ? 0 : dxm;
    const int sy = centre ? 0 : dym;
    const bool vec_src = (sy % VEC) == 0;

    const int64_t HW = static_cast<int64_t>(H) * W;
    const E* g = guide + (b * C + c) * HW;
    E* o = out + plane * HW;
    E* m = (mask != nullptr && co == 0) ? mask + sb * HW : nullptr;
    const int WV = W / VEC;  // vectors per row
    const int64_t nvec = static_cast<int64_t>(H) * WV;

#pragma unroll
    for (int it = 0; it < kGIter; ++it) {
        const int64_t i = (chunk * kGIter + it) * kThreads + threadIdx.x;
        if (i >= nvec) break;
        const int h = static_cast<int>(i / WV);
        const int w0 = static_cast<int>(i - static_cast<int64_t>(h) * WV) * VEC;
        int hh = h + sx;
        hh -= hh >= H ? H : 0;
        const E* row = g + static_cast<uint32_t>(hh) * W;
        Pack<E, VEC> v;
        if (vec_src) {
            int ww = w0 + sy;
            ww -= ww >= W ? W : 0;
            v = load_pack<E, VEC>(row + ww);
        } else {
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int ww = w0 + k + sy;
                ww -= ww >= W ? W : 0;
                v.e[k] = row[ww];
            }
        }
        store_pack_nt<E, VEC>(o + static_cast<uint32_t>(h) * W + w0, v);
        if (m != nullptr) {
            const bool rok = in_range(h + dxc, H);
            Pack<E, VEC> mv;
#pragma unroll
            for (int k = 0; k < VEC; ++k) mv.e[k] = (rok && in_range(w0 + k + dyc, W)) ? one : E(0);
            store_pack_nt<E, VEC>(m + static_cast<uint32_t>(h) * W + w0, mv);
        }
    }
}

template <typename T, int VEC, bool PAIR>
__global__ __launch_bounds__(kThreads) void gather_bwd_kernel(
    const T* __restrict__ gout, const int64_t* __restrict__ shifts, int cols, int S, int B, int C,
    int H, int W, int64_t chunks, T* __restrict__ grad) {
    using A = acc_t<T>;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    stage_shifts(shl, shifts, S, cols, H, W, false);

    const int64_t bc = blockIdx.x / chunks;
    const int64_t chunk = blockIdx.x - bc * chunks;
    const int64_t b = bc / C;
    const int64_t c = bc - b * C;
    const int Cout = PAIR ? 2 * C : C;
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t plane_step = static_cast<int64_t>(B) * Cout * HW;  // next shift, same (b, c)
    const int WV = W / VEC;
    const int64_t nvec = static_cast<int64_t>(H) * WV;

#pragma unroll 1
    for (int it = 0; it < kGIter; ++it) {
        const int64_t i = (chunk * kGIter + it) * kThreads + threadIdx.x;
        if (i >= nvec) break;
        const int h = static_cast<int>(i / WV);
        const int w0 = static_cast<int>(i - static_cast<int64_t>(h) * WV) * VEC;
        const uint32_t own = static_cast<uint32_t>(h) * W + w0;
        A acc[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] = A(0);
        const T* gp = gout + (b * Cout + (PAIR ? C + c : c)) * HW;  // shifted half, shift 0
        const T* cp = gout + (b * Cout + c) * HW;                   // centre half (pair only)
        for (int s = 0; s < S; ++s, gp += plane_step, cp += plane_step) {
            const ShiftRec r = read_shift(shl, s);
            if (PAIR) {
                A cv[VEC];
                load_acc<T, VEC>(cp + own, cv);
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[k] += cv[k];
            }
            int hm = h - r.dxm;
            hm += hm < 0 ? H : 0;
            const T* row = gp + static_cast<uint32_t>(hm) * W;
            if ((r.dym % VEC) == 0) {
                int wm = w0 - r.dym;
                wm += wm < 0 ? W : 0;
                A v[VEC];
                load_acc<T, VEC>(row + wm, v);
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc[k] += v[k];
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    int wm = w0 + k - r.dym;
                    wm += wm < 0 ? W : 0;
                    acc[k] += to_acc(row[wm]);
                }
            }
        }
        store_acc<T, VEC>(grad + bc * HW + own, acc, false);
    }
}

// ---------------------------------------------------------------------------
// Tiled kernels (16-byte vectors, W a multiple of the vector width).
//
// A workgroup owns a tile of kGTH rows x TW columns of one (b, c) plane and
// walks all S shifts.  The forward stages the guide tile with a kRmax halo
// (circularly wrapped) in LDS once, then writes every shift's output tile
// with aligned 16-byte stores read from the LDS tile at the shifted offset
// (plus the pair's centre copy and, from the c == 0 workgroup, the mask).
// The backward stages, per shift, the rows (h - dx) mod H of the shifted
// gradient plane over columns [w0 - kRmax, w0 + TW + kRmax) with aligned
// loads (double-buffered: the next shift's loads are in flight while this
// one is summed), so every gradient element is read once (plus the 2 kRmax
// column halo) and summed from LDS.  Shifts beyond the LDS halo take an
// element-wise path in a separate loop.
// ---------------------------------------------------------------------------
constexpr int kGTH = 8;       // tile rows
constexpr int kGTWMax = 256;  // tile columns (elements)

__device__ __forceinline__ int wrap_any(int v, int n) {
    v %= n;
    return v < 0 ? v + n : v;
}

template <int ES, int VEC, bool PAIR>
__global__ __launch_bounds__(kThreads) void gather_fwd_tile_kernel(
    const typename Bits<ES>::type* __restrict__ guide, const int64_t* __restrict__ shifts,
    int cols, int S, int B, int C, int H, int W, int TW, int ntw, int nth,
    typename Bits<ES>::type* __restrict__ out, typename Bits<ES>::type* __restrict__ mask,
    typename Bits<ES>::type one) {
    using E = typename Bits<ES>::type;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    E* lt = reinterpret_cast<E*>(smem + shift_lds_bytes(S));
    const int LP = TW + 2 * kRmax;
    const int LR = kGTH + 2 * kRmax;

    const int64_t per_plane = static_cast<int64_t>(ntw) * nth;
    const int64_t bc = blockIdx.x / per_plane;
    const int rem = static_cast<int>(blockIdx.x - bc * per_plane);
    const int h0 = (rem / ntw) * kGTH;
    const int w0 = (rem % ntw) * TW;
    const int64_t b = bc / C;
    const int c = static_cast<int>(bc - b * C);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const E* g = guide + bc * HW;

    stage_shifts(shl, shifts, S, cols, H, W, false);
    const int LV = LP / VEC;
    for (int i = threadIdx.x; i < LR * LV; i += blockDim.x) {
        const int r = i / LV;
        const int jv = i - r * LV;
        const int gh = wrap_any(h0 - kRmax + r, H);
        const int gw = wrap_any(w0 - kRmax + jv * VEC, W);  // a vector never straddles the wrap
        store_pack<E, VEC>(lt + r * LP + jv * VEC,
                           load_pack<E, VEC>(g + static_cast<uint32_t>(gh) * W + gw));
    }
    __syncthreads();

    const int th = min(kGTH, H - h0);
    const int tw = min(TW, W - w0);
    const int TV = TW / VEC;
    const int Cout = PAIR ? 2 * C : C;
    // The lane's vectors of the tile (the same for every shift): row, column
    // and LDS index computed once, outside the shift loop.
    constexpr int NI = (kGTH * kGTWMax / VEC + kThreads - 1) / kThreads;
    bool act[NI];
    int hk[NI], wk[NI], lk[NI];
#pragma unroll
    for (int n = 0; n < NI; ++n) {
        const int i = static_cast<int>(threadIdx.x) + n * kThreads;
        const int row = i / TV;
        const int vc = i - row * TV;
        act[n] = i < kGTH * TV && row < th && vc * VEC < tw;
        hk[n] = h0 + row;
        wk[n] = w0 + vc * VEC;
        lk[n] = (row + kRmax) * LP + vc * VEC + kRmax;  // LDS index of the unshifted vector
    }
    for (int s = 0; s < S; ++s) {
        const ShiftRec rc = read_shift(shl, s);
        const bool near = shift_in_lds(rc);
        const bool aligned = (rc.dy % VEC) == 0;
        const int64_t sb = static_cast<int64_t>(s) * B + b;
        E* op = out + (sb * Cout + (PAIR ? C + c : c)) * HW;
        E* cp = PAIR ? out + (sb * Cout + c) * HW : nullptr;
        E* mp = (mask != nullptr && c == 0) ? mask + sb * HW : nullptr;
        const int lsh = rc.dx * LP + rc.dy;  // LDS offset of the shifted vector
#pragma unroll
        for (int n = 0; n < NI; ++n) {
            if (!act[n]) continue;
            const int h = hk[n];
            const int w = wk[n];
            const uint32_t o = static_cast<uint32_t>(h) * W + w;
            Pack<E, VEC> v;
            if (near) {
                const E* src = lt + lk[n] + lsh;
                if (aligned) {
                    v = load_pack<E, VEC>(src);
                } else {
#pragma unroll
                    for (int k = 0; k < VEC; ++k) v.e[k] = src[k];
                }
            } else {
                int hh = h + rc.dxm;
                hh -= hh >= H ? H : 0;
                const E* row_p = g + static_cast<uint32_t>(hh) * W;
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    int ww = w + k + rc.dym;
                    ww -= ww >= W ? W : 0;
                    v.e[k] = row_p[ww];
                }
            }
            store_pack_nt<E, VEC>(op + o, v);
            if (PAIR)
                store_pack_nt<E, VEC>(cp + o, load_pack<E, VEC>(lt + lk[n]));
            if (mp != nullptr) {
                const bool rok = in_range(h + rc.dx, H);
                Pack<E, VEC> mv;
#pragma unroll
                for (int k = 0; k < VEC; ++k) mv.e[k] = (rok && in_range(w + k + rc.dy, W)) ? one : E(0);
                store_pack_nt<E, VEC>(mp + o, mv);
            }
        }
    }
}

// Gradient-stack loads of the tiled pair backward as nontemporal (streaming)
// loads: c1 pair backward 0.074 -> 0.070 ms (box) and 0.140 -> 0.131 ms
// (periodic); the shift_gather backward keeps plain loads (0.055 -> 0.065 ms
// with streaming ones).
constexpr bool kGatherPairNtLoads = true;

// NL: window vectors per lane per shift; NV: output vectors per lane.
template <typename T, int VEC, bool PAIR, int NL, int NV>
__global__ __launch_bounds__(kThreads) void gather_bwd_tile_kernel(
    const T* __restrict__ gout, const int64_t* __restrict__ shifts, int cols, int S, int B, int C,
    int H, int W, int TW, int ntw, int nth, T* __restrict__ grad) {
    using A = acc_t<T>;
    using E = typename Bits<sizeof(T)>::type;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    const int LP = TW + 2 * kRmax;
    E* buf0 = reinterpret_cast<E*>(smem + shift_lds_bytes(S));
    E* buf1 = buf0 + kGTH * LP;

    const int64_t per_plane = static_cast<int64_t>(ntw) * nth;
    const int64_t bc = blockIdx.x / per_plane;
    const int rem = static_cast<int>(blockIdx.x - bc * per_plane);
    const int h0 = (rem / ntw) * kGTH;
    const int w0 = (rem % ntw) * TW;
    const int64_t b = bc / C;
    const int64_t c = bc - b * C;
    const int Cout = PAIR ? 2 * C : C;
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t plane_step = static_cast<int64_t>(B) * Cout * HW;  // next shift, same (b, c)
    const E* g0 = reinterpret_cast<const E*>(gout) + (b * Cout + (PAIR ? C + c : c)) * HW;
    const E* c0 = reinterpret_cast<const E*>(gout) + (b * Cout + c) * HW;  // centre half (pair)

    stage_shifts(shl, shifts, S, cols, H, W, false);
    const int th = min(kGTH, H - h0);
    const int tw = min(TW, W - w0);
    const int LV = LP / VEC;
    const int TV = TW / VEC;

    // own output vectors
    int orow[NV], ocol[NV];
    bool oact[NV];
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int i = threadIdx.x + n * kThreads;
        orow[n] = i / TV;
        ocol[n] = (i - orow[n] * TV) * VEC;
        oact[n] = i < kGTH * TV && orow[n] < th && ocol[n] < tw;
    }
    A acc[NV][VEC];
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[n][k] = A(0);

    // The lane's window vectors (the same for every shift): LDS index,
    // source column (wrapped) and unshifted source row (wrapped; rows beyond
    // the tile clamp to its last row), computed once outside the shift loop.
    int wl[NL], wcol[NL], wrow[NL];
    bool wact[NL];
#pragma unroll
    for (int n = 0; n < NL; ++n) {
        const int i = threadIdx.x + n * kThreads;
        const int r = i / LV;
        const int jv = i - r * LV;
        wact[n] = i < kGTH * LV;
        wl[n] = r * LP + jv * VEC;
        wcol[n] = wrap_any(w0 - kRmax + jv * VEC, W);
        wrow[n] = wrap_any(h0 + min(r, kGTH - 1), H);
    }
    constexpr bool kGatherNtLoads = PAIR && kGatherPairNtLoads;
    // window vector i of shift s: row r (output row h0 + r reads source row
    // (h0 + r - dx) mod H), columns [w0 - kRmax + jv*VEC, +VEC) mod W.
    // Two register slots keep the loads of two shifts in flight: the loads
    // of shift s + 2 are issued as shift s is summed (the loop is unrolled
    // by two so that the slot index is a compile-time constant).
    Pack<E, VEC> pf[2][NL];
    Pack<E, VEC> cf[2][NV];
    auto issue = [&](int s, auto slot_tag) {
        constexpr int SL = decltype(slot_tag)::value;
        const ShiftRec rc = read_shift(shl, s);
        const E* gp = g0 + static_cast<int64_t>(s) * plane_step;
#pragma unroll
        for (int n = 0; n < NL; ++n) {
            int gh = wrow[n] - rc.dxm;  // (row - dx) mod H, dxm = dx mod H in [0, H)
            gh += gh < 0 ? H : 0;
            const int gw = wcol[n];
            pf[SL][n] = kGatherNtLoads
                            ? load_pack_nt<E, VEC>(gp + static_cast<uint32_t>(gh) * W + gw)
                            : load_pack<E, VEC>(gp + static_cast<uint32_t>(gh) * W + gw);
        }
        if (PAIR) {
            const E* cpp = c0 + static_cast<int64_t>(s) * plane_step;
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                const int h = h0 + (oact[n] ? orow[n] : 0);
                const int w = w0 + (oact[n] ? ocol[n] : 0);
                cf[SL][n] = kGatherNtLoads
                                ? load_pack_nt<E, VEC>(cpp + static_cast<uint32_t>(h) * W + w)
                                : load_pack<E, VEC>(cpp + static_cast<uint32_t>(h) * W + w);
            }
        }
    };
    auto body = [&](int s, auto slot_tag) {
        constexpr int SL = decltype(slot_tag)::value;
        E* bw = SL ? buf1 : buf0;
#pragma unroll
        for (int n = 0; n < NL; ++n)
            if (wact[n]) store_pack<E, VEC>(bw + wl[n], pf[SL][n]);
        if (PAIR) {
#pragma unroll
            for (int n = 0; n < NV; ++n)
#pragma unroll
                for (int k = 0; k < VEC; ++k)
                    acc[n][k] += to_acc(__builtin_bit_cast(T, cf[SL][n].e[k]));
        }
        // LDS-only barrier (the other slot's loads stay in flight), then the
        // refill issued unconditionally (the tail re-reads plane S-1): a
        // conditional refill made the compiler's wait counts drain both slots.
        lds_barrier();
        issue(min(s + 2, S - 1), slot_tag);
        const ShiftRec rc = read_shift(shl, s);
        if (rc.dy >= -kRmax && rc.dy <= kRmax) {
            const bool aligned = (rc.dy % VEC) == 0;
#pragma unroll
            for (int n = 0; n < NV; ++n) {
                const E* src = bw + orow[n] * LP + ocol[n] + kRmax - rc.dy;
                if (!oact[n]) continue;
                if (aligned) {
                    const Pack<E, VEC> v = load_pack<E, VEC>(src);
#pragma unroll
                    for (int k = 0; k < VEC; ++k) acc[n][k] += to_acc(__builtin_bit_cast(T, v.e[k]));
                } else {
#pragma unroll
                    for (int k = 0; k < VEC; ++k) acc[n][k] += to_acc(__builtin_bit_cast(T, src[k]));
                }
            }
        }
    };
    using Slot0 = std::integral_constant<int, 0>;
    using Slot1 = std::integral_constant<int, 1>;
    if (S > 0) issue(0, Slot0{});
    if (S > 1) issue(1, Slot1{});
    // whole pairs, then an odd last shift (no conditional inside the loop:
    // the wait counts stay exact and keep the other slot in flight)
    int s_pair = 0;
    for (; s_pair + 1 < S; s_pair += 2) {
        body(s_pair, Slot0{});
        body(s_pair + 1, Slot1{});
    }
    if (s_pair < S) body(s_pair, Slot0{});
    // Shifts beyond the column halo: element-wise from HBM.
    for (int s = 0; s < S; ++s) {
        const ShiftRec rc = read_shift(shl, s);
        if (rc.dy >= -kRmax && rc.dy <= kRmax) continue;
        const E* gp = g0 + static_cast<int64_t>(s) * plane_step;
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            if (!oact[n]) continue;
            int hm = h0 + orow[n] - rc.dxm;
            hm += hm < 0 ? H : 0;
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                int wm = w0 + ocol[n] + k - rc.dym;
                wm += wm < 0 ? W : 0;
                acc[n][k] += to_acc(__builtin_bit_cast(T, gp[static_cast<uint32_t>(hm) * W + wm]));
            }
        }
    }
    T* gr = grad + bc * HW;
#pragma unroll
    for (int n = 0; n < NV; ++n)
        if (oact[n])
            store_acc<T, VEC>(gr + static_cast<uint32_t>(h0 + orow[n]) * W + w0 + ocol[n], acc[n],
                              false);
}

template <int ES>
static int pick_copy_vec(int W, std::initializer_list<const void*> ptrs) {
    for (int v = 16 / ES; v > 1; v /= 2) {
        if (W % v) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && (p == nullptr || nsh_host::aligned(p, v * ES));
        if (ok) return v;
    }
    return 1;
}

template <int ES, int VEC, bool PAIR>
static int g_fwd_launch(const void* guide, const int64_t* sh, int cols, int S, int B, int C, int H,
                        int W, void* out, void* mask, uint64_t one_bits, hipStream_t st) {
    using E = typename Bits<ES>::type;
    const int64_t nvec = static_cast<int64_t>(H) * (W / VEC);
    const int64_t chunks = nsh_host::ceil_div(nvec, static_cast<int64_t>(kThreads) * kGIter);
    const int64_t planes = static_cast<int64_t>(S) * B * (PAIR ? 2 * C : C);
    const int64_t blocks = planes * chunks;
    if (blocks > 0x7fffffff) return nsh_host::fail(NSH_ERR_INVALID, "gather: grid too large");
    hipLaunchKernelGGL((gather_fwd_kernel<ES, VEC, PAIR>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kThreads), 0, st, static_cast<const E*>(guide), sh, cols, B, C, H, W,
                       chunks, static_cast<E*>(out), static_cast<E*>(mask),
                       static_cast<E>(one_bits));
    return nsh_host::check_launch(PAIR ? "pair_gather_forward" : "shift_gather_forward");
}

// Tiled path: 16-byte vectors, W a multiple of the vector width, aligned
// pointers, S <= 1024 (the shift table lives in LDS).
static bool g_tile_ok(int S, int W, int vec, std::initializer_list<const void*> ptrs) {
    if (S > 1024 || W % vec) return false;
    for (const void* p : ptrs)
        if (p != nullptr && !nsh_host::aligned(p, 16)) return false;
    return true;
}

template <int ES, bool PAIR>
static int g_fwd_tile(const void* guide, const int64_t* sh, int cols, int S, int B, int C, int H,
                      int W, void* out, void* mask, uint64_t one_bits, hipStream_t st) {
    using E = typename Bits<ES>::type;
    constexpr int VEC = 16 / ES;
    const int TW = W < kGTWMax ? W : kGTWMax;
    const int ntw = static_cast<int>(nsh_host::ceil_div(W, TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(H, kGTH));
    const int64_t blocks = static_cast<int64_t>(B) * C * ntw * nth;
    if (blocks > 0x7fffffff) return nsh_host::fail(NSH_ERR_INVALID, "gather: grid too large");
    const size_t lds = shift_lds_bytes(S) +
                       static_cast<size_t>(kGTH + 2 * kRmax) * (TW + 2 * kRmax) * ES;
    hipLaunchKernelGGL((gather_fwd_tile_kernel<ES, VEC, PAIR>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kThreads), lds, st, static_cast<const E*>(guide), sh, cols, S, B, C, H,
                       W, TW, ntw, nth, static_cast<E*>(out), static_cast<E*>(mask),
                       static_cast<E>(one_bits));
    return nsh_host::check_launch(PAIR ? "pair_gather_forward" : "shift_gather_forward");
}

template <typename T, bool PAIR>
static int g_bwd_tile(const void* gout, const int64_t* sh, int cols, int S, int B, int C, int H,
                      int W, void* grad, hipStream_t st) {
    constexpr int VEC = 16 / static_cast<int>(sizeof(T));
    constexpr int NL = (kGTH * (kGTWMax + 2 * kRmax) / VEC + kThreads - 1) / kThreads;
    constexpr int NV = (kGTH * kGTWMax / VEC + kThreads - 1) / kThreads;
    const int TW = W < kGTWMax ? W : kGTWMax;
    const int ntw = static_cast<int>(nsh_host::ceil_div(W, TW));
    const int nth = static_cast<int>(nsh_host::ceil_div(H, kGTH));
    const int64_t blocks = static_cast<int64_t>(B) * C * ntw * nth;
    if (blocks > 0x7fffffff) return nsh_host::fail(NSH_ERR_INVALID, "gather backward: grid too large");
    const size_t lds = shift_lds_bytes(S) +
                       2 * static_cast<size_t>(kGTH) * (TW + 2 * kRmax) * sizeof(T);
    hipLaunchKernelGGL((gather_bwd_tile_kernel<T, VEC, PAIR, NL, NV>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, st,
                       static_cast<const T*>(gout), sh, cols, S, B, C, H, W, TW, ntw, nth,
                       static_cast<T*>(grad));
    return nsh_host::check_launch(PAIR ? "pair_gather_backward" : "shift_gather_backward");
}

template <int ES, bool PAIR>
static int g_fwd(const void* guide, const int64_t* sh, int cols, int S, int B, int C, int H, int W,
                 void* out, void* mask, uint64_t one_bits, hipStream_t st) {
    if (g_tile_ok(S, W, 16 / ES, {guide, out, mask}))
        return g_fwd_tile<ES, PAIR>(guide, sh, cols, S, B, C, H, W, out, mask, one_bits, st);
    switch (pick_copy_vec<ES>(W, {guide, out, mask})) {
        case 8: if constexpr (ES == 2) return g_fwd_launch<ES, 8, PAIR>(guide, sh, cols, S, B, C, H, W, out, mask, one_bits, st); break;
        case 4: if constexpr (ES <= 4) return g_fwd_launch<ES, 4, PAIR>(guide, sh, cols, S, B, C, H, W, out, mask, one_bits, st); break;
        case 2: return g_fwd_launch<ES, 2, PAIR>(guide, sh, cols, S, B, C, H, W, out, mask, one_bits, st);
        default: break;
    }
    return g_fwd_launch<ES, 1, PAIR>(guide, sh, cols, S, B, C, H, W, out, mask, one_bits, st);
}

template <typename T, int VEC, bool PAIR>
static int g_bwd_launch(const void* gout, const int64_t* sh, int cols, int S, int B, int C, int H,
                        int W, void* grad, hipStream_t st) {
    const int64_t nvec = static_cast<int64_t>(H) * (W / VEC);
    const int64_t chunks = nsh_host::ceil_div(nvec, static_cast<int64_t>(kThreads) * kGIter);
    const int64_t blocks = static_cast<int64_t>(B) * C * chunks;
    if (blocks > 0x7fffffff) return nsh_host::fail(NSH_ERR_INVALID, "gather backward: grid too large");
    hipLaunchKernelGGL((gather_bwd_kernel<T, VEC, PAIR>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kThreads), shift_lds_bytes(S), st,
                       static_cast<const T*>(gout), sh, cols, S, B, C, H, W, chunks,
                       static_cast<T*>(grad));
    return nsh_host::check_launch(PAIR ? "pair_gather_backward" : "shift_gather_backward");
}

template <typename T, bool PAIR>
static int g_bwd(const void* gout, const int64_t* sh, int cols, int S, int B, int C, int H, int W,
                 void* grad, hipStream_t st) {
    if (g_tile_ok(S, W, 16 / static_cast<int>(sizeof(T)), {gout, grad}))
        return g_bwd_tile<T, PAIR>(gout, sh, cols, S, B, C, H, W, grad, st);
    switch (pick_copy_vec<sizeof(T)>(W, {gout, grad})) {
        case 8: if constexpr (sizeof(T) == 2) return g_bwd_launch<T, 8, PAIR>(gout, sh, cols, S, B, C, H, W, grad, st); break;
        case 4: if constexpr (sizeof(T) <= 4) return g_bwd_launch<T, 4, PAIR>(gout, sh, cols, S, B, C, H, W, grad, st); break;
        case 2: return g_bwd_launch<T, 2, PAIR>(gout, sh, cols, S, B, C, H, W, grad, st);
        default: break;
    }
    return g_bwd_launch<T, 1, PAIR>(gout, sh, cols, S, B, C, H, W, grad, st);
}

}  // namespace nsh

using nsh_host::fail;

static int g_check(const char* op, int64_t S, int64_t cols, int64_t B, int64_t C, int64_t H,
                   int64_t W, int dtype, bool bwd) {
    if (S < 0) return fail(NSH_ERR_INVALID, "%s: negative shift count", op);
    if (bwd && S > 1024) return fail(NSH_ERR_INVALID, "%s: requires S <= 1024", op);
    if (cols != 2 && cols != 3) return fail(NSH_ERR_INVALID, "%s: shifts must have 2 or 3 columns", op);
    if (B < 0 || C < 0 || H < 1 || W < 1) return fail(NSH_ERR_INVALID, "%s: bad tensor shape", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (S * B * 2 * C > (int64_t(1) << 31)) return fail(NSH_ERR_INVALID, "%s: S*B*C too large", op);
    return NSH_OK;
}

static uint64_t one_bits(int dtype) {
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return 0x3C00u;
        case NSH_DTYPE_BFLOAT16: return 0x3F80u;
        case NSH_DTYPE_FLOAT32: return 0x3F800000u;
        default: return 0x3FF0000000000000ull;
    }
}

template <bool PAIR>
static int gather_forward(const char* op, const void* guide, const int64_t* shifts, int64_t S,
                          int64_t cols, int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                          void* out, void* mask, void* stream) {
    if (int rc = g_check(op, S, cols, B, C, H, W, dtype, false)) return rc;
    if (S == 0 || B == 0 || C == 0) return NSH_OK;
    if (!guide || !shifts || !out) return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int s = static_cast<int>(S), c = static_cast<int>(cols), b = static_cast<int>(B);
    const int ch = static_cast<int>(C), h = static_cast<int>(H), w = static_cast<int>(W);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
        case NSH_DTYPE_BFLOAT16:
            return nsh::g_fwd<2, PAIR>(guide, shifts, c, s, b, ch, h, w, out, mask, one_bits(dtype), st);
        case NSH_DTYPE_FLOAT32:
            return nsh::g_fwd<4, PAIR>(guide, shifts, c, s, b, ch, h, w, out, mask, one_bits(dtype), st);
        default:
            return nsh::g_fwd<8, PAIR>(guide, shifts, c, s, b, ch, h, w, out, mask, one_bits(dtype), st);
    }
}

template <bool PAIR>
static int gather_backward(const char* op, const void* gout, const int64_t* shifts, int64_t S,
                           int64_t cols, int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                           void* grad, void* stream) {
    if (int rc = g_check(op, S, cols, B, C, H, W, dtype, true)) return rc;
    if (B == 0 || C == 0) return NSH_OK;
    // S == 0 runs the same kernel with an empty shift loop: it writes zeros.
    if (!grad || (S > 0 && (!gout || !shifts)))
        return fail(NSH_ERR_INVALID, "%s: null pointer argument", op);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int s = static_cast<int>(S), c = static_cast<int>(cols), b = static_cast<int>(B);
    const int ch = static_cast<int>(C), h = static_cast<int>(H), w = static_cast<int>(W);
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::g_bwd<nsh::f16, PAIR>(gout, shifts, c, s, b, ch, h, w, grad, st);
        case NSH_DTYPE_BFLOAT16: return nsh::g_bwd<nsh::bf16, PAIR>(gout, shifts, c, s, b, ch, h, w, grad, st);
        case NSH_DTYPE_FLOAT32: return nsh::g_bwd<float, PAIR>(gout, shifts, c, s, b, ch, h, w, grad, st);
        default: return nsh::g_bwd<double, PAIR>(gout, shifts, c, s, b, ch, h, w, grad, st);
    }
}

extern "C" int nsh_shift_gather_forward(const void* guide, const int64_t* shifts, int64_t S,
                                        int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                        int64_t W, int dtype, void* out, void* mask, void* stream) {
    return gather_forward<false>("shift_gather", guide, shifts, S, shift_cols, B, C, H, W, dtype,
                                 out, mask, stream);
}

extern "C" int nsh_pair_gather_forward(const void* guide, const int64_t* shifts, int64_t S,
                                       int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                       int64_t W, int dtype, void* out, void* mask, void* stream) {
    return gather_forward<true>("pair_gather", guide, shifts, S, shift_cols, B, C, H, W, dtype, out,
                                mask, stream);
}

extern "C" int nsh_shift_gather_backward(const void* grad_out, const int64_t* shifts, int64_t S,
                                         int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                         int64_t W, int dtype, void* grad_guide, void* stream) {
    return gather_backward<false>("shift_gather_backward", grad_out, shifts, S, shift_cols, B, C, H,
                                  W, dtype, grad_guide, stream);
}

extern "C" int nsh_pair_gather_backward(const void* grad_out, const int64_t* shifts, int64_t S,
                                        int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                        int64_t W, int dtype, void* grad_guide, void* stream) {
    return gather_backward<true>("pair_gather_backward", grad_out, shifts, S, shift_cols, B, C, H, W,
                                 dtype, grad_guide, stream);
}
