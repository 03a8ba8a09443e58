// scatter.hpp -- shared pieces of the scatter-form kernels (accumulate_uz,
// metropolis_aggregate) on gfx950.
//
// A scatter kernel's lane that owns pixel q reads its weight w_s[q] once,
// aligned, and adds the term it contributes to pixel q + s into an LDS
// accumulator window covering its tile plus a HALO border (kRmax = 8, or 16
// for the accumulate_uz instantiations that serve wider tables).  After the
// shift
// loop the window's border (targets outside the tile) is written to a
// per-tile spill block in a workspace; a fix-up launch then adds, for every
// pixel within R of its tile's edge, the spills of the (up to 8) neighbouring
// tiles in a fixed order.  Neighbour tiles wrap around the image (torus), so
// circular targets are covered as well as box-masked ones.
#pragma once

#include "nsh_common.hpp"

namespace nsh {

// Whether any row of the staged table carries the forward box (row code 4);
// uniform across the workgroup.
__device__ __forceinline__ bool table_any_fbox(const int4* shl, int S) {
    const int lane = threadIdx.x & 63;
    int any = 0;
    for (int s = lane; s < S; s += 64) any |= (shl[s].z & 0x40000000) != 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) any |= __shfl_xor(any, o, 64);
    return __builtin_amdgcn_readfirstlane(any) != 0;
}

// Largest max(|dx|, |dy|) over the table rows (only has_inverse rows when
// `only_inv`); computed by every wave from the staged table, so the result
// is uniform across the workgroup without a barrier.
__device__ __forceinline__ int table_radius(const int4* shl, int S, bool only_inv) {
    const int lane = threadIdx.x & 63;
    int m = 0;
    for (int s = lane; s < S; s += 64) {
        const int4 r = shl[s];
        if (only_inv && r.z >= 0) continue;
        const int ax = r.x < 0 ? -r.x : r.x;
        const int ay = r.y < 0 ? -r.y : r.y;
        m = max(m, max(ax, ay));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    return __builtin_amdgcn_readfirstlane(m);
}

// Spill block of a th x tw tile with an R border: the top R rows and bottom
// R rows of the (th+2R) x (tw+2R) window, then the left and right R columns
// of the middle th rows.  (i, j) are window coordinates relative to the tile
// origin.
__device__ __forceinline__ int spill_count(int th, int tw, int R) {
    return 2 * R * (tw + 2 * R) + 2 * R * th;
}

__device__ __forceinline__ int spill_index(int i, int j, int th, int tw, int R) {
    const int ww = tw + 2 * R;
    if (i < 0) return (i + R) * ww + (j + R);
    if (i >= th) return R * ww + (i - th) * ww + (j + R);
    return 2 * R * ww + i * 2 * R + (j < 0 ? j + R : R + (j - tw));
}

__device__ __forceinline__ void spill_coords(int e, int th, int tw, int R, int& i, int& j) {
    const int ww = tw + 2 * R;
    const int band = R * ww;
    if (e < band) {
        i = e / ww - R;
        j = e - (i + R) * ww - R;
        return;
    }
    e -= band;
    if (e < band) {
        const int r = e / ww;
        i = th + r;
        j = e - r * ww - R;
        return;
    }
    e -= band;
    i = e / (2 * R);
    const int c = e - i * 2 * R;
    j = c < R ? c - R : tw + (c - R);
}

// Scatter-path tile: TPR lanes across, ROWS rows down, one row per lane;
// lane tx owns the VEC pixels tx, tx + TPR, ... of its row (strided), so
// every LDS access of a wave covers TPR consecutive words per row.  The
// image tiles and the accumulator windows carry a HALO border and share a
// row pitch congruent to 16 words mod 32, so the two rows of a half-wave
// (TPR = 16) fall on disjoint banks.  A wave owns 64 / TPR whole tile rows.
// STRIDED = false is the contiguous variant (lane tx owns pixels
// tx*VEC .. tx*VEC + VEC-1, moved with one 16-byte access) with an odd
// pitch; its LDS reads of a wave are 4-way strided.
template <int VEC, int ROWS, int TPR, bool STRIDED = true, int HALO = kRmax>
struct SGeo {
    static_assert(64 % TPR == 0, "a wave must own whole tile rows");
    static_assert(HALO >= 1 && HALO <= kMaxHalo, "halo beyond the fix-up's slot rows");
    static constexpr int THREADS = TPR * ROWS;
    static constexpr int TW = TPR * VEC;
    static constexpr int TH = ROWS;
    static constexpr int LW = TW + 2 * HALO;
    static constexpr int LH = TH + 2 * HALO;
    static constexpr int PITCH = STRIDED ? LW + ((16 - LW % 32) + 32) % 32 : LW + 1;
    // Contiguous lanes with VEC 2 or 4 store de-interleaved rows (BwdLayout)
    // at a pitch congruent to 16 mod 32, which can exceed LW + 1.
    static constexpr int DI_PITCH =
        (!STRIDED && (VEC == 2 || VEC == 4)) ? LW + ((16 - LW % 32) + 32) % 32 : 0;
    static constexpr int TILE = LH * (PITCH > DI_PITCH ? PITCH : DI_PITCH);
    // spill block stride (entries), sized for the largest border
    static constexpr int SPILL = 2 * HALO * (TW + 2 * HALO) + 2 * HALO * TH;
    // own ring partials (entries): >= ring_count of any tile
    static constexpr int RING = 2 * HALO * (TW + TH);
};

// Column layout of the LDS tiles read by contiguous lanes.  With VEC > 1 a
// lane owns VEC consecutive pixels, so in a plain row-major tile the lanes of
// a wave would read words VEC apart (VEC-way bank conflicts on every access).
// The tiles are instead stored de-interleaved by column mod VEC: tile column
// j lives at (j % VEC) * QW + j / VEC of its row (QW = LW / VEC).  For a
// given shift and pixel k the class j % VEC is the same for all lanes, so the
// lanes read consecutive words, and col(VEC * tx + c) = tx + col(c) for
// c >= 0; the global loads and stores stay VEC-element vectors.
template <int VEC, int LW, int PITCH_LINEAR>
struct BwdLayout {
    static constexpr bool DI = VEC == 2 || VEC == 4;
    static constexpr int QW = LW / VEC;  // LW = TPR * VEC + 2 * HALO
    static constexpr int PITCH =
        DI ? LW + ((16 - LW % 32) + 32) % 32 : PITCH_LINEAR;  // 16 mod 32 (see SGeo)
    static_assert(!DI || LW % VEC == 0, "de-interleaved rows need LW divisible by VEC");
    // offset of tile column j within its row
    __device__ static constexpr int col(int j) { return DI ? (j % VEC) * QW + j / VEC : j; }
};

// &base[idx] with the byte offset formed in 32 bits (an in-plane offset is
// below 2^31 bytes), so the address is a uniform base plus a 32-bit lane
// offset: one VGPR per address instead of a 64-bit pair.
template <typename T>
__device__ __forceinline__ const T* elem_ptr(const T* base, uint32_t idx) {
    return reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) +
                                      static_cast<uint32_t>(idx * sizeof(T)));
}
template <typename T>
__device__ __forceinline__ T* elem_ptr(T* base, uint32_t idx) {
    return reinterpret_cast<T*>(reinterpret_cast<char*>(base) +
                                static_cast<uint32_t>(idx * sizeof(T)));
}

// The lane's pixels: activity and in-plane offsets (inactive pixels point at
// the plane's first element so that their loads stay in bounds).
template <int VEC, int TPR>
struct LanePix {
    bool act[VEC];
    uint32_t own[VEC];
    int any;
};

template <int VEC, int TPR>
__device__ __forceinline__ LanePix<VEC, TPR> lane_pixels(int h, int w0, int tx, int H, int W) {
    LanePix<VEC, TPR> l;
    l.any = 0;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const int w = w0 + tx + k * TPR;
        l.act[k] = h < H && w < W;
        l.own[k] = l.act[k] ? static_cast<uint32_t>(h) * static_cast<uint32_t>(W) +
                                  static_cast<uint32_t>(w)
                            : 0u;
        l.any |= l.act[k];
    }
    return l;
}

template <typename T, int VEC, int TPR, bool NT = false>
__device__ __forceinline__ void load_pixels(const T* __restrict__ p, const LanePix<VEC, TPR>& l,
                                            acc_t<T> (&o)[VEC]) {
    using R = typename RawOf<sizeof(T)>::type;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const R* q = reinterpret_cast<const R*>(elem_ptr(p, l.own[k]));
        o[k] = to_acc(__builtin_bit_cast(T, NT ? __builtin_nontemporal_load(q) : *q));
    }
}

// The lane's pixels into a prefetch-ring slot: raw bits per pixel, promoted
// by slot_get_pixels where the slot is consumed.
template <typename T, int VEC>
struct PixSlot {
    typename RawOf<sizeof(T)>::type r[VEC];
};

// Buffer loads: the plane base in SGPRs, the pixel's 32-bit byte offset per
// lane (no per-load address arithmetic in the shift loops).
template <typename T, int VEC, int TPR, bool NT = false>
__device__ __forceinline__ void slot_load_pixels(const T* __restrict__ p,
                                                 const LanePix<VEC, TPR>& l, PixSlot<T, VEC>& o) {
    using R = typename RawOf<sizeof(T)>::type;
    const __amdgpu_buffer_rsrc_t rs = plane_rsrc(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k)
        o.r[k] = buf_load<R, NT>(rs, l.own[k] * static_cast<uint32_t>(sizeof(T)));
}

template <typename T, int VEC>
__device__ __forceinline__ void slot_get_pixels(const PixSlot<T, VEC>& s, acc_t<T> (&o)[VEC]) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = raw_get<T>(s.r[k]);
}

// Register budget of the scatter kernels: enough waves per SIMD for two
// workgroups per CU (whose LDS the tile geometries are sized to allow).
template <int THREADS>
constexpr int kScatterWavesPerEU = 2 * (THREADS / 64) / 4 > 0 ? 2 * (THREADS / 64) / 4 : 1;

template <typename A>
__device__ __forceinline__ void lds_zero(A* p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = A(0);
}

// Fix-up view of one tile (tiles in row-major order, plane by plane, as
// tile_of(t, ..., order 0) numbers them) and of its 3x3 neighbourhood on the
// torus of tiles.
struct FixTile {
    int64_t bc, per_plane;
    int ntw, h0, w0, th, tw;
    int trn[3], tcn[3], thn[3], twn[3];
};

__device__ __forceinline__ FixTile fix_tile(int64_t t, int H, int W, int TH, int TW, int ntw,
                                            int nth) {
    FixTile f;
    f.ntw = ntw;
    f.per_plane = static_cast<int64_t>(ntw) * nth;
    f.bc = t / f.per_plane;
    const int rem = static_cast<int>(t - f.bc * f.per_plane);
    const int tr = rem / ntw;
    const int tc = rem - tr * ntw;
    f.h0 = tr * TH;
    f.w0 = tc * TW;
    f.th = min(TH, H - f.h0);
    f.tw = min(TW, W - f.w0);
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        f.trn[a] = (tr + a - 1 + nth) % nth;
        f.tcn[a] = (tc + a - 1 + ntw) % ntw;
        f.thn[a] = min(TH, H - f.trn[a] * TH);
        f.twn[a] = min(TW, W - f.tcn[a] * TW);
    }
    return f;
}

// The pixels of a th x tw tile that can receive spills with radius R: the
// border ring of width R (top band, bottom band, then the left and right R
// columns of the middle rows), or every pixel when the tile is too small for
// a ring.  ring_count / ring_pixel enumerate them; ring_slot is the inverse
// (-1 for an interior pixel).
__device__ __forceinline__ bool ring_mode(int th, int tw, int R) {
    return R > 0 && th >= 2 * R && tw >= 2 * R;
}

__device__ __forceinline__ int ring_count(int th, int tw, int R) {
    return ring_mode(th, tw, R) ? 2 * R * tw + (th - 2 * R) * 2 * R : th * tw;
}

__device__ __forceinline__ void ring_pixel(int idx, int th, int tw, int R, int& lr, int& lc) {
    const int band = R * tw;
    if (!ring_mode(th, tw, R) || idx < band) {
        lr = idx / tw;
        lc = idx - lr * tw;
    } else if (idx < 2 * band) {
        const int k = idx - band;
        lr = th - R + k / tw;
        lc = k - (k / tw) * tw;
    } else {
        const int k = idx - 2 * band;
        lr = R + k / (2 * R);
        const int c = k - (k / (2 * R)) * 2 * R;
        lc = c < R ? c : tw - 2 * R + c;
    }
}

__device__ __forceinline__ int ring_slot(int lr, int lc, int th, int tw, int R) {
    if (!ring_mode(th, tw, R) || lr < R) return lr * tw + lc;
    if (lr >= th - R) return R * tw + (lr - (th - R)) * tw + lc;
    if (lc < R) return 2 * R * tw + (lr - R) * 2 * R + lc;
    if (lc >= tw - R) return 2 * R * tw + (lr - R) * 2 * R + (lc - (tw - 2 * R));
    return -1;
}

// Visits the neighbouring tiles' spill entries that target pixel (lr, lc) of
// tile f, calling fn(tn, e) with the neighbour tile index and the entry
// index in its spill block.  The pixel sits in the window of the tile above
// (a = 0) at row lr + th_above when lr < R, of the tile below (a = 2) at row
// lr - th when lr >= th - R, of its own tile row (a = 1) at row lr; columns
// likewise.  Neighbours are visited in a fixed order, so any reduction over
// them is deterministic.
template <typename Fn>
__device__ __forceinline__ void spill_visit(const FixTile& f, int R, int lr, int lc, Fn&& fn) {
    const bool up = lr < R, down = lr >= f.th - R, left = lc < R, right = lc >= f.tw - R;
    if (!(up || down || left || right)) return;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        if ((a == 0 && !up) || (a == 2 && !down)) continue;
        const int i = a == 0 ? lr + f.thn[0] : (a == 1 ? lr : lr - f.th);
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            if ((b == 0 && !left) || (b == 2 && !right) || (a == 1 && b == 1)) continue;
            const int j = b == 0 ? lc + f.twn[0] : (b == 1 ? lc : lc - f.tw);
            const int64_t tn =
                f.bc * f.per_plane + static_cast<int64_t>(f.trn[a]) * f.ntw + f.tcn[b];
            fn(tn, spill_index(i, j, f.thn[a], f.twn[b], R));
        }
    }
}

// Sum of the neighbouring tiles' spills into pixel (lr, lc) of tile f, for
// NARR spill arrays (array q of tile n at spill + (q*ntiles + n)*stride).
template <typename A, int NARR>
__device__ __forceinline__ void spill_sum(const FixTile& f, int R, int lr, int lc,
                                          const A* __restrict__ spill, int64_t ntiles,
                                          int stride, A (&acc)[NARR]) {
#pragma unroll
    for (int q = 0; q < NARR; ++q) acc[q] = A(0);
    spill_visit(f, R, lr, lc, [&](int64_t tn, int e) {
#pragma unroll
        for (int q = 0; q < NARR; ++q) acc[q] += spill[(q * ntiles + tn) * stride + e];
    });
}

// Slot enumeration of a fix-up tile for a full tile width TW = 2^lg: slots
// map to pixels with shifts and masks only.  ALL (every pixel of the tile)
// takes th rows of TW slots; otherwise the ring tile (th, tw >= 2R) takes
// its 2R band rows of TW slots (the top R rows, then the bottom R), then the
// th - 2R middle rows of 2^lgm slots each (16 for R <= 8, 32 for R <= 16,
// 64 for R <= 32), whose first 2R are the left R and the right R columns.
// Slots past tw (edge tiles) or past 2R in a middle row are idle.  A ring pixel takes the spill entries of at most one
// vertical, one horizontal and the diagonal neighbour tile between them;
// their offsets are the neighbour's spill-block base (uniform per block)
// plus a small per-pixel index, listed in spill_visit's order.
struct FixRing {
    int R, lg, lgm, nband, n, ww, wwl, wwr;
    int64_t t00, t01, t02, t10, t12, t20, t21, t22;  // spill-block bases of the neighbours
    int64_t pb;                                       // offset of the tile's first pixel
};

template <bool ALL>
__device__ __forceinline__ FixRing fix_ring(const FixTile& f, int R, int lg, int64_t HW, int W,
                                            int stride) {
    FixRing g;
    const int R2 = 2 * R;
    g.R = R;
    g.lg = lg;
    g.lgm = R <= 8 ? 4 : (R <= 16 ? 5 : 6);
    g.nband = ALL ? f.th << lg : R2 << lg;
    g.n = ALL ? g.nband : g.nband + ((f.th - R2) << g.lgm);
    g.ww = f.tw + R2;       // spill row width of the tiles above and below
    g.wwl = f.twn[0] + R2;  // ... of the left column of tiles
    g.wwr = f.twn[2] + R2;  // ... of the right column of tiles
    auto tile_base = [&](int a, int b) {
        return (f.bc * f.per_plane + static_cast<int64_t>(f.trn[a]) * f.ntw + f.tcn[b]) * stride;
    };
    g.t00 = tile_base(0, 0);
    g.t01 = tile_base(0, 1);
    g.t02 = tile_base(0, 2);
    g.t10 = tile_base(1, 0);
    g.t12 = tile_base(1, 2);
    g.t20 = tile_base(2, 0);
    g.t21 = tile_base(2, 1);
    g.t22 = tile_base(2, 2);
    g.pb = f.bc * HW + static_cast<int64_t>(f.h0) * W + f.w0;
    return g;
}

// Slot s: its pixel (lr, lc), whether it is active (idle slots name pixel
// (0, 0)), the in-tile offset p = lr * W + lc, and its spill entries in
// visit order (-1 when unused).  Outputs by reference (plain registers).
template <bool ALL>
__device__ __forceinline__ void fix_slot(const FixTile& f, const FixRing& g, int s, int W,
                                         int& olr, int& olc, bool& oact, uint32_t& op,
                                         int64_t (&oe)[3]) {
    const int R = g.R, R2 = 2 * R;
    // the block's values as plain scalars (selects below pick values, not
    // members of g)
    const int64_t t00 = g.t00, t01 = g.t01, t02 = g.t02, t10 = g.t10, t12 = g.t12;
    const int64_t t20 = g.t20, t21 = g.t21, t22 = g.t22;
    const int ww = g.ww, wwl = g.wwl, wwr = g.wwr;
    int lr, lc;
    bool ok;
    if (ALL || s < g.nband) {
        const int br = s >> g.lg;
        lc = s & ((1 << g.lg) - 1);
        lr = ALL ? br : (br < R ? br : f.th - R2 + br);
        ok = s < g.n && lc < f.tw;
    } else {
        const int s2 = s - g.nband;
        const int cm = s2 & ((1 << g.lgm) - 1);
        lr = R + (s2 >> g.lgm);
        lc = cm < R ? cm : f.tw - R2 + cm;
        ok = s < g.n && cm < R2;
    }
    oact = ok;
    lr = ok ? lr : 0;
    lc = ok ? lc : 0;
    olr = lr;
    olc = lc;
    op = static_cast<uint32_t>(lr) * static_cast<uint32_t>(W) + static_cast<uint32_t>(lc);
    const bool up = lr < R, dn = lr >= f.th - R, lf = lc < R, rt = lc >= f.tw - R;
    // row in the top (tile above) or bottom (tile below) band
    const int vi = up ? R + lr : lr - f.th + R;
    const int wwh = lf ? wwl : wwr;
    const int64_t V = (up ? t01 : t21) + (vi * ww + lc + R);
    const int64_t Hz = (lf ? t10 : t12) + (R2 * wwh + lr * R2 + (lf ? R + lc : lc - f.tw + R));
    const int64_t Cn = (up ? (lf ? t00 : t02) : (lf ? t20 : t22)) +
                       (vi * wwh + (lf ? lc + f.twn[0] : lc - f.tw) + R);
    const bool hv = up || dn, hh = lf || rt, cor = hv && hh;
    // visit order: above-left C V H, above-right V C H, below-left H C V,
    // below-right H V C; one edge: V or H alone
    oe[0] = cor ? (up ? (lf ? Cn : V) : Hz) : (hv ? V : (hh ? Hz : int64_t(-1)));
    oe[1] = cor ? (up ? (lf ? V : Cn) : (lf ? Cn : V)) : int64_t(-1);
    oe[2] = cor ? (up ? Hz : (lf ? V : Cn)) : int64_t(-1);
}

// Slot path available: a ring tile (or, for ALL, any tile) and TW = 2^lg.
__device__ __forceinline__ bool fix_slots_ok(const FixTile& f, int R, int TW, bool all, int& lg) {
    lg = 31 - __builtin_clz(static_cast<unsigned>(TW));
    return TW == (1 << lg) && (all ? (R == 0 || ring_mode(f.th, f.tw, R)) : ring_mode(f.th, f.tw, R));
}

// Fix-up of a whole tile through the slots (PART: every pixel, else the
// ring).  Each lane takes kFixBatch slots at a time and issues all their
// loads (the outputs or partial sums and up to three spill entries each)
// before it sums any, so a lane has a batch of loads in flight; the sums
// keep spill_visit's order.
constexpr int kFixBatch = 4;

template <typename OutT, typename A, int NARR, bool PART>
__device__ __forceinline__ void fixup_tile_slots(const FixTile& f, int R, int lg, int64_t HW,
                                                 int W, int stride,
                                                 const A* __restrict__ spill, int64_t qstride,
                                                 const A* __restrict__ part,
                                                 OutT* __restrict__ out0,
                                                 OutT* __restrict__ out1) {
    const FixRing g = fix_ring<PART>(f, R, lg, HW, W, stride);
    const int step = static_cast<int>(blockDim.x);
    OutT* o[2] = {out0, out1};
    for (int s0 = threadIdx.x; s0 < g.n; s0 += step * kFixBatch) {
        int lr[kFixBatch], lc[kFixBatch];
        bool act[kFixBatch];
        uint32_t p[kFixBatch];
        int64_t e[kFixBatch][3];
#pragma unroll
        for (int k = 0; k < kFixBatch; ++k)
            fix_slot<PART>(f, g, s0 + k * step, W, lr[k], lc[k], act[k], p[k], e[k]);
        // all loads first: own value (or partial sum) and the spill entries
        A base_v[kFixBatch][NARR], sv[kFixBatch][NARR][3];
#pragma unroll
        for (int k = 0; k < kFixBatch; ++k) {
#pragma unroll
            for (int q = 0; q < NARR; ++q) {
                if constexpr (PART)
                    base_v[k][q] = part[g.pb + p[k]];
                else
                    base_v[k][q] = o[q][g.pb + p[k]];
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const int64_t ix = e[k][c] >= 0 ? q * qstride + e[k][c] : 0;
                    sv[k][q][c] = spill[ix];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kFixBatch; ++k) {
            if (!act[k]) continue;
#pragma unroll
            for (int q = 0; q < NARR; ++q) {
                A acc = A(0);
#pragma unroll
                for (int c = 0; c < 3; ++c) acc += e[k][c] >= 0 ? sv[k][q][c] : A(0);
                if constexpr (PART)
                    o[0][g.pb + p[k]] = from_acc<OutT>(base_v[k][q] + acc);
                else
                    o[q][g.pb + p[k]] = base_v[k][q] + acc;
            }
        }
    }
}

// Adds the neighbouring tiles' spills into every ring pixel of its tile, in
// place.  R comes from the workspace header written by the main kernel
// (kFarRadius: the main kernel ran the gather algorithm, nothing to do).
// With PART (16-bit outputs) every pixel is rewritten as
// out = T(part + spills) instead.  Tiles too small for a ring, and tile
// widths TW that are not a power of two, take the one-pixel loop.
template <typename OutT, typename A, int NARR, bool PART>
__global__ __launch_bounds__(256) void spill_fixup_kernel(
    int H, int W, int TH, int TW, int ntw, int nth, int spill_stride, const int* __restrict__ hdr,
    const A* __restrict__ spill, int64_t ntiles, const A* __restrict__ part,
    OutT* __restrict__ out0, OutT* __restrict__ out1) {
    const int R = __builtin_amdgcn_readfirstlane(hdr[0]);
    if (R > kMaxHalo || (R == 0 && !PART)) return;
    const FixTile f = fix_tile(blockIdx.x, H, W, TH, TW, ntw, nth);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t qstride = ntiles * spill_stride;  // spill array q at spill + q * qstride
    int lg;
    if (fix_slots_ok(f, R, TW, PART, lg)) {
        fixup_tile_slots<OutT, A, NARR, PART>(f, R, lg, HW, W, spill_stride, spill, qstride, part,
                                              out0, out1);
        return;
    }
    // Pixels to visit: every pixel (PART: R = 0 turns the ring into the
    // whole tile), else the border ring.
    OutT* o[2] = {out0, out1};
    const int Rv = PART ? 0 : R;
    const int n = ring_count(f.th, f.tw, Rv);
    for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
        int lr, lc;
        ring_pixel(idx, f.th, f.tw, Rv, lr, lc);
        A acc[NARR];
        if (R > 0) {
            spill_sum<A, NARR>(f, R, lr, lc, spill, ntiles, spill_stride, acc);
        } else {
#pragma unroll
            for (int q = 0; q < NARR; ++q) acc[q] = A(0);
        }
        const int64_t p = f.bc * HW + static_cast<int64_t>(f.h0 + lr) * W + (f.w0 + lc);
        if constexpr (PART) {
            o[0][p] = from_acc<OutT>(part[p] + acc[0]);
        } else {
#pragma unroll
            for (int q = 0; q < NARR; ++q) o[q][p] = o[q][p] + acc[q];
        }
    }
}

}  // namespace nsh
