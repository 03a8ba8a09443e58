// scatter.hpp -- shared pieces of the scatter-form kernels (accumulate_uz,
// metropolis_aggregate) on gfx950.
//
// A scatter kernel's lane that owns pixel q reads its weight w_s[q] once,
// aligned, and adds the term it contributes to pixel q + s into an LDS
// accumulator window covering its tile plus a kRmax border.  After the shift
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
// image tiles and the accumulator windows carry a kRmax border and share a
// row pitch congruent to 16 words mod 32, so the two rows of a half-wave
// (TPR = 16) fall on disjoint banks.  A wave owns 64 / TPR whole tile rows.
// STRIDED = false is the contiguous variant (lane tx owns pixels
// tx*VEC .. tx*VEC + VEC-1, moved with one 16-byte access) with an odd
// pitch; its LDS reads of a wave are 4-way strided.
template <int VEC, int ROWS, int TPR, bool STRIDED = true>
struct SGeo {
    static_assert(64 % TPR == 0, "a wave must own whole tile rows");
    static constexpr int THREADS = TPR * ROWS;
    static constexpr int TW = TPR * VEC;
    static constexpr int TH = ROWS;
    static constexpr int LW = TW + 2 * kRmax;
    static constexpr int LH = TH + 2 * kRmax;
    static constexpr int PITCH = STRIDED ? LW + ((16 - LW % 32) + 32) % 32 : LW + 1;
    static constexpr int TILE = LH * PITCH;
    // spill block stride (entries), sized for the largest border
    static constexpr int SPILL = 2 * kRmax * (TW + 2 * kRmax) + 2 * kRmax * TH;
    // own ring partials (entries): >= ring_count of any tile
    static constexpr int RING = 2 * kRmax * (TW + TH);
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
    static constexpr int QW = LW / VEC;  // LW = TPR * VEC + 2 * kRmax
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

// The (up to 3) spill entries that target pixel (lr, lc) of tile f when the
// tile holds a full ring (th, tw >= 2R: a pixel is near at most one
// horizontal and one vertical edge), as flat offsets tn * stride + e of the
// first spill array, in spill_visit's order: e[c - 1] is visited first,
// e[0] last, unused slots hold -1.  Branch-free, so that a caller can issue
// the loads of several pixels before it sums any.
__device__ __forceinline__ void ring_contribs(const FixTile& f, int R, int lr, int lc, int stride,
                                              int64_t (&e)[3]) {
    const bool up = lr < R, down = lr >= f.th - R, left = lc < R, right = lc >= f.tw - R;
    e[0] = e[1] = e[2] = -1;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            if (a == 1 && b == 1) continue;
            const bool va = a == 1 || (a == 0 ? up : down);
            const bool vb = b == 1 || (b == 0 ? left : right);
            const int i = a == 0 ? lr + f.thn[0] : (a == 1 ? lr : lr - f.th);
            const int j = b == 0 ? lc + f.twn[0] : (b == 1 ? lc : lc - f.tw);
            const int64_t tn =
                f.bc * f.per_plane + static_cast<int64_t>(f.trn[a]) * f.ntw + f.tcn[b];
            const int64_t v = va && vb ? tn * stride + spill_index(i, j, f.thn[a], f.twn[b], R) : -1;
            // shift register: the newest valid entry goes to e[0]
            const bool take = v >= 0;
            e[2] = take ? e[1] : e[2];
            e[1] = take ? e[0] : e[1];
            e[0] = take ? v : e[0];
        }
    }
}

// Adds the neighbouring tiles' spills into every ring pixel of its tile, in
// place.  R comes from the workspace header written by the main kernel
// (R > kRmax: the main kernel ran the gather algorithm, nothing to do).
// With PART (16-bit outputs) every pixel is rewritten as
// out = T(part + spills) instead.  Each lane takes kFixBatch pixels at a
// time and issues all their loads (the outputs or partial sums and up to
// three spill entries each) before it sums any, so a lane has a batch of
// loads in flight instead of one pixel's dependent chain; the sums keep
// spill_visit's order.  Tiles too small for a ring take the one-pixel loop.
constexpr int kFixBatch = 4;

template <typename OutT, typename A, int NARR, bool PART>
__global__ __launch_bounds__(256) void spill_fixup_kernel(
    int H, int W, int TH, int TW, int ntw, int nth, int spill_stride, const int* __restrict__ hdr,
    const A* __restrict__ spill, int64_t ntiles, const A* __restrict__ part,
    OutT* __restrict__ out0, OutT* __restrict__ out1) {
    const int R = __builtin_amdgcn_readfirstlane(hdr[0]);
    if (R > kRmax || (R == 0 && !PART)) return;
    const FixTile f = fix_tile(blockIdx.x, H, W, TH, TW, ntw, nth);
    const int64_t HW = static_cast<int64_t>(H) * W;
    OutT* o[2] = {out0, out1};
    // Pixels to visit: every pixel (PART: R = 0 turns the ring into the
    // whole tile), else the border ring.
    const int Rv = PART ? 0 : R;
    const int n = ring_count(f.th, f.tw, Rv);
    const int64_t qstride = ntiles * spill_stride;  // spill array q at spill + q * qstride
    if (R > 0 && !ring_mode(f.th, f.tw, R)) {
        for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
            int lr, lc;
            ring_pixel(idx, f.th, f.tw, Rv, lr, lc);
            A acc[NARR];
            spill_sum<A, NARR>(f, R, lr, lc, spill, ntiles, spill_stride, acc);
            const int64_t p = f.bc * HW + static_cast<int64_t>(f.h0 + lr) * W + (f.w0 + lc);
            if constexpr (PART) {
                o[0][p] = from_acc<OutT>(part[p] + acc[0]);
            } else {
#pragma unroll
                for (int q = 0; q < NARR; ++q) o[q][p] = o[q][p] + acc[q];
            }
        }
        return;
    }
    for (int base = threadIdx.x; base < n; base += blockDim.x * kFixBatch) {
        int64_t p[kFixBatch], e[kFixBatch][3];
        bool act[kFixBatch];
#pragma unroll
        for (int k = 0; k < kFixBatch; ++k) {
            const int idx = base + k * static_cast<int>(blockDim.x);
            act[k] = idx < n;
            int lr, lc;
            ring_pixel(act[k] ? idx : n - 1, f.th, f.tw, Rv, lr, lc);  // idle: a valid pixel
            p[k] = f.bc * HW + static_cast<int64_t>(f.h0 + lr) * W + (f.w0 + lc);
            if (R > 0)
                ring_contribs(f, R, lr, lc, spill_stride, e[k]);
            else
                e[k][0] = e[k][1] = e[k][2] = -1;
        }
        // all loads first: own value (or partial sum) and the spill entries
        A base_v[kFixBatch][NARR], sv[kFixBatch][NARR][3];
#pragma unroll
        for (int k = 0; k < kFixBatch; ++k) {
#pragma unroll
            for (int q = 0; q < NARR; ++q) {
                if constexpr (PART)
                    base_v[k][q] = part[p[k]];
                else
                    base_v[k][q] = o[q][p[k]];
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
                for (int c = 2; c >= 0; --c) acc += e[k][c] >= 0 ? sv[k][q][c] : A(0);
                if constexpr (PART)
                    o[0][p[k]] = from_acc<OutT>(base_v[k][q] + acc);
                else
                    o[q][p[k]] = base_v[k][q] + acc;
            }
        }
    }
}

}  // namespace nsh
