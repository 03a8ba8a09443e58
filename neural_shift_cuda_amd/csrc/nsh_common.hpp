// nsh_common.hpp -- shared device/host plumbing for the gfx950 shift-window
// kernels: storage dtypes and their promotion to the accumulator type, 16-byte
// vector memory helpers, the per-workgroup shift table staged in LDS, the
// XCD-aware tile order, and the C-ABI error channel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "neural_shift_hip.h"

namespace nsh {

// ---------------------------------------------------------------------------
// Storage types.  fp16/bf16/fp32 promote to fp32 at load; fp64 stays fp64.
// ---------------------------------------------------------------------------
using f16 = _Float16;
struct bf16 {
    uint16_t bits;
};

template <typename T> struct AccOf { using type = float; };
template <> struct AccOf<double> { using type = double; };
template <typename T> using acc_t = typename AccOf<T>::type;

__device__ __forceinline__ float to_acc(float v) { return v; }
__device__ __forceinline__ double to_acc(double v) { return v; }
__device__ __forceinline__ float to_acc(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_acc(bf16 v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

template <typename T> __device__ __forceinline__ T from_acc(acc_t<T> v);
template <> __device__ __forceinline__ float from_acc<float>(float v) { return v; }
template <> __device__ __forceinline__ double from_acc<double>(double v) { return v; }
template <> __device__ __forceinline__ f16 from_acc<f16>(float v) {
    return static_cast<f16>(v);  // round to nearest even
}
template <> __device__ __forceinline__ bf16 from_acc<bf16>(float v) {
    // Round to nearest even; every NaN becomes the canonical quiet 0x7FC0,
    // the same encoding torch's float->bfloat16 conversion produces.
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return bf16{0x7FC0};
    u += 0x7fffu + ((u >> 16) & 1u);
    return bf16{static_cast<uint16_t>(u >> 16)};
}

// Fused multiply-add in the accumulator type (single rounding).  Note that
// __builtin_fma is the double-precision builtin: on float operands it would
// convert to double and back.
__device__ __forceinline__ float fma_acc(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_acc(double a, double b, double c) { return __builtin_fma(a, b, c); }

// ---------------------------------------------------------------------------
// Vector memory.  A Pack<T, VEC> moves VEC consecutive elements with one
// load/store of VEC*sizeof(T) bytes (2, 4, 8 or 16).
// ---------------------------------------------------------------------------
template <int BYTES> struct RawOf;
template <> struct RawOf<2> { using type = uint16_t; };
template <> struct RawOf<4> { using type = uint32_t; };
template <> struct RawOf<8> { typedef uint32_t type __attribute__((ext_vector_type(2))); };
template <> struct RawOf<16> { typedef uint32_t type __attribute__((ext_vector_type(4))); };

template <typename T, int VEC> struct Pack {
    T e[VEC];
};

template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> load_pack(const T* p) {
    using R = typename RawOf<sizeof(T) * VEC>::type;
    const R r = *reinterpret_cast<const R*>(p);
    return __builtin_bit_cast(Pack<T, VEC>, r);
}

template <typename T, int VEC>
__device__ __forceinline__ void store_pack(T* p, const Pack<T, VEC>& v) {
    using R = typename RawOf<sizeof(T) * VEC>::type;
    *reinterpret_cast<R*>(p) = __builtin_bit_cast(R, v);
}

// Streaming store for outputs that are never re-read by the same kernel.
template <typename T, int VEC>
__device__ __forceinline__ void store_pack_nt(T* p, const Pack<T, VEC>& v) {
    using R = typename RawOf<sizeof(T) * VEC>::type;
    __builtin_nontemporal_store(__builtin_bit_cast(R, v), reinterpret_cast<R*>(p));
}

// One element, streaming (nontemporal) store.
template <typename T>
__device__ __forceinline__ void store_elem_nt(T* p, T v) {
    using R = typename RawOf<sizeof(T)>::type;
    __builtin_nontemporal_store(__builtin_bit_cast(R, v), reinterpret_cast<R*>(p));
}

template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> load_pack_nt(const T* p) {
    using R = typename RawOf<sizeof(T) * VEC>::type;
    const R r = __builtin_nontemporal_load(reinterpret_cast<const R*>(p));
    return __builtin_bit_cast(Pack<T, VEC>, r);
}

// Load VEC elements and promote them to the accumulator type.
template <typename T, int VEC, bool NT = false>
__device__ __forceinline__ void load_acc(const T* p, acc_t<T> (&o)[VEC]) {
    const Pack<T, VEC> v = NT ? load_pack_nt<T, VEC>(p) : load_pack<T, VEC>(p);
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = to_acc(v.e[k]);
}

// Workgroup barrier that orders LDS traffic only: outstanding global loads
// (the weight prefetches) are not waited for.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Prefetch-ring slots.  A slot keeps VEC loaded elements as the raw bits of
// one vector load and promotes them where the slot is consumed: promoting
// (or even splitting) 16-bit elements right after their load makes the wave
// wait for that load at once, which drains the ring (each ring iteration
// then pays a full memory latency).  For fp32 and fp64 the promotion is the
// identity.
template <typename T, int VEC>
using SlotRaw = typename RawOf<sizeof(T) * VEC>::type;

template <typename T, int VEC, bool NT = false>
__device__ __forceinline__ void slot_load(const T* p, SlotRaw<T, VEC>& s) {
    const SlotRaw<T, VEC>* q = reinterpret_cast<const SlotRaw<T, VEC>*>(p);
    s = NT ? __builtin_nontemporal_load(q) : *q;
}

// Buffer access to one plane: the base sits in the resource's SGPRs and each
// lane supplies a 32-bit byte offset (an in-plane offset is below 2^31
// bytes).  A loop that walks the shift planes then advances the base with
// scalar adds, and its loads and stores take no per-lane address arithmetic
// (a flat pointer per lane costs a 64-bit vector add per access).  The range
// check is off (num_records = 2^32 - 1); dword 3 is the raw-buffer format
// word of the gfx9 family.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), -1,
                                             0x00020000);
}

// Cache-policy bits of a buffer access: nontemporal (streaming) or default.
template <bool NT>
constexpr int kBufAux = NT ? 2 : 0;

template <typename R, bool NT = false>
__device__ __forceinline__ R buf_load(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    if constexpr (sizeof(R) == 2)
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, kBufAux<NT>));
    else if constexpr (sizeof(R) == 4)
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kBufAux<NT>));
    else if constexpr (sizeof(R) == 8)
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kBufAux<NT>));
    else
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kBufAux<NT>));
}

template <typename R, bool NT = false>
__device__ __forceinline__ void buf_store(R v, __amdgpu_buffer_rsrc_t rs, uint32_t off) {
    using U16 = uint16_t;
    using U32 = uint32_t;
    using U64 = typename RawOf<8>::type;
    using U128 = typename RawOf<16>::type;
    if constexpr (sizeof(R) == 2)
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(U16, v), rs, off, 0, kBufAux<NT>);
    else if constexpr (sizeof(R) == 4)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(U32, v), rs, off, 0, kBufAux<NT>);
    else if constexpr (sizeof(R) == 8)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(U64, v), rs, off, 0, kBufAux<NT>);
    else
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(U128, v), rs, off, 0,
                                               kBufAux<NT>);
}

// A ring slot from plane p at the lane's byte offset (contiguous lanes).
template <typename T, int VEC, bool NT = false>
__device__ __forceinline__ void slot_load_at(const T* p, uint32_t boff, SlotRaw<T, VEC>& s) {
    s = buf_load<SlotRaw<T, VEC>, NT>(plane_rsrc(p), boff);
}

template <typename T, int VEC>
__device__ __forceinline__ void slot_get(const SlotRaw<T, VEC>& s, acc_t<T> (&o)[VEC]) {
    const Pack<T, VEC> v = __builtin_bit_cast(Pack<T, VEC>, s);
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = to_acc(v.e[k]);
}

// One element's raw bits (strided lanes load their pixels one by one).
template <typename T>
__device__ __forceinline__ acc_t<T> raw_get(typename RawOf<sizeof(T)>::type r) {
    return to_acc(__builtin_bit_cast(T, r));
}

// One element into plane p at the lane's byte offset.
template <typename T, bool NT>
__device__ __forceinline__ void store_elem_at(T* p, uint32_t boff, T v) {
    using R = typename RawOf<sizeof(T)>::type;
    buf_store<R, NT>(__builtin_bit_cast(R, v), plane_rsrc(p), boff);
}

// Store VEC accumulator values as T (rounding once) into plane p at the
// lane's byte offset.
template <typename T, int VEC, bool NT>
__device__ __forceinline__ void store_acc_at(T* p, uint32_t boff, const acc_t<T> (&v)[VEC]) {
    Pack<T, VEC> o;
#pragma unroll
    for (int k = 0; k < VEC; ++k) o.e[k] = from_acc<T>(v[k]);
    using R = typename RawOf<sizeof(T) * VEC>::type;
    buf_store<R, NT>(__builtin_bit_cast(R, o), plane_rsrc(p), boff);
}

// Store VEC accumulator values as T (rounding once).
template <typename T, int VEC>
__device__ __forceinline__ void store_acc(T* p, const acc_t<T> (&v)[VEC], bool nontemporal) {
    Pack<T, VEC> o;
#pragma unroll
    for (int k = 0; k < VEC; ++k) o.e[k] = from_acc<T>(v[k]);
    if (nontemporal)
        store_pack_nt<T, VEC>(p, o);
    else
        store_pack<T, VEC>(p, o);
}

// Accumulator-typed output (fp32 or fp64) of VEC elements; splits into
// 16-byte stores when VEC*sizeof(A) exceeds 16.
template <typename A, int VEC>
__device__ __forceinline__ void store_out(A* p, const A (&v)[VEC]) {
    constexpr int PER = (16 / static_cast<int>(sizeof(A))) < VEC ? (16 / static_cast<int>(sizeof(A))) : VEC;
#pragma unroll
    for (int k0 = 0; k0 < VEC; k0 += PER) {
        Pack<A, PER> o;
#pragma unroll
        for (int k = 0; k < PER; ++k) o.e[k] = v[k0 + k];
        store_pack<A, PER>(p + k0, o);
    }
}

template <typename A, int VEC>
__device__ __forceinline__ void load_out(const A* p, A (&v)[VEC]) {
    constexpr int PER = (16 / static_cast<int>(sizeof(A))) < VEC ? (16 / static_cast<int>(sizeof(A))) : VEC;
#pragma unroll
    for (int k0 = 0; k0 < VEC; k0 += PER) {
        const Pack<A, PER> o = load_pack<A, PER>(p + k0);
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k0 + k] = o.e[k];
    }
}

// ---------------------------------------------------------------------------
// Shift table.  The caller's (S, cols) int64 table is decoded once per
// workgroup into LDS records so the hot loop never does 64-bit modulo:
//   x  = dx clamped to +-2^30 (exact for every box test on a < 2^30 extent)
//   y  = dy clamped likewise
//   z  = (dx mod H) | has_inv << 31
//   w  = (dy mod W) | periodic << 31
// has_inverse column.  Without `codes` it is the reference's flag: nonzero
// means a mirror term dropped where its source wraps.  With `codes` (the
// caller asked for an extension) a value v in [0, 7] is a row code: bits 0-1
// select the mirror (0 none, 2 circular: the periodic operator, 1 or 3
// dropped where its source wraps), bit 2 drops the forward term where
// (h + dx, w + dy) leaves the image (the caller's box mask, applied here).
// With bit 2 set a circular mirror is the dropped-at-wrap one (its weight is
// the masked forward weight).  Any other value is a mirror dropped at the
// wrap.
// ---------------------------------------------------------------------------
constexpr int kClamp = 1 << 30;

// Bits of the `codes` argument of the accumulate_uz and normalized kernels:
// the table's third column holds row codes (see below), and the weights are
// shared by every channel (one plane per (shift, batch) instead of one per
// (shift, batch, channel): the reference installers' single-head weights,
// broadcast to the channels).
constexpr int kCodesRows = 1;
constexpr int kCodesSharedW = 2;

// The kernels' `codes` from the flags a call ORs into its dtype argument.
__host__ __forceinline__ int dtype_codes(int dtype) {
    return ((dtype & NSH_SHIFT_CODES) ? kCodesRows : 0) |
           ((dtype & NSH_SHARED_WEIGHTS) ? kCodesSharedW : 0);
}

// Weight plane of image (b, c) within one shift block, and the distance
// between shift blocks, for per-channel (plane_step = B*C*H*W) or
// channel-shared weights (B*H*W).
__host__ __device__ __forceinline__ int64_t weight_plane(int64_t b, int64_t c, int64_t C,
                                                          bool shared) {
    return shared ? b : b * C + c;
}
__host__ __device__ __forceinline__ int64_t weight_step(int64_t plane_step, int64_t C,
                                                         bool shared) {
    return shared ? plane_step / C : plane_step;
}

struct ShiftRec {
    int dx, dy, dxm, dym;
    bool inv;   // the row has a mirror term
    bool per;   // ... taken circularly (no image-border mask)
    bool fbox;  // the forward term is dropped where p + s leaves the image
};

__device__ __forceinline__ int clamp_shift(int64_t v) {
    return static_cast<int>(v < -kClamp ? -kClamp : (v > kClamp ? kClamp : v));
}

__device__ __forceinline__ int64_t mod_pos(int64_t v, int64_t n) {
    int64_t r = v % n;
    return r < 0 ? r + n : r;
}

// LDS bytes of the staged table (S records; 16-byte aligned, so the arrays a
// kernel places after it stay aligned).
__host__ __device__ constexpr size_t shift_lds_bytes(int S) {
    return static_cast<size_t>(S) * 16;
}

// Cooperative decode of the whole table into lds[0..S).  Ends with a barrier.
__device__ __forceinline__ void stage_shifts(int4* lds, const int64_t* __restrict__ shifts,
                                             int S, int cols, int H, int W, bool codes) {
    for (int s = threadIdx.x; s < S; s += blockDim.x) {
        const int64_t dx = shifts[static_cast<int64_t>(s) * cols + 0];
        const int64_t dy = shifts[static_cast<int64_t>(s) * cols + 1];
        int64_t v = cols >= 3 ? shifts[static_cast<int64_t>(s) * cols + 2] : 0;
        if (!codes) v = v != 0 ? 1 : 0;
        const bool small = v >= 0 && v <= 7;
        const int64_t mir = small ? (v & 3) : 1;
        const bool fbox = small && (v & 4) != 0;
        int4 r;
        r.x = clamp_shift(dx);
        r.y = clamp_shift(dy);
        r.z = static_cast<int>(mod_pos(dx, H)) | (mir != 0 ? static_cast<int>(0x80000000u) : 0) |
              (fbox ? 0x40000000 : 0);
        r.w = static_cast<int>(mod_pos(dy, W)) |
              (mir == 2 && !fbox ? static_cast<int>(0x80000000u) : 0);
        lds[s] = r;
    }
    __syncthreads();
}

__device__ __forceinline__ ShiftRec read_shift(const int4* lds, int s) {
    const int4 r = lds[s];
    ShiftRec o;
    o.dx = __builtin_amdgcn_readfirstlane(r.x);
    o.dy = __builtin_amdgcn_readfirstlane(r.y);
    const int z = __builtin_amdgcn_readfirstlane(r.z);
    o.dxm = z & 0x3fffffff;
    o.inv = z < 0;
    o.fbox = (z & 0x40000000) != 0;
    const int w = __builtin_amdgcn_readfirstlane(r.w);
    o.dym = w & 0x7fffffff;
    o.per = w < 0;
    return o;
}

// (v mod n) for v in [-n, 2n): the hot-loop wrap once the shift is reduced.
__device__ __forceinline__ int wrap1(int v, int n) {
    return v < 0 ? v + n : (v >= n ? v - n : v);
}

__device__ __forceinline__ bool in_range(int v, int n) {
    return static_cast<unsigned>(v) < static_cast<unsigned>(n);
}

// ---------------------------------------------------------------------------
// Tiles.  A workgroup of 256 lanes owns a TH x TW tile of one (b, c) plane;
// lane (ty, tx) owns VEC consecutive pixels of row ty.  Neighbouring tiles
// share halos, so the linear tile order is remapped so that each of the 8
// XCDs (which receive workgroups round-robin) works on one contiguous band of
// tiles and its L2 sees the halo reuse.
// ---------------------------------------------------------------------------
constexpr int kThreads = 256;
constexpr int kTPR = 16;   // lanes per tile row
constexpr int kRows = 16;  // tile rows
constexpr int kRmax = 8;   // LDS halo radius
// Header radius a scatter kernel writes when its tiles ran the gather form
// (the table reaches beyond the tile's halo): its fix-up has nothing to do.
constexpr int kFarRadius = 1 << 30;
// Widest halo of any scatter instantiation (the fix-up's slot enumeration
// covers border bands up to this width).
constexpr int kMaxHalo = 32;
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t xcd_tile(int64_t bid, int64_t nblocks) {
    const int64_t xcd = bid % kXcds;
    const int64_t local = bid / kXcds;
    const int64_t per = nblocks / kXcds;
    const int64_t rem = nblocks % kXcds;
    return xcd * per + (xcd < rem ? xcd : rem) + local;
}

struct TileIdx {
    int64_t bc;  // plane index b*C + c
    int h0, w0;  // top-left pixel of the tile
};

// Tile t of the launch.  order 0: the tiles of a plane row-major; order 2:
// bands of `band` tile rows, row-major across bands and column-major inside
// a band, so the tiles above and below a tile are dispatched right next to it
// (their shared halo rows are then read while still in L2) while every
// band still walks whole rows of the weight planes (few TLB pages per band).
__device__ __forceinline__ TileIdx tile_of(int64_t t, int ntw, int nth, int TH, int TW,
                                           int order = 0, int band = 1) {
    const int64_t per_plane = static_cast<int64_t>(ntw) * nth;
    TileIdx r;
    r.bc = t / per_plane;
    const int rem = static_cast<int>(t - r.bc * per_plane);
    int tr, tc;
    if (order == 2 && band > 1) {
        const int band_tiles = band * ntw;
        const int bi = rem / band_tiles;
        const int within = rem - bi * band_tiles;
        const int rows = nth - bi * band < band ? nth - bi * band : band;
        tc = within / rows;
        tr = bi * band + (within - tc * rows);
    } else {
        tr = rem / ntw;
        tc = rem - tr * ntw;
    }
    r.h0 = tr * TH;
    r.w0 = tc * TW;
    return r;
}

// Stage a plane tile with a kRmax halo into LDS (circularly wrapped), promoted
// to the accumulator type.  The staged region is LH x LW elements stored with
// row pitch `pitch` (>= LW; an odd pitch spreads the rows over the banks).
// Offset within its (b, c) plane of element i (row-major over LW columns)
// of the tile window that starts HALO rows above and HALO columns left of
// (h0, w0), wrapped around the image.  `cheap`: H >= window rows and
// W >= LW, so one conditional wrap per coordinate suffices.
template <int HALO = kRmax>
__device__ __forceinline__ uint32_t halo_offset(int i, int LW, int h0, int w0, int H, int W,
                                                bool cheap) {
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
    return static_cast<uint32_t>(gh) * static_cast<uint32_t>(W) + static_cast<uint32_t>(gw);
}

// Loads the LH x LW window whose top-left pixel is (h0 - halo, w0 - halo),
// wrapped circularly, into LDS: window element (r, c) goes to lds[ix(r, c)].
// Each lane issues kStageBatch loads before it stores any, so a batch of
// loads is in flight per lane instead of one load-wait-store chain per
// element (the tail of a batch re-loads the last element, in bounds, and
// does not store it): c4 backward 7.89 -> 7.54-7.71 ms, forward 4.25 ->
// 4.19 ms.  (The c3 fp64 forwards measured 0.071 -> 0.073 ms in the same
// runs, also with their staging left one element at a time.)  Batches of 4
// or 16 measured slower (c4 backward 7.55-7.67 ms at 4; c3 forwards 2-5%
// slower at 16).
constexpr int kStageBatch = 8;

template <typename T, typename A, typename Ix>
__device__ __forceinline__ void stage_window(A* lds, const T* __restrict__ plane, int H, int W,
                                             int h0, int w0, int LH, int LW, Ix ix,
                                             int halo = kRmax) {
    constexpr int NB = kStageBatch;
    const bool cheap = H >= LH && W >= LW;  // one conditional wrap suffices
    const int n = LH * LW;
    const int step = static_cast<int>(blockDim.x);
    for (int base = threadIdx.x; base < n; base += step * NB) {
        T v[NB];
        int li[NB];
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int i = min(base + k * step, n - 1);
            const int r = i / LW;
            const int c = i - r * LW;
            int gh = h0 - halo + r;
            int gw = w0 - halo + c;
            if (cheap) {
                gh = wrap1(gh, H);
                gw = wrap1(gw, W);
            } else {
                gh = static_cast<int>(mod_pos(gh, H));
                gw = static_cast<int>(mod_pos(gw, W));
            }
            li[k] = ix(r, c);
            v[k] = plane[static_cast<uint32_t>(gh) * static_cast<uint32_t>(W) +
                         static_cast<uint32_t>(gw)];
        }
#pragma unroll
        for (int k = 0; k < NB; ++k)
            if (base + k * step < n) lds[li[k]] = to_acc(v[k]);
    }
}

template <typename T, typename A>
__device__ __forceinline__ void stage_tile(A* lds, const T* __restrict__ plane, int H, int W,
                                           int h0, int w0, int LH, int LW, int pitch,
                                           int halo = kRmax) {
    stage_window<T, A>(lds, plane, H, W, h0, w0, LH, LW,
                       [pitch](int r, int c) { return r * pitch + c; }, halo);
}

template <typename T, typename A>
__device__ __forceinline__ void stage_tile(A* lds, const T* __restrict__ plane, int H, int W,
                                           int h0, int w0, int LH, int LW) {
    stage_tile<T, A>(lds, plane, H, W, h0, w0, LH, LW, LW);
}

template <typename A>
__device__ __forceinline__ void stage_tile_acc(A* lds, const A* __restrict__ plane, int H, int W,
                                               int h0, int w0, int LH, int LW) {
    stage_tile<A, A>(lds, plane, H, W, h0, w0, LH, LW, LW);
}

// Rows of a band.  A kernel may run on one horizontal band of a larger
// image (a spatial split: the band's own rows plus halo rows above and below
// that hold the neighbouring rows, wrapped around the image at its top and
// bottom edges).  Local row h is then the image's row (org + h) mod Hg, and
// every box test (a mirror term dropped where its source wraps, the forward
// box) is taken on those image rows, so the band's own rows come out as in
// the whole-image call.  The whole image is org = 0, Hg = H.
struct Band {
    int org, Hg;
};

__device__ __forceinline__ int band_row(const Band& b, int h) {
    const int r = b.org + h;
    if (__builtin_expect(static_cast<unsigned>(r) < static_cast<unsigned>(b.Hg), 1))
        return r;  // every row of a whole-image call: no division
    const int m = r % b.Hg;
    return m < 0 ? m + b.Hg : m;
}

// Whether local rows h0..h1 are image rows org + h0 .. org + h1 without
// wrapping and stay inside the image when displaced by dx.
__device__ __forceinline__ bool band_rows_inside(const Band& b, int h0, int h1, int dx) {
    const int g0 = b.org + h0, g1 = b.org + h1;
    return g0 >= 0 && g1 < b.Hg && g0 + dx >= 0 && g1 + dx < b.Hg;
}

// The forward term of pixel (h, w) is kept: always, or (forward box) where
// (h + dx, w + dy) lies inside the image.
__device__ __forceinline__ bool fwd_kept(const ShiftRec& r, int h, int w, int H, int W) {
    return !r.fbox || (in_range(h + r.dx, H) && in_range(w + r.dy, W));
}

// The forward term whose target is pixel (h, w), i.e. the one owned by
// ((h - dx) mod H, (w - dy) mod W), is kept: always, or (forward box) where
// that owner was reached without wrapping.
__device__ __forceinline__ bool fwd_kept_src(const ShiftRec& r, int h, int w, int H, int W) {
    return !r.fbox || (in_range(h - r.dx, H) && in_range(w - r.dy, W));
}

// The shift stays within a tile window's HALO border (|dx|, |dy| <= HALO).
template <int HALO = kRmax>
__device__ __forceinline__ bool shift_in_lds(const ShiftRec& r) {
    return static_cast<unsigned>(r.dx + HALO) <= 2u * HALO &&
           static_cast<unsigned>(r.dy + HALO) <= 2u * HALO;
}

}  // namespace nsh

// ---------------------------------------------------------------------------
// Host side: error channel and launch helpers (defined in nsh_capi.cpp).
// ---------------------------------------------------------------------------
namespace nsh_host {
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
bool aligned(const void* p, size_t bytes);
int64_t ceil_div(int64_t a, int64_t b);
// Compute units of the current device, queried once per device (256, the
// MI355X count, when there is no device to query).
int compute_units();
}  // namespace nsh_host
