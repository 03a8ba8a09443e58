// scalar.hip -- accumulate_uz_scalar (GASD scalar-per-transform weights).
//
// Semantics (reference csrc/shift_ops_cuda.cu:806-980, ops.py:350-390):
//   U[b,c,p]  = sum_s w[s,b,c] x[b,c,(p+s) mod]        Z[b,c,p] = sum_s w[s,b,c]
//   gx[q]     = sum_s w[s,b,c] gU[(q-s) mod]
//   gw[s,b,c] = sum_{p} gU[p] x[(p+s) mod] + gZ[p]
// The weights are tiny (S*B*C) and x, gU are re-read S times, so the op is
// bound by LDS and VALU work, not HBM.  One workgroup (512 lanes) owns a
// 64 x 32 tile of one (b, c) plane: the tile of x (or gU) with a kRmax
// halo, the plane's S weights and the shift table sit in LDS, and lane tx
// owns the 4 pixels tx, tx + 16, tx + 32, tx + 48 of its row (strided: the
// LDS reads of a wave cover 16 consecutive words per row, free of bank
// conflicts).  gw is a deterministic two-level reduction: each tile forms,
// for every shift, sum over its pixels of gU[p] x[p+s] + gZ[p] (lane sums,
// a wave64 xor-shuffle butterfly, the wave sums in fixed order) into a
// caller workspace of S*B*C*ntiles partials, and a second kernel adds the
// tiles of each (s, b, c) in index order.
#include <initializer_list>

#include "nsh_common.hpp"
#include "scatter.hpp"

namespace nsh {

constexpr int kScVec = 4;
constexpr int kScTpr = 16;
constexpr int kScRows = 32;
using ScG = SGeo<kScVec, kScRows, kScTpr>;
constexpr int kScThreads = ScG::THREADS;

// MODE 0: forward (src = x, writes U and Z);  MODE 1: gx (src = gU).
template <typename T, int MODE>
__global__ __launch_bounds__(kScThreads) void scalar_tile_kernel(
    const void* __restrict__ src_v, const T* __restrict__ w, const int64_t* __restrict__ shifts,
    int cols, int S, int B, int C, int H, int W, int ntw, int nth, void* __restrict__ out0,
    acc_t<T>* __restrict__ out1) {
    using A = acc_t<T>;
    using G = ScG;
    constexpr int VEC = kScVec, TPR = kScTpr;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* wl = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* st = reinterpret_cast<A*>(smem + shift_lds_bytes(S) + static_cast<size_t>(S) * sizeof(A));

    const TileIdx ti = tile_of(xcd_tile(blockIdx.x, gridDim.x), ntw, nth, G::TH, G::TW);
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t BC = static_cast<int64_t>(B) * C;
    for (int s = threadIdx.x; s < S; s += blockDim.x) wl[s] = to_acc(w[s * BC + ti.bc]);
    if (MODE == 0)
        stage_tile<T, A>(st, static_cast<const T*>(src_v) + ti.bc * HW, H, W, ti.h0, ti.w0, G::LH,
                         G::LW, G::PITCH);
    else
        stage_tile<A, A>(st, static_cast<const A*>(src_v) + ti.bc * HW, H, W, ti.h0, ti.w0, G::LH,
                         G::LW, G::PITCH);
    stage_shifts(shl, shifts, S, cols, H, W, false);  // ends with a barrier

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + kRmax) * G::PITCH + tx + kRmax;  // pixel k at lc + k*TPR
    constexpr int sgn = MODE == 0 ? 1 : -1;

    A u[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) u[k] = A(0);
    A z = A(0);
    for (int s = 0; s < S; ++s) {
        const ShiftRec r = read_shift(shl, s);
        const A ws = wl[s];
        z += ws;
        if (shift_in_lds(r)) {
            const A* sr = st + lc + sgn * (r.dx * G::PITCH + r.dy);
#pragma unroll
            for (int k = 0; k < VEC; ++k) u[k] = fma_acc(ws, sr[k * TPR], u[k]);
        } else {
            int hh = MODE == 0 ? h + r.dxm : h - r.dxm;
            hh = MODE == 0 ? (hh >= H ? hh - H : hh) : (hh < 0 ? hh + H : hh);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                if (!px.act[k]) continue;
                const int wq = ti.w0 + tx + k * TPR;
                int ww = MODE == 0 ? wq + r.dym : wq - r.dym;
                ww = MODE == 0 ? (ww >= W ? ww - W : ww) : (ww < 0 ? ww + W : ww);
                const uint32_t i = static_cast<uint32_t>(hh) * W + ww;
                const A v = MODE == 0 ? to_acc(static_cast<const T*>(src_v)[ti.bc * HW + i])
                                      : static_cast<const A*>(src_v)[ti.bc * HW + i];
                u[k] = fma_acc(ws, v, u[k]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        if (!px.act[k]) continue;
        const int64_t o = ti.bc * HW + px.own[k];
        if (MODE == 0) {
            static_cast<A*>(out0)[o] = u[k];
            out1[o] = z;
        } else {
            static_cast<T*>(out0)[o] = from_acc<T>(u[k]);
        }
    }
}

// Sum over the 64 lanes of a wave, returned uniform (in every lane).
// fp32: DPP adds (row_shr 1, 2, 4, 8 leave each 16-lane row's sum in its
// lane 15; row_bcast 15 and 31 fold the rows into lane 63), all VALU work;
// fp64: xor butterfly.  The order of additions is fixed.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xf, true);
    return v + __int_as_float(moved);
}
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0x111, 0xf>(v);  // row_shr:1
    v = dpp_add<0x112, 0xf>(v);  // row_shr:2
    v = dpp_add<0x114, 0xf>(v);  // row_shr:4
    v = dpp_add<0x118, 0xf>(v);  // row_shr:8
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// gw partials of one tile: part[(s*BC + bc)*ntp + tile] =
//   sum_{p in tile} gU[p] x[(p+s) mod] + gZ[p]
// Shifts go in blocks of kScGwBlk: each wave leaves its sums in LDS, then
// kScGwBlk lanes add the waves in order.
constexpr int kScGwBlk = 8;
constexpr int kScWaves = kScThreads / 64;

template <typename T>
__global__ __launch_bounds__(kScThreads) void scalar_gw_tile_kernel(
    const T* __restrict__ x, const acc_t<T>* __restrict__ gU, const acc_t<T>* __restrict__ gZ,
    const int64_t* __restrict__ shifts, int cols, int S, int B, int C, int H, int W, int ntw,
    int nth, acc_t<T>* __restrict__ part) {
    using A = acc_t<T>;
    using G = ScG;
    constexpr int VEC = kScVec, TPR = kScTpr;
    extern __shared__ __align__(16) unsigned char smem[];
    int4* shl = reinterpret_cast<int4*>(smem);
    A* xt = reinterpret_cast<A*>(smem + shift_lds_bytes(S));
    A* red = xt + G::TILE;  // [kScWaves][kScGwBlk + 1]

    // plain tile order: the partial index is the tile's position in its plane
    const int64_t ntp = static_cast<int64_t>(ntw) * nth;
    const TileIdx ti = tile_of(blockIdx.x, ntw, nth, G::TH, G::TW);
    const int64_t tile = blockIdx.x - ti.bc * ntp;
    const int64_t HW = static_cast<int64_t>(H) * W;
    const int64_t BC = static_cast<int64_t>(B) * C;
    const T* xp = x + ti.bc * HW;
    stage_tile<T, A>(xt, xp, H, W, ti.h0, ti.w0, G::LH, G::LW, G::PITCH);
    stage_shifts(shl, shifts, S, cols, H, W, false);  // ends with a barrier

    const int tx = threadIdx.x % TPR;
    const int ty = threadIdx.x / TPR;
    const int h = ti.h0 + ty;
    const LanePix<VEC, TPR> px = lane_pixels<VEC, TPR>(h, ti.w0, tx, H, W);
    const int lc = (ty + kRmax) * G::PITCH + tx + kRmax;
    const int wave = threadIdx.x / 64;
    const int lane = threadIdx.x & 63;

    A gu[VEC];
    A gz = A(0);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        gu[k] = px.act[k] ? gU[ti.bc * HW + px.own[k]] : A(0);
        gz += px.act[k] ? gZ[ti.bc * HW + px.own[k]] : A(0);
    }
    // sum of gZ over the tile (added to every shift's partial)
    gz = wave_sum(gz);
    if (lane == 0) red[wave * (kScGwBlk + 1) + kScGwBlk] = gz;
    __syncthreads();
    A gz_tile = A(0);
#pragma unroll
    for (int i = 0; i < kScWaves; ++i) gz_tile += red[i * (kScGwBlk + 1) + kScGwBlk];

    for (int s0 = 0; s0 < S; s0 += kScGwBlk) {
#pragma unroll
        for (int j = 0; j < kScGwBlk; ++j) {
            const int s = s0 + j;
            if (s >= S) break;
            const ShiftRec r = read_shift(shl, s);
            A acc = A(0);
            if (shift_in_lds(r)) {
                const A* sr = xt + lc + r.dx * G::PITCH + r.dy;
#pragma unroll
                for (int k = 0; k < VEC; ++k) acc = fma_acc(gu[k], sr[k * TPR], acc);
            } else {
                int hh = h + r.dxm;
                hh -= hh >= H ? H : 0;
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    if (!px.act[k]) continue;
                    int ww = ti.w0 + tx + k * TPR + r.dym;
                    ww -= ww >= W ? W : 0;
                    acc = fma_acc(gu[k], to_acc(xp[static_cast<uint32_t>(hh) * W + ww]), acc);
                }
            }
            acc = wave_sum(acc);
            if (lane == 0) red[wave * (kScGwBlk + 1) + j] = acc;
        }
        __syncthreads();
        if (threadIdx.x < kScGwBlk && s0 + threadIdx.x < S) {
            A t = A(0);
#pragma unroll
            for (int i = 0; i < kScWaves; ++i) t += red[i * (kScGwBlk + 1) + threadIdx.x];
            const int64_t sbc = static_cast<int64_t>(s0 + threadIdx.x) * BC + ti.bc;
            part[sbc * ntp + tile] = t + gz_tile;
        }
        __syncthreads();
    }
}

template <typename T>
__global__ __launch_bounds__(256) void scalar_gw_final_kernel(const acc_t<T>* __restrict__ partial,
                                                              int64_t n, int nsplit,
                                                              T* __restrict__ gw) {
    using A = acc_t<T>;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    A t = A(0);
    for (int k = 0; k < nsplit; ++k) t += partial[i * nsplit + k];
    gw[i] = from_acc<T>(t);
}

static void sc_tiles(int H, int W, int* ntw, int* nth) {
    *ntw = static_cast<int>(nsh_host::ceil_div(W, ScG::TW));
    *nth = static_cast<int>(nsh_host::ceil_div(H, ScG::TH));
}

template <typename T, int MODE>
static int s_tile(const void* src, const void* w, const int64_t* sh, int cols, int S, int B, int C,
                  int H, int W, void* out0, void* out1, hipStream_t st) {
    using A = acc_t<T>;
    int ntw, nth;
    sc_tiles(H, W, &ntw, &nth);
    const int64_t tiles = static_cast<int64_t>(B) * C * ntw * nth;
    const size_t lds = shift_lds_bytes(S) + static_cast<size_t>(S) * sizeof(A) +
                       static_cast<size_t>(ScG::TILE) * sizeof(A);
    hipLaunchKernelGGL((scalar_tile_kernel<T, MODE>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kScThreads), lds, st, src, static_cast<const T*>(w), sh, cols, S, B, C,
                       H, W, ntw, nth, out0, static_cast<A*>(out1));
    return nsh_host::check_launch(MODE == 0 ? "accumulate_uz_scalar_forward"
                                            : "accumulate_uz_scalar_backward");
}

// Partials per (s, b, c): the tiles of one plane.
static int scalar_splits(int64_t H, int64_t W) {
    int ntw, nth;
    sc_tiles(static_cast<int>(H), static_cast<int>(W), &ntw, &nth);
    return ntw * nth;
}

template <typename T>
static int s_gw(const void* x, const void* gU, const void* gZ, const int64_t* sh, int cols, int S,
                int B, int C, int H, int W, void* gw, void* partial, hipStream_t st) {
    using A = acc_t<T>;
    int ntw, nth;
    sc_tiles(H, W, &ntw, &nth);
    const int nsplit = ntw * nth;
    const int64_t tiles = static_cast<int64_t>(B) * C * nsplit;
    const size_t lds = shift_lds_bytes(S) +
                       (static_cast<size_t>(ScG::TILE) + kScWaves * (kScGwBlk + 1)) * sizeof(A);
    hipLaunchKernelGGL((scalar_gw_tile_kernel<T>), dim3(static_cast<unsigned>(tiles)),
                       dim3(kScThreads), lds, st, static_cast<const T*>(x),
                       static_cast<const A*>(gU), static_cast<const A*>(gZ), sh, cols, S, B, C, H,
                       W, ntw, nth, static_cast<A*>(partial));
    if (int rc = nsh_host::check_launch("accumulate_uz_scalar_backward (gw partial)")) return rc;
    const int64_t n = static_cast<int64_t>(S) * B * C;
    hipLaunchKernelGGL((scalar_gw_final_kernel<T>),
                       dim3(static_cast<unsigned>(nsh_host::ceil_div(n, 256))), dim3(256), 0, st,
                       static_cast<const A*>(partial), n, nsplit, static_cast<T*>(gw));
    return nsh_host::check_launch("accumulate_uz_scalar_backward (gw final)");
}

}  // namespace nsh

using nsh_host::fail;

static int s_check(const char* op, int64_t S, int64_t cols, int64_t B, int64_t C, int64_t H,
                   int64_t W, int dtype) {
    if (S < 1 || S > 1024) return fail(NSH_ERR_INVALID, "%s: tree reduction requires 1 <= S <= 1024", op);
    if (cols != 2 && cols != 3) return fail(NSH_ERR_INVALID, "%s: shifts must have 2 or 3 columns", op);
    if (B < 1 || C < 1 || H < 1 || W < 1) return fail(NSH_ERR_INVALID, "%s: empty tensor", op);
    if (dtype < NSH_DTYPE_FLOAT16 || dtype > NSH_DTYPE_FLOAT64)
        return fail(NSH_ERR_INVALID, "%s: unsupported dtype code %d", op, dtype);
    const int64_t es = dtype == NSH_DTYPE_FLOAT64 ? 8 : 4;
    if (H * W * es >= (int64_t(1) << 31))
        return fail(NSH_ERR_INVALID, "%s: one (b, c) plane must stay below 2^31 bytes", op);
    if (B * C > (int64_t(1) << 24)) return fail(NSH_ERR_INVALID, "%s: B*C too large", op);
    return NSH_OK;
}

extern "C" int nsh_scalar_backward_splits(int64_t H, int64_t W) { return nsh::scalar_splits(H, W); }

extern "C" int nsh_accumulate_uz_scalar_forward(const void* x, const void* weights,
                                                const int64_t* shifts, int64_t S,
                                                int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                                int64_t W, int dtype, void* U, void* Z,
                                                void* stream) {
    if (int rc = s_check("accumulate_uz_scalar", S, shift_cols, B, C, H, W, dtype)) return rc;
    if (!x || !weights || !shifts || !U || !Z)
        return fail(NSH_ERR_INVALID, "accumulate_uz_scalar: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int s = (int)S, c = (int)shift_cols, b = (int)B, ch = (int)C, h = (int)H, w = (int)W;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16: return nsh::s_tile<nsh::f16, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
        case NSH_DTYPE_BFLOAT16: return nsh::s_tile<nsh::bf16, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
        case NSH_DTYPE_FLOAT32: return nsh::s_tile<float, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
        default: return nsh::s_tile<double, 0>(x, weights, shifts, c, s, b, ch, h, w, U, Z, st);
    }
}

extern "C" int nsh_accumulate_uz_scalar_backward(const void* x, const void* weights,
                                                 const void* grad_U, const void* grad_Z,
                                                 const int64_t* shifts, int64_t S,
                                                 int64_t shift_cols, int64_t B, int64_t C,
                                                 int64_t H, int64_t W, int dtype, void* grad_x,
                                                 void* grad_w, void* grad_w_partial, void* stream) {
    if (int rc = s_check("accumulate_uz_scalar_backward", S, shift_cols, B, C, H, W, dtype)) return rc;
    if (!x || !weights || !grad_U || !grad_Z || !shifts || !grad_x || !grad_w || !grad_w_partial)
        return fail(NSH_ERR_INVALID, "accumulate_uz_scalar_backward: null pointer argument");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int s = (int)S, c = (int)shift_cols, b = (int)B, ch = (int)C, h = (int)H, w = (int)W;
    int rc = NSH_OK;
    switch (dtype) {
        case NSH_DTYPE_FLOAT16:
            rc = nsh::s_tile<nsh::f16, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<nsh::f16>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
        case NSH_DTYPE_BFLOAT16:
            rc = nsh::s_tile<nsh::bf16, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<nsh::bf16>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
        case NSH_DTYPE_FLOAT32:
            rc = nsh::s_tile<float, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<float>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
        default:
            rc = nsh::s_tile<double, 1>(grad_U, weights, shifts, c, s, b, ch, h, w, grad_x, nullptr, st);
            return rc ? rc : nsh::s_gw<double>(x, grad_U, grad_Z, shifts, c, s, b, ch, h, w, grad_w, grad_w_partial, st);
    }
}
