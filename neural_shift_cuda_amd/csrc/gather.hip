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
    stage_shifts(shl, shifts, S, cols, H, W);

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

template <int ES, bool PAIR>
static int g_fwd(const void* guide, const int64_t* sh, int cols, int S, int B, int C, int H, int W,
                 void* out, void* mask, uint64_t one_bits, hipStream_t st) {
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
                       dim3(kThreads), static_cast<size_t>(S) * sizeof(int4), st,
                       static_cast<const T*>(gout), sh, cols, S, B, C, H, W, chunks,
                       static_cast<T*>(grad));
    return nsh_host::check_launch(PAIR ? "pair_gather_backward" : "shift_gather_backward");
}

template <typename T, bool PAIR>
static int g_bwd(const void* gout, const int64_t* sh, int cols, int S, int B, int C, int H, int W,
                 void* grad, hipStream_t st) {
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
