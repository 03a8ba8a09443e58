/*
 * oracle.c -- CPU restatement of the neural_shift_cuda shift-window operators.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing under neural_shift_cuda_amd/ may load or
 * call this library; it exists so that tests/, the smoke check and the CPU
 * baseline leg of bench.py can check the HIP kernels against an independent
 * statement of the reference algorithm.
 *
 * Every function states the reference code it follows.  Paths are relative to
 * the reference repository root (trishitmg/neural_shift_cuda):
 *   ops.py          = neural_shift_cuda/ops.py
 *   metropolis.py   = neural_shift_cuda/metropolis.py
 *   cuda.cu         = csrc/shift_ops_cuda.cu
 *   metro.cu        = csrc/metropolis_cuda.cu
 *
 * Conventions shared by every op (ops.py:580-586, cuda.cu:4-22):
 *   - tensors are contiguous NCHW; weights are shift-major, plane s*B+b of a
 *     (S*B, C, H, W) tensor; Metropolis weights are batch-major (B,S,C,H,W);
 *   - a shift row is (dx, dy[, has_inv]); the forward term of pixel (h, w)
 *     reads x[(h+dx) mod H, (w+dy) mod W] (gather convention);
 *   - box(h, w) is 1 iff 0 <= h < H and 0 <= w < W (the F.pad(ones) mask).
 *
 * Two numeric modes exist per op: element type float (the reference's fp32
 * arithmetic, including its pairwise-tree summation order where the reference
 * CPU fallback uses one) and double (used by the tests as a near-exact value
 * for tolerance checks of fp32 results).  The file is compiled with
 * -ffp-contract=off so that a*b+c is never fused: the reference CPU fallback
 * rounds every product and every sum separately.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

static inline int64_t wrapi(int64_t i, int64_t n) {
    int64_t r = i % n;
    return r < 0 ? r + n : r;
}
static inline int in_range(int64_t i, int64_t n) { return i >= 0 && i < n; }

static inline void shift_row(const int64_t* shifts, int64_t stride, int64_t s,
                             int64_t* dx, int64_t* dy, int* inv) {
    *dx = shifts[s * stride + 0];
    *dy = shifts[s * stride + 1];
    *inv = (stride >= 3) ? (shifts[s * stride + 2] != 0) : 0;
}

EXPORT void nso_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

EXPORT int nso_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------
 * shift_gather / pair_gather forward: byte copies, bit-exact for any dtype.
 *   gs[s*B+b, c, h, w]   = guide[b, c, (h+dx) mod H, (w+dy) mod W]
 *   mask[s*B+b, 0, h, w] = box(h+dx, w+dy)  (in the guide dtype)
 * Follows shift_gather_reference (ops.py:95-135): circular F.pad by R then a
 * window slice at (R+dx, R+dy) equals the modular gather for |dx|,|dy| <= R;
 * the R==0 branch (ops.py:112-116) is the same formula with an all-ones mask.
 * pair_gather_reference (ops.py:138-154) puts guide[b] in channels [0, C)
 * and the shifted guide in [C, 2C).
 * ---------------------------------------------------------------------- */
static void gather_impl(const uint8_t* guide, int64_t es, const int64_t* shifts,
                        int64_t S, int64_t stride, int64_t B, int64_t C,
                        int64_t H, int64_t W, uint8_t* out, uint8_t* mask,
                        const uint8_t* one, const uint8_t* zero, int pair) {
    const int64_t HW = H * W;
    const int64_t Cout = pair ? 2 * C : C;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t s = 0; s < S; ++s) {
        for (int64_t b = 0; b < B; ++b) {
            int64_t dx, dy;
            int inv;
            shift_row(shifts, stride, s, &dx, &dy, &inv);
            uint8_t* o = out + ((s * B + b) * Cout) * HW * es;
            for (int64_t c = 0; c < C; ++c) {
                const uint8_t* g = guide + (b * C + c) * HW * es;
                uint8_t* oc = o + (pair ? (C + c) : c) * HW * es;
                for (int64_t h = 0; h < H; ++h) {
                    const int64_t sh = wrapi(h + dx, H);
                    for (int64_t w = 0; w < W; ++w) {
                        const int64_t sw = wrapi(w + dy, W);
                        memcpy(oc + (h * W + w) * es, g + (sh * W + sw) * es, es);
                    }
                }
                if (pair) memcpy(o + c * HW * es, g, HW * es);
            }
            if (mask) {
                uint8_t* m = mask + (s * B + b) * HW * es;
                for (int64_t h = 0; h < H; ++h)
                    for (int64_t w = 0; w < W; ++w) {
                        const int ok = in_range(h + dx, H) && in_range(w + dy, W);
                        memcpy(m + (h * W + w) * es, ok ? one : zero, es);
                    }
            }
        }
    }
}

EXPORT void nso_shift_gather_fwd(const void* guide, int64_t es, const int64_t* shifts,
                                 int64_t S, int64_t stride, int64_t B, int64_t C,
                                 int64_t H, int64_t W, void* out, void* mask,
                                 const void* one, const void* zero) {
    gather_impl(guide, es, shifts, S, stride, B, C, H, W, out, mask, one, zero, 0);
}

EXPORT void nso_pair_gather_fwd(const void* guide, int64_t es, const int64_t* shifts,
                                int64_t S, int64_t stride, int64_t B, int64_t C,
                                int64_t H, int64_t W, void* out, void* mask,
                                const void* one, const void* zero) {
    gather_impl(guide, es, shifts, S, stride, B, C, H, W, out, mask, one, zero, 1);
}

/* ------------------------------------------------------------------------
 * The remaining ops are written once per element type T via a macro.
 * ---------------------------------------------------------------------- */

/* Pairwise adjacent-pair tree over buf[0..n), odd tail carried to the end of
 * the next level: _tree_sum (ops.py:77-92). */
#define DEFINE_TREE(T, SUF)                                                   \
    static T tree_sum_##SUF(T* buf, int64_t n) {                              \
        while (n > 1) {                                                       \
            const int64_t half = n / 2;                                       \
            for (int64_t i = 0; i < half; ++i) buf[i] = buf[2 * i] + buf[2 * i + 1]; \
            if (n & 1) {                                                      \
                buf[half] = buf[n - 1];                                       \
                n = half + 1;                                                 \
            } else {                                                          \
                n = half;                                                     \
            }                                                                 \
        }                                                                     \
        return buf[0];                                                        \
    }

DEFINE_TREE(float, f32)
DEFINE_TREE(double, f64)

#define DEFINE_OPS(T, SUF, LOG, EXP, ISNAN, ISINF, ISFINITE)                  \
                                                                              \
/* shift_gather backward: g[b,c,q] = sum_s gout[s*B+b, c, (q-s) mod]         \
 * (the adjoint of the modular gather; cuda.cu:165-203 states the same sum). */\
EXPORT void nso_shift_gather_bwd_##SUF(                                       \
    const T* gout, const int64_t* shifts, int64_t S, int64_t stride,          \
    int64_t B, int64_t C, int64_t H, int64_t W, T* g) {                       \
    const int64_t HW = H * W;                                                 \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c)                                       \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, stride, s, &dx, &dy, &inv);         \
                        acc += gout[((s * B + b) * C + c) * HW +              \
                                    wrapi(h - dx, H) * W + wrapi(w - dy, W)]; \
                    }                                                         \
                    g[(b * C + c) * HW + h * W + w] = acc;                    \
                }                                                             \
}                                                                             \
                                                                              \
/* pair_gather backward: center half plus the shifted half's adjoint         \
 * (the gradient of pair_gather_reference, ops.py:138-154). */               \
EXPORT void nso_pair_gather_bwd_##SUF(                                        \
    const T* gout, const int64_t* shifts, int64_t S, int64_t stride,          \
    int64_t B, int64_t C, int64_t H, int64_t W, T* g) {                       \
    const int64_t HW = H * W;                                                 \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c)                                       \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, stride, s, &dx, &dy, &inv);         \
                        const T* go = gout + ((s * B + b) * 2 * C) * HW;      \
                        acc += go[c * HW + h * W + w];                        \
                        acc += go[(C + c) * HW + wrapi(h - dx, H) * W +       \
                                  wrapi(w - dy, W)];                          \
                    }                                                         \
                    g[(b * C + c) * HW + h * W + w] = acc;                    \
                }                                                             \
}                                                                             \
                                                                              \
/* accumulate_uz forward, reference CPU fallback order (ops.py:157-206):     \
 *   terms [fwd_0, inv_0?, fwd_1, inv_1?, ...], every has_inv row adds an    \
 *   inverse term even where the box zeroes it; U, Z are _tree_sum's of the   \
 *   term stacks.  fwd: w_s[p] * x[(p+s) mod];                                \
 *   inv: (w_s[(p-s) mod] * box(p-s)) * x[(p-s) mod]   (ops.py:192-203).      \
 * scratch must hold 2*(2S) elements per thread; it is allocated here. */     \
EXPORT int nso_accumulate_uz_fwd_##SUF(                                       \
    const T* x, const T* wt, const int64_t* shifts, int64_t S,                \
    int64_t B, int64_t C, int64_t H, int64_t W, T* U, T* Z) {                 \
    const int64_t HW = H * W;                                                 \
    int fail = 0;                                                             \
    _Pragma("omp parallel")                                                   \
    {                                                                         \
        T* ub = (T*)malloc(sizeof(T) * 2 * (size_t)S);                        \
        T* zb = (T*)malloc(sizeof(T) * 2 * (size_t)S);                        \
        if (!ub || !zb) {                                                     \
            _Pragma("omp atomic write")                                       \
            fail = 1;                                                         \
        } else {                                                              \
        _Pragma("omp for collapse(2) schedule(static)")                       \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c)                                   \
                for (int64_t h = 0; h < H; ++h)                               \
                    for (int64_t w = 0; w < W; ++w) {                         \
                        const T* xb = x + (b * C + c) * HW;                   \
                        int64_t n = 0;                                        \
                        for (int64_t s = 0; s < S; ++s) {                     \
                            int64_t dx, dy; int inv;                          \
                            shift_row(shifts, 3, s, &dx, &dy, &inv);          \
                            const T* ws = wt + ((s * B + b) * C + c) * HW;    \
                            const T wf = ws[h * W + w];                       \
                            const T vf = xb[wrapi(h + dx, H) * W + wrapi(w + dy, W)]; \
                            ub[n] = wf * vf;                                  \
                            zb[n] = wf;                                       \
                            ++n;                                              \
                            if (inv) {                                        \
                                const int64_t ih = wrapi(h - dx, H);          \
                                const int64_t iw = wrapi(w - dy, W);          \
                                const T cb = (in_range(h - dx, H) &&          \
                                              in_range(w - dy, W)) ? 1 : 0;   \
                                const T wi = ws[ih * W + iw] * cb;            \
                                ub[n] = wi * xb[ih * W + iw];                 \
                                zb[n] = wi;                                   \
                                ++n;                                          \
                            }                                                 \
                        }                                                     \
                        const int64_t o = (b * C + c) * HW + h * W + w;       \
                        U[o] = tree_sum_##SUF(ub, n);                         \
                        Z[o] = tree_sum_##SUF(zb, n);                         \
                    }                                                         \
        }                                                                     \
        free(ub);                                                             \
        free(zb);                                                             \
    }                                                                         \
    return fail ? -1 : 0;                                                     \
}                                                                             \
                                                                              \
/* accumulate_uz backward, the analytic adjoint of the forward above:         \
 *   gx[q]  = sum_s w_s[(q-s) mod] gU[(q-s) mod]                              \
 *          + sum_{s:inv, box(q+s)} w_s[q] gU[q+s]                            \
 *   gw_s[q] = x[(q+s) mod] gU[q] + gZ[q]                                     \
 *          + [inv and box(q+s)] (x[q] gU[q+s] + gZ[q+s])                     \
 * The forward term keeps its circular derivative (no box), as in            \
 * cuda.cu:371-373 and 441-442; the inverse branch is box-masked             \
 * (cuda.cu:384-395 and 447-454).  Serial summation order over s. */         \
EXPORT void nso_accumulate_uz_bwd_##SUF(                                      \
    const T* x, const T* wt, const T* gU, const T* gZ,                        \
    const int64_t* shifts, int64_t S, int64_t B, int64_t C, int64_t H,        \
    int64_t W, T* gx, T* gw) {                                                \
    const int64_t HW = H * W;                                                 \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c) {                                     \
            const int64_t bc = (b * C + c) * HW;                              \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = wt + ((s * B + b) * C + c) * HW;        \
                        const int64_t o = wrapi(h - dx, H) * W + wrapi(w - dy, W); \
                        acc += ws[o] * gU[bc + o];                            \
                        if (inv && in_range(h + dx, H) && in_range(w + dy, W)) \
                            acc += ws[h * W + w] *                            \
                                   gU[bc + (h + dx) * W + (w + dy)];          \
                    }                                                         \
                    gx[bc + h * W + w] = acc;                                 \
                }                                                             \
        }                                                                     \
    _Pragma("omp parallel for collapse(3) schedule(static)")                  \
    for (int64_t s = 0; s < S; ++s)                                           \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c) {                                 \
                int64_t dx, dy; int inv;                                      \
                shift_row(shifts, 3, s, &dx, &dy, &inv);                      \
                const int64_t bc = (b * C + c) * HW;                          \
                T* g = gw + ((s * B + b) * C + c) * HW;                       \
                for (int64_t h = 0; h < H; ++h)                               \
                    for (int64_t w = 0; w < W; ++w) {                         \
                        const int64_t q = bc + h * W + w;                     \
                        T v = x[bc + wrapi(h + dx, H) * W + wrapi(w + dy, W)] \
                              * gU[q] + gZ[q];                                \
                        if (inv && in_range(h + dx, H) && in_range(w + dy, W)) { \
                            const int64_t o = bc + (h + dx) * W + (w + dy);   \
                            v += x[q] * gU[o] + gZ[o];                        \
                        }                                                     \
                        g[h * W + w] = v;                                     \
                    }                                                         \
            }                                                                 \
}                                                                             \
                                                                              \
/* normalized_accumulate_uz forward.  Term list as in the accumulate        \
 * forward; each term has a key and a value.                                  \
 *   policy 0 = reference CPU fallback (ops.py:234-320): key = log w for     \
 *     w > 0 and -inf otherwise (positive mode, ops.py:227-231), key = w in  \
 *     log mode; the inverse term is masked to -inf (log) or multiplied by   \
 *     the box (positive); m = NaN-propagating max; empty row (m == -inf)    \
 *     gives D = 0, log_C = -inf; otherwise a = exp(key - m),                 \
 *     D = tree(a v) / tree(a), log_C = m + log(tree(a)).                     \
 *   policy 1 = reference GPU kernel (cuda.cu:474-653): positive-mode keys   \
 *     are the weights themselves (NaN for a negative weight), a = w / m;     \
 *     log mode a = exp(l - m); masked terms (w == 0 / l == -inf) are        \
 *     skipped; empty row gives D = 0, log_C = -inf; a non-finite max or     \
 *     sum gives NaN; log_C = log(m) + log(z) (positive) or m + log(z).       \
 * Sums use the pairwise tree in both policies. */                           \
EXPORT int nso_normalized_fwd_##SUF(                                          \
    const T* x, const T* wt, const int64_t* shifts, int64_t S,                \
    int64_t B, int64_t C, int64_t H, int64_t W, int log_weights, int policy,  \
    T* D, T* logC) {                                                          \
    const int64_t HW = H * W;                                                 \
    const T NEG_INF = -(T)INFINITY;                                           \
    const T QNAN = (T)NAN;                                                    \
    int fail = 0;                                                             \
    _Pragma("omp parallel")                                                   \
    {                                                                         \
        T* key = (T*)malloc(sizeof(T) * 2 * (size_t)S);                       \
        T* val = (T*)malloc(sizeof(T) * 2 * (size_t)S);                       \
        T* ub = (T*)malloc(sizeof(T) * 2 * (size_t)S);                        \
        T* zb = (T*)malloc(sizeof(T) * 2 * (size_t)S);                        \
        if (!key || !val || !ub || !zb) {                                     \
            _Pragma("omp atomic write")                                       \
            fail = 1;                                                         \
        } else {                                                              \
        _Pragma("omp for collapse(2) schedule(static)")                       \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c)                                   \
                for (int64_t h = 0; h < H; ++h)                               \
                    for (int64_t w = 0; w < W; ++w) {                         \
                        const T* xb = x + (b * C + c) * HW;                   \
                        int64_t n = 0;                                        \
                        for (int64_t s = 0; s < S; ++s) {                     \
                            int64_t dx, dy; int inv;                          \
                            shift_row(shifts, 3, s, &dx, &dy, &inv);          \
                            const T* ws = wt + ((s * B + b) * C + c) * HW;    \
                            T wv = ws[h * W + w];                             \
                            key[n] = wv;                                      \
                            val[n] = xb[wrapi(h + dx, H) * W + wrapi(w + dy, W)]; \
                            ++n;                                              \
                            if (inv) {                                        \
                                const int64_t ih = wrapi(h - dx, H);          \
                                const int64_t iw = wrapi(w - dy, W);          \
                                const int ok = in_range(h - dx, H) &&         \
                                               in_range(w - dy, W);           \
                                T wi = ws[ih * W + iw];                       \
                                if (log_weights) wi = ok ? wi : NEG_INF;      \
                                else if (policy == 0) wi = wi * (T)(ok ? 1 : 0); \
                                else wi = ok ? wi : (T)0;                     \
                                key[n] = wi;                                  \
                                val[n] = xb[ih * W + iw];                     \
                                ++n;                                          \
                            }                                                 \
                        }                                                     \
                        const int64_t o = (b * C + c) * HW + h * W + w;       \
                        if (policy == 0) {                                    \
                            T m = NEG_INF;                                    \
                            int nan_seen = 0;                                 \
                            for (int64_t t = 0; t < n; ++t) {                 \
                                if (!log_weights)                             \
                                    key[t] = key[t] > 0 ? LOG(key[t]) : NEG_INF; \
                                if (ISNAN(key[t])) nan_seen = 1;              \
                                else if (key[t] > m) m = key[t];              \
                            }                                                 \
                            if (nan_seen) m = QNAN;                           \
                            const int empty = ISINF(m) && m < 0;              \
                            for (int64_t t = 0; t < n; ++t) {                 \
                                const T a = empty ? (T)0 : EXP(key[t] - m);   \
                                ub[t] = a * val[t];                           \
                                zb[t] = a;                                    \
                            }                                                 \
                            const T u = tree_sum_##SUF(ub, n);                \
                            const T z = tree_sum_##SUF(zb, n);                \
                            D[o] = empty ? (T)0 : u / z;                      \
                            logC[o] = empty ? NEG_INF : m + LOG(z);           \
                        } else {                                              \
                            /* reduction_key / max_propagate_nan           \
                             * (cuda.cu:484-503, 553-580) */                 \
                            T m = NEG_INF;                                    \
                            int nan_seen = 0;                                 \
                            for (int64_t t = 0; t < n; ++t) {                 \
                                T k = key[t];                                 \
                                if (!log_weights && !(k >= 0)) k = QNAN;      \
                                if (ISNAN(k)) nan_seen = 1;                   \
                                else if (k > m) m = k;                        \
                            }                                                 \
                            if (nan_seen) m = QNAN;                           \
                            const int empty = log_weights ? (m == NEG_INF)    \
                                                          : (m == 0);         \
                            int64_t k2 = 0;                                   \
                            if (!empty) {                                     \
                                for (int64_t t = 0; t < n; ++t) {             \
                                    const T v = key[t];                       \
                                    if (log_weights ? (v == NEG_INF) : (v == 0)) \
                                        continue;                             \
                                    const T a = log_weights ? EXP(v - m) : v / m; \
                                    ub[k2] = a * val[t];                      \
                                    zb[k2] = a;                               \
                                    ++k2;                                     \
                                }                                             \
                            }                                                 \
                            const T u = k2 ? tree_sum_##SUF(ub, k2) : (T)0;   \
                            const T z = k2 ? tree_sum_##SUF(zb, k2) : (T)0;   \
                            if (empty && z == 0) {                            \
                                D[o] = 0;                                     \
                                logC[o] = NEG_INF;                            \
                            } else if (ISFINITE(m) && z > 0 && ISFINITE(z)) { \
                                D[o] = u / z;                                 \
                                logC[o] = (log_weights ? m : LOG(m)) + LOG(z); \
                            } else {                                          \
                                D[o] = QNAN;                                  \
                                logC[o] = QNAN;                               \
                            }                                                 \
                        }                                                     \
                    }                                                         \
        }                                                                     \
        free(key); free(val); free(ub); free(zb);                             \
    }                                                                         \
    return fail ? -1 : 0;                                                     \
}                                                                             \
                                                                              \
/* normalized backward, the analytic gradient stated by the reference GPU     \
 * kernels (cuda.cu:505-525, 655-791):                                         \
 *   f(v, L) = 0 if lw(v) == -inf or L == -inf, else exp(lw(v) - L), with     \
 *   lw(v) = v (log mode) or log v / -inf / NaN for v >0 / ==0 / <0;          \
 *   gx[q] = sum_s f(w_s[o], L[o]) gD[o] at o = (q-s) mod                     \
 *         + [inv and box(q+s)] f(w_s[q], L[q+s]) gD[q+s];                    \
 *   gw_s[q] = 0 if lw(w_s[q]) == -inf, else                                  \
 *     F(q) score(q, x[(q+s) mod]) + [inv and box(q+s)] F(q+s) score(q+s, x[q])\
 *   with score(o, v) = gD[o] (v - D[o]) + gLogC[o] and                       \
 *   F(o) = f(w_s[q], L[o]) (log mode) or exp(-L[o]) (positive mode). */      \
EXPORT void nso_normalized_bwd_##SUF(                                         \
    const T* x, const T* wt, const T* Dv, const T* Lv, const T* gD,           \
    const T* gL, const int64_t* shifts, int64_t S, int64_t B, int64_t C,      \
    int64_t H, int64_t W, int log_weights, T* gx, T* gw) {                    \
    const int64_t HW = H * W;                                                 \
    const T NEG_INF = -(T)INFINITY;                                           \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c) {                                     \
            const int64_t bc = (b * C + c) * HW;                              \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = wt + ((s * B + b) * C + c) * HW;        \
                        const int64_t o = wrapi(h - dx, H) * W + wrapi(w - dy, W); \
                        acc += nso_frac_##SUF(ws[o], Lv[bc + o], log_weights, \
                                              NEG_INF) * gD[bc + o];          \
                        if (inv && in_range(h + dx, H) && in_range(w + dy, W)) { \
                            const int64_t oi = bc + (h + dx) * W + (w + dy);  \
                            acc += nso_frac_##SUF(ws[h * W + w], Lv[oi],      \
                                                  log_weights, NEG_INF) * gD[oi]; \
                        }                                                     \
                    }                                                         \
                    gx[bc + h * W + w] = acc;                                 \
                }                                                             \
        }                                                                     \
    _Pragma("omp parallel for collapse(3) schedule(static)")                  \
    for (int64_t s = 0; s < S; ++s)                                           \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c) {                                 \
                int64_t dx, dy; int inv;                                      \
                shift_row(shifts, 3, s, &dx, &dy, &inv);                      \
                const int64_t bc = (b * C + c) * HW;                          \
                const T* ws = wt + ((s * B + b) * C + c) * HW;                \
                T* g = gw + ((s * B + b) * C + c) * HW;                       \
                for (int64_t h = 0; h < H; ++h)                               \
                    for (int64_t w = 0; w < W; ++w) {                         \
                        const T v = ws[h * W + w];                            \
                        const T lw = nso_aslog_##SUF(v, log_weights, NEG_INF); \
                        if (lw == NEG_INF) { g[h * W + w] = 0; continue; }    \
                        const int64_t q = bc + h * W + w;                     \
                        const T sf = gD[q] * (x[bc + wrapi(h + dx, H) * W +   \
                                                 wrapi(w + dy, W)] - Dv[q]) + gL[q]; \
                        T r = (log_weights ? nso_frac_##SUF(v, Lv[q], 1, NEG_INF) \
                                           : EXP(-Lv[q])) * sf;               \
                        if (inv && in_range(h + dx, H) && in_range(w + dy, W)) { \
                            const int64_t oi = bc + (h + dx) * W + (w + dy);  \
                            const T si = gD[oi] * (x[q] - Dv[oi]) + gL[oi];   \
                            r += (log_weights ? nso_frac_##SUF(v, Lv[oi], 1, NEG_INF) \
                                              : EXP(-Lv[oi])) * si;           \
                        }                                                     \
                        g[h * W + w] = r;                                     \
                    }                                                         \
            }                                                                 \
}                                                                             \
                                                                              \
/* Metropolis aggregate (inference form), following the reference kernels    \
 * metro.cu:70-186 and metropolis_aggregate_torch (metropolis.py:54-114):     \
 *   d[p] = sum_s kf w_s[p] + sum_{s:inv} ki w_s[(p-s) mod]                   \
 *   per edge wk = w / max(max(d_p, d_j), eps); khat += wk img[j]; dhat += wk \
 *   forward j = (p+s) mod with weight w_s[p]; inverse j = (p-s) mod with     \
 *   weight w_s[j]; kf = box(p+s), ki = box(p-s) when use_box else 1;         \
 *   Wx = img - dhat img + khat.  w_half is (B, S, C, H, W).  Serial order.   \
 * d_out may be NULL. */                                                      \
EXPORT int nso_metropolis_fwd_##SUF(                                          \
    const T* wh, const T* img, const int64_t* shifts, int64_t B, int64_t S,   \
    int64_t C, int64_t H, int64_t W, int use_box, double eps, T* Wx,          \
    T* dhat, T* d_out) {                                                      \
    const int64_t HW = H * W;                                                 \
    const int64_t N = B * C * HW;                                             \
    T* d = d_out ? d_out : (T*)malloc(sizeof(T) * (size_t)N);                 \
    if (!d) return -1;                                                        \
    const T teps = (T)eps;                                                    \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c)                                       \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = wh + ((b * S + s) * C + c) * HW;        \
                        if (!use_box || (in_range(h + dx, H) && in_range(w + dy, W))) \
                            acc += ws[h * W + w];                             \
                        if (inv && (!use_box || (in_range(h - dx, H) &&       \
                                                 in_range(w - dy, W))))       \
                            acc += ws[wrapi(h - dx, H) * W + wrapi(w - dy, W)]; \
                    }                                                         \
                    d[(b * C + c) * HW + h * W + w] = acc;                    \
                }                                                             \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c) {                                     \
            const int64_t bc = (b * C + c) * HW;                              \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    const T di = d[bc + h * W + w];                           \
                    T kx = 0, dh = 0;                                         \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = wh + ((b * S + s) * C + c) * HW;        \
                        if (!use_box || (in_range(h + dx, H) && in_range(w + dy, W))) { \
                            const int64_t j = wrapi(h + dx, H) * W + wrapi(w + dy, W); \
                            const T dj = d[bc + j];                           \
                            const T den = di > dj ? di : dj;                  \
                            const T wk = ws[h * W + w] / (den > teps ? den : teps); \
                            kx += wk * img[bc + j];                           \
                            dh += wk;                                         \
                        }                                                     \
                        if (inv && (!use_box || (in_range(h - dx, H) &&       \
                                                 in_range(w - dy, W)))) {     \
                            const int64_t j = wrapi(h - dx, H) * W + wrapi(w - dy, W); \
                            const T dj = d[bc + j];                           \
                            const T den = di > dj ? di : dj;                  \
                            const T wk = ws[j] / (den > teps ? den : teps);   \
                            kx += wk * img[bc + j];                           \
                            dh += wk;                                         \
                        }                                                     \
                    }                                                         \
                    const T xi = img[bc + h * W + w];                         \
                    Wx[bc + h * W + w] = xi - dh * xi + kx;                   \
                    dhat[bc + h * W + w] = dh;                                \
                }                                                             \
        }                                                                     \
    if (!d_out) free(d);                                                      \
    return 0;                                                                 \
}                                                                             \
                                                                              \
/* accumulate_uz_scalar (GASD), accumulate_uz_scalar_reference               \
 * (ops.py:350-390): U = tree_s(w[s,b,c] x[(p+s) mod]), Z = tree_s(w[s,b,c]) \
 * broadcast over (h, w).  Backward (cuda.cu:868-980):                        \
 *   gx[q] = sum_s w[s,b,c] gU[(q-s) mod];                                    \
 *   gw[s,b,c] = sum_{h,w} (gU[p] x[(p+s) mod] + gZ[p]). */                   \
EXPORT int nso_accumulate_uz_scalar_fwd_##SUF(                                \
    const T* x, const T* wt, const int64_t* shifts, int64_t stride,           \
    int64_t S, int64_t B, int64_t C, int64_t H, int64_t W, T* U, T* Z) {      \
    const int64_t HW = H * W;                                                 \
    int fail = 0;                                                             \
    _Pragma("omp parallel")                                                   \
    {                                                                         \
        T* ub = (T*)malloc(sizeof(T) * (size_t)S);                            \
        T* zb = (T*)malloc(sizeof(T) * (size_t)S);                            \
        if (!ub || !zb) {                                                     \
            _Pragma("omp atomic write")                                       \
            fail = 1;                                                         \
        } else {                                                              \
        _Pragma("omp for collapse(2) schedule(static)")                       \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c)                                   \
                for (int64_t h = 0; h < H; ++h)                               \
                    for (int64_t w = 0; w < W; ++w) {                         \
                        for (int64_t s = 0; s < S; ++s) {                     \
                            int64_t dx, dy; int inv;                          \
                            shift_row(shifts, stride, s, &dx, &dy, &inv);     \
                            const T ws = wt[(s * B + b) * C + c];             \
                            ub[s] = ws * x[(b * C + c) * HW + wrapi(h + dx, H) * W + \
                                           wrapi(w + dy, W)];                 \
                            zb[s] = ws;                                       \
                        }                                                     \
                        const int64_t o = (b * C + c) * HW + h * W + w;       \
                        U[o] = tree_sum_##SUF(ub, S);                         \
                        Z[o] = tree_sum_##SUF(zb, S);                         \
                    }                                                         \
        }                                                                     \
        free(ub); free(zb);                                                   \
    }                                                                         \
    return fail ? -1 : 0;                                                     \
}                                                                             \
                                                                              \
EXPORT void nso_accumulate_uz_scalar_bwd_##SUF(                               \
    const T* x, const T* wt, const T* gU, const T* gZ, const int64_t* shifts, \
    int64_t stride, int64_t S, int64_t B, int64_t C, int64_t H, int64_t W,    \
    T* gx, T* gw) {                                                           \
    const int64_t HW = H * W;                                                 \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c)                                       \
            for (int64_t h = 0; h < H; ++h)                                   \
                for (int64_t w = 0; w < W; ++w) {                             \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, stride, s, &dx, &dy, &inv);         \
                        acc += wt[(s * B + b) * C + c] *                      \
                               gU[(b * C + c) * HW + wrapi(h - dx, H) * W +   \
                                  wrapi(w - dy, W)];                          \
                    }                                                         \
                    gx[(b * C + c) * HW + h * W + w] = acc;                   \
                }                                                             \
    _Pragma("omp parallel for collapse(3) schedule(static)")                  \
    for (int64_t s = 0; s < S; ++s)                                           \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c) {                                 \
                int64_t dx, dy; int inv;                                      \
                shift_row(shifts, stride, s, &dx, &dy, &inv);                 \
                const int64_t bc = (b * C + c) * HW;                          \
                T acc = 0;                                                    \
                for (int64_t h = 0; h < H; ++h)                               \
                    for (int64_t w = 0; w < W; ++w)                           \
                        acc += gU[bc + h * W + w] *                           \
                               x[bc + wrapi(h + dx, H) * W + wrapi(w + dy, W)] \
                               + gZ[bc + h * W + w];                          \
                gw[(s * B + b) * C + c] = acc;                                \
            }                                                                 \
}

/* helpers used by the normalized backward, defined before the macro use */
static inline float nso_aslog_f32(float v, int lw, float ninf) {
    if (lw) return v;
    if (v > 0) return logf(v);
    if (v == 0) return ninf;
    return NAN;
}
static inline double nso_aslog_f64(double v, int lw, double ninf) {
    if (lw) return v;
    if (v > 0) return log(v);
    if (v == 0) return ninf;
    return NAN;
}
static inline float nso_frac_f32(float v, float L, int lw, float ninf) {
    const float l = nso_aslog_f32(v, lw, ninf);
    if (l == ninf || L == ninf) return 0.0f;
    return expf(l - L);
}
static inline double nso_frac_f64(double v, double L, int lw, double ninf) {
    const double l = nso_aslog_f64(v, lw, ninf);
    if (l == ninf || L == ninf) return 0.0;
    return exp(l - L);
}

DEFINE_OPS(float, f32, logf, expf, isnan, isinf, isfinite)
DEFINE_OPS(double, f64, log, exp, isnan, isinf, isfinite)

/* ------------------------------------------------------------------------
 * Window evaluation for images too large for the full oracle.
 *
 * A window is a (Hw, Ww) block of a global (H, W) plane: window element
 * (i, j) holds global pixel ((gh0 - halo + i) mod H, (gw0 - halo + j) mod W).
 * Outputs are produced for the ch x cw crop of global pixels
 * (gh0 + i, gw0 + j), with every box test done on GLOBAL coordinates, so the
 * results equal the full-image oracle on those pixels (same term order and
 * tree) as long as every shift satisfies |dx|, |dy| <= halo.
 * ---------------------------------------------------------------------- */
#define DEFINE_WINDOW_OPS(T, SUF)                                             \
EXPORT int nso_accumulate_uz_window_fwd_##SUF(                                \
    const T* xw, const T* ww, const int64_t* shifts, int64_t S, int64_t B,    \
    int64_t C, int64_t halo, int64_t H, int64_t W, int64_t gh0, int64_t gw0,  \
    int64_t ch, int64_t cw, T* U, T* Z) {                                     \
    const int64_t Hw = ch + 2 * halo, Ww = cw + 2 * halo, HWw = Hw * Ww;      \
    int fail = 0;                                                             \
    _Pragma("omp parallel")                                                   \
    {                                                                         \
        T* ub = (T*)malloc(sizeof(T) * 2 * (size_t)S);                        \
        T* zb = (T*)malloc(sizeof(T) * 2 * (size_t)S);                        \
        if (!ub || !zb) {                                                     \
            _Pragma("omp atomic write")                                       \
            fail = 1;                                                         \
        } else {                                                              \
        _Pragma("omp for collapse(2) schedule(static)")                       \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c)                                   \
                for (int64_t i = 0; i < ch; ++i)                              \
                    for (int64_t j = 0; j < cw; ++j) {                        \
                        const T* xb = xw + (b * C + c) * HWw;                 \
                        const int64_t gh = wrapi(gh0 + i, H), gw = wrapi(gw0 + j, W);             \
                        const int64_t wi = i + halo, wj = j + halo;           \
                        int64_t n = 0;                                        \
                        for (int64_t s = 0; s < S; ++s) {                     \
                            int64_t dx, dy; int inv;                          \
                            shift_row(shifts, 3, s, &dx, &dy, &inv);          \
                            const T* ws = ww + ((s * B + b) * C + c) * HWw;   \
                            const T wf = ws[wi * Ww + wj];                    \
                            ub[n] = wf * xb[(wi + dx) * Ww + (wj + dy)];      \
                            zb[n] = wf;                                       \
                            ++n;                                              \
                            if (inv) {                                        \
                                const T cb = (in_range(gh - dx, H) &&         \
                                              in_range(gw - dy, W)) ? 1 : 0;  \
                                const int64_t o = (wi - dx) * Ww + (wj - dy); \
                                const T wv = ws[o] * cb;                      \
                                ub[n] = wv * xb[o];                           \
                                zb[n] = wv;                                   \
                                ++n;                                          \
                            }                                                 \
                        }                                                     \
                        const int64_t o = (b * C + c) * ch * cw + i * cw + j; \
                        U[o] = tree_sum_##SUF(ub, n);                         \
                        Z[o] = tree_sum_##SUF(zb, n);                         \
                    }                                                         \
        }                                                                     \
        free(ub); free(zb);                                                   \
    }                                                                         \
    return fail ? -1 : 0;                                                     \
}                                                                             \
                                                                              \
EXPORT void nso_accumulate_uz_window_bwd_##SUF(                               \
    const T* xw, const T* ww, const T* gUw, const T* gZw,                     \
    const int64_t* shifts, int64_t S, int64_t B, int64_t C, int64_t halo,     \
    int64_t H, int64_t W, int64_t gh0, int64_t gw0, int64_t ch, int64_t cw,   \
    T* gx, T* gw) {                                                           \
    const int64_t Hw = ch + 2 * halo, Ww = cw + 2 * halo, HWw = Hw * Ww;      \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c) {                                     \
            const int64_t bc = (b * C + c) * HWw;                             \
            for (int64_t i = 0; i < ch; ++i)                                  \
                for (int64_t j = 0; j < cw; ++j) {                            \
                    const int64_t gh = wrapi(gh0 + i, H), gwc = wrapi(gw0 + j, W);                \
                    const int64_t wi = i + halo, wj = j + halo;               \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = ww + ((s * B + b) * C + c) * HWw;       \
                        const int64_t o = (wi - dx) * Ww + (wj - dy);         \
                        acc += ws[o] * gUw[bc + o];                           \
                        if (inv && in_range(gh + dx, H) && in_range(gwc + dy, W)) \
                            acc += ws[wi * Ww + wj] *                         \
                                   gUw[bc + (wi + dx) * Ww + (wj + dy)];      \
                    }                                                         \
                    gx[(b * C + c) * ch * cw + i * cw + j] = acc;             \
                }                                                             \
        }                                                                     \
    _Pragma("omp parallel for collapse(3) schedule(static)")                  \
    for (int64_t s = 0; s < S; ++s)                                           \
        for (int64_t b = 0; b < B; ++b)                                       \
            for (int64_t c = 0; c < C; ++c) {                                 \
                int64_t dx, dy; int inv;                                      \
                shift_row(shifts, 3, s, &dx, &dy, &inv);                      \
                const int64_t bc = (b * C + c) * HWw;                         \
                T* g = gw + ((s * B + b) * C + c) * ch * cw;                  \
                for (int64_t i = 0; i < ch; ++i)                              \
                    for (int64_t j = 0; j < cw; ++j) {                        \
                        const int64_t gh = wrapi(gh0 + i, H), gwc = wrapi(gw0 + j, W);            \
                        const int64_t q = bc + (i + halo) * Ww + (j + halo);  \
                        const int64_t qp = q + dx * Ww + dy;                  \
                        T v = xw[qp] * gUw[q] + gZw[q];                       \
                        if (inv && in_range(gh + dx, H) && in_range(gwc + dy, W)) \
                            v += xw[q] * gUw[qp] + gZw[qp];                   \
                        g[i * cw + j] = v;                                    \
                    }                                                         \
            }                                                                 \
}                                                                             \
                                                                              \
/* Metropolis on a window with halo >= 2R (degree needed on crop + R). */    \
EXPORT int nso_metropolis_window_##SUF(                                       \
    const T* whw, const T* imgw, const int64_t* shifts, int64_t B, int64_t S, \
    int64_t C, int64_t halo, int64_t H, int64_t W, int64_t gh0, int64_t gw0,  \
    int64_t ch, int64_t cw, int use_box, double eps, T* Wx, T* dhat) {        \
    const int64_t Hw = ch + 2 * halo, Ww = cw + 2 * halo, HWw = Hw * Ww;      \
    int64_t R = 0;                                                            \
    for (int64_t s = 0; s < S; ++s) {                                         \
        int64_t dx, dy; int inv;                                              \
        shift_row(shifts, 3, s, &dx, &dy, &inv);                              \
        if (llabs(dx) > R) R = llabs(dx);                                     \
        if (llabs(dy) > R) R = llabs(dy);                                     \
    }                                                                         \
    if (2 * R > halo) return -2;                                              \
    T* d = (T*)calloc((size_t)(B * C * HWw), sizeof(T));                      \
    if (!d) return -1;                                                        \
    const T teps = (T)eps;                                                    \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c)                                       \
            for (int64_t i = halo - R; i < halo + ch + R; ++i)                \
                for (int64_t j = halo - R; j < halo + cw + R; ++j) {          \
                    const int64_t gh = wrapi(gh0 - halo + i, H), gwc = wrapi(gw0 - halo + j, W);  \
                    T acc = 0;                                                \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = whw + ((b * S + s) * C + c) * HWw;      \
                        if (!use_box || (in_range(gh + dx, H) && in_range(gwc + dy, W))) \
                            acc += ws[i * Ww + j];                            \
                        if (inv && (!use_box || (in_range(gh - dx, H) &&      \
                                                 in_range(gwc - dy, W))))     \
                            acc += ws[(i - dx) * Ww + (j - dy)];              \
                    }                                                         \
                    d[(b * C + c) * HWw + i * Ww + j] = acc;                  \
                }                                                             \
    _Pragma("omp parallel for collapse(2) schedule(static)")                  \
    for (int64_t b = 0; b < B; ++b)                                           \
        for (int64_t c = 0; c < C; ++c) {                                     \
            const int64_t bc = (b * C + c) * HWw;                             \
            for (int64_t i0 = 0; i0 < ch; ++i0)                               \
                for (int64_t j0 = 0; j0 < cw; ++j0) {                         \
                    const int64_t i = i0 + halo, j = j0 + halo;               \
                    const int64_t gh = wrapi(gh0 + i0, H), gwc = wrapi(gw0 + j0, W);              \
                    const T di = d[bc + i * Ww + j];                          \
                    T kx = 0, dh = 0;                                         \
                    for (int64_t s = 0; s < S; ++s) {                         \
                        int64_t dx, dy; int inv;                              \
                        shift_row(shifts, 3, s, &dx, &dy, &inv);              \
                        const T* ws = whw + ((b * S + s) * C + c) * HWw;      \
                        if (!use_box || (in_range(gh + dx, H) && in_range(gwc + dy, W))) { \
                            const int64_t jj = (i + dx) * Ww + (j + dy);      \
                            const T dj = d[bc + jj];                          \
                            const T den = di > dj ? di : dj;                  \
                            const T wk = ws[i * Ww + j] / (den > teps ? den : teps); \
                            kx += wk * imgw[bc + jj];                         \
                            dh += wk;                                         \
                        }                                                     \
                        if (inv && (!use_box || (in_range(gh - dx, H) &&      \
                                                 in_range(gwc - dy, W)))) {   \
                            const int64_t jj = (i - dx) * Ww + (j - dy);      \
                            const T dj = d[bc + jj];                          \
                            const T den = di > dj ? di : dj;                  \
                            const T wk = ws[jj] / (den > teps ? den : teps);  \
                            kx += wk * imgw[bc + jj];                         \
                            dh += wk;                                         \
                        }                                                     \
                    }                                                         \
                    const T xi = imgw[bc + i * Ww + j];                       \
                    Wx[(b * C + c) * ch * cw + i0 * cw + j0] = xi - dh * xi + kx; \
                    dhat[(b * C + c) * ch * cw + i0 * cw + j0] = dh;          \
                }                                                             \
        }                                                                     \
    free(d);                                                                  \
    return 0;                                                                 \
}

DEFINE_WINDOW_OPS(float, f32)
DEFINE_WINDOW_OPS(double, f64)
