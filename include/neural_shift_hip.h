/*
 * neural_shift_hip.h -- C ABI of libneural_shift_hip.so, the gfx950 (MI355X)
 * implementation of the neural_shift_cuda shift-window operators.
 *
 * This is the drop-in boundary under the Python package: each entry point
 * replaces one function of the reference's pybind11 module
 * `neural_shift_cuda._C` (csrc/shift_ops.cpp:347-368, csrc/metropolis.cpp:42-48
 * in trishitmg/neural_shift_cuda).  The ABI is plain C: raw device pointers,
 * int64 sizes, an int dtype code and a hipStream_t passed as void*.  No torch
 * types cross it, and the library never allocates or frees device memory:
 * the caller passes every input, output and workspace buffer.
 *
 * Common conventions
 *   - All tensors are contiguous, row-major.  x/guide/img are (B, C, H, W).
 *     Per-pixel weights are shift-major (S*B, C, H, W): plane s*B + b.
 *     Metropolis weights are batch-major (B, S, C, H, W).
 *   - `shifts` is a DEVICE pointer to a contiguous int64 (S, shift_cols)
 *     table of (dx, dy[, has_inverse]) rows.  The forward term of pixel
 *     (h, w) reads (h + dx, w + dy) circularly (gather convention); any int64
 *     shift value is reduced modulo H / W on the device.  has_inverse of the
 *     accumulations is the reference's flag: 0 = no mirror term, any other
 *     value = the mirror term, dropped where its source (h - dx, w - dy)
 *     falls outside the image.  Only when the call ORs NSH_SHIFT_CODES into
 *     `dtype` does the column hold this library's row codes instead (see
 *     NSH_SHIFT_CODES).
 *   - `dtype` selects the element type of the "user" tensors (x, weights,
 *     guide, gradients w.r.t. them); see NSH_DTYPE_*.  Accumulation happens
 *     in float for fp16/bf16/fp32 and in double for fp64: "acc" tensors
 *     (U, Z, D, log_C and their gradients) use that accumulator type.
 *   - Every call is asynchronous on `stream` (NULL = the null stream) and
 *     returns 0 on success or an NSH_ERR_* code; nsh_last_error() then holds
 *     a message (thread-local).  Calls hold no global state and are
 *     re-entrant.
 *   - A single (b, c) plane must satisfy H*W*sizeof(element) < 2^31 bytes;
 *     tensor totals are unrestricted (64-bit plane offsets).
 */
#ifndef NEURAL_SHIFT_HIP_H
#define NEURAL_SHIFT_HIP_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define NSH_API __attribute__((visibility("default")))
#else
#define NSH_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
#define NSH_DTYPE_FLOAT16 1
#define NSH_DTYPE_BFLOAT16 2
#define NSH_DTYPE_FLOAT32 3
#define NSH_DTYPE_FLOAT64 4

/* Flag ORed into `dtype` of the accumulate_uz and normalized_accumulate_uz
 * calls (and their workspace queries): the third column of `shifts` holds
 * row codes, an extension with no counterpart in the reference.  For a value
 * v in [0, 7], bits 0-1 select the mirror term (0 none; 1 or 3 the
 * reference's mirror, dropped where its source wraps; 2 a circular mirror:
 * the fully periodic symmetric operator without explicit rolled rows) and
 * bit 2 drops the forward term where (h + dx, w + dy) leaves the image (the
 * caller's box mask applied in the kernel).  Any other value is the
 * reference's mirror. */
#define NSH_SHIFT_CODES 0x100

/* Flag ORed into `dtype` of the accumulate_uz and normalized_accumulate_uz
 * calls (and their workspace queries): the weights are shared by every
 * channel, (S*B, 1, H, W) instead of (S*B, C, H, W) -- the reference
 * installers' single-head weights, which they broadcast to the channels
 * before the call (nekde_drunet_attn_patch.py:117-140).  The kernels read
 * the shared plane for every channel instead of a materialised copy per
 * channel.  Gradients w.r.t. the weights stay per channel: grad_w is
 * (S*B, C, H, W) (its sum over the channels is the shared weights'
 * gradient).  An extension with no counterpart in the reference. */
#define NSH_SHARED_WEIGHTS 0x200

/* Flag ORed into `dtype` of the accumulate_uz calls (and their workspace
 * queries): a hint that the table's radius max(|dx|, |dy|) lies in 9..16.
 * The scatter path then stages a 16-pixel border around its tiles (larger
 * workspace), so every weight element is still read once; without the hint
 * such tables take the gather form inside the launch (x, gU, gZ re-read per
 * shift from the caches).  A hint only: the kernels check the radius on the
 * device, so any table gives the same results with or without it (a table
 * of radius <= 8 runs on the wider border, one above 16 in the gather
 * form).  An extension with no counterpart in the reference. */
#define NSH_WIDE_HALO 0x400
/* The same hint for a radius in 17..24 (a 24-pixel border; the half-plane
 * tables up to R = 22, S = 1013, the largest the 1 <= S <= 1024 contract
 * admits).  NSH_WIDE_HALO is ignored when both are set. */
#define NSH_WIDER_HALO 0x800
#define NSH_DTYPE_FLAGS \
    (NSH_SHIFT_CODES | NSH_SHARED_WEIGHTS | NSH_WIDE_HALO | NSH_WIDER_HALO | NSH_NARROW_HALO)

/* Flag ORed into `dtype`: a hint that every shift of the table has
 * max(|dx|, |dy|) <= 6, for two passes that then stage a 6-pixel border
 * instead of 8 and fit three workgroups on a compute unit:
 *  - nsh_metropolis_aggregate_backward (fp16/bf16/fp32; its workspace query
 *    accepts and ignores the flag): the edge pass, which then keeps no rho
 *    array in LDS (it forms 1/max(d, eps) from the staged degree);
 *  - nsh_normalized_accumulate_uz_backward (fp64) on 32 x 16 tiles instead of
 *    32 x 32; its workspace query (backward != 0) with the flag returns the
 *    larger of the two plans' sizes, and a smaller workspace runs the 8-pixel
 *    border.
 * The other calls that take NSH_DTYPE_FLAGS accept and ignore it.  A hint
 * only: shifts beyond the border take the gather form inside the same
 * launch, so any table gives the same results with or without it.  An
 * extension with no counterpart in the reference. */
#define NSH_NARROW_HALO 0x1000

/* Return codes. */
#define NSH_OK 0
#define NSH_ERR_INVALID 1 /* argument check failed (the reference's TORCH_CHECK) */
#define NSH_ERR_HIP 2     /* HIP runtime reported an error at launch */
#define NSH_ERR_UNSUPPORTED 3 /* valid arguments this entry point does not serve (nothing
                               * was launched); the caller takes its general path */

/* Message for the last failing call on this thread ("" if none). */
NSH_API const char* nsh_last_error(void);

/* ABI marker; always 64.  Replaces `index_width_bits`
 * (csrc/shift_ops.cpp:351-352): 64-bit shifts and flattened offsets. */
NSH_API int nsh_index_width_bits(void);

/* Library build identifier (for diagnostics). */
NSH_API const char* nsh_version(void);

/* shift_gather forward.  Replaces `shift_gather_forward(guide, shifts)`
 * (csrc/shift_ops.cpp:81-100; kernels csrc/shift_ops_cuda.cu:61-91, 133-157).
 *   out[s*B+b, c, h, w]  = guide[b, c, (h+dx) mod H, (w+dy) mod W]
 *   mask[s*B+b, 0, h, w] = 1 if 0<=h+dx<H and 0<=w+dy<W else 0
 * out is (S*B, C, H, W) and mask (S*B, 1, H, W), both in `dtype` (the
 * reference returns the mask in the guide dtype).  Bit-exact copies.
 * shift_cols is 2 or 3 (only dx, dy are read).  mask may be NULL. */
NSH_API int nsh_shift_gather_forward(const void* guide, const int64_t* shifts, int64_t S,
                             int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                             int64_t W, int dtype, void* out, void* mask, void* stream);

/* shift_gather backward (gather-form adjoint, deterministic).  Replaces
 * `shift_gather_backward(grad_out, shifts, B, C, H, W)`
 * (csrc/shift_ops.cpp:102-115; kernel csrc/shift_ops_cuda.cu:165-203).
 *   grad_guide[b,c,h,w] = sum_s grad_out[s*B+b, c, (h-dx) mod H, (w-dy) mod W]
 * Sums in the accumulator type, rounds once to `dtype`. */
NSH_API int nsh_shift_gather_backward(const void* grad_out, const int64_t* shifts, int64_t S,
                              int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                              int64_t W, int dtype, void* grad_guide, void* stream);

/* pair_gather forward.  Replaces `pair_gather_forward(guide, shifts)`
 * (csrc/shift_ops.cpp:121-140; kernels csrc/shift_ops_cuda.cu:93-131, 133-157).
 *   out[s*B+b, 0:C]  = guide[b]
 *   out[s*B+b, C:2C] = shift_gather output
 * out is (S*B, 2C, H, W); mask as for shift_gather (may be NULL). */
NSH_API int nsh_pair_gather_forward(const void* guide, const int64_t* shifts, int64_t S,
                            int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                            int64_t W, int dtype, void* out, void* mask, void* stream);

/* pair_gather backward.  Replaces `pair_gather_backward(...)`
 * (csrc/shift_ops.cpp:142-154; kernel csrc/shift_ops_cuda.cu:205-246), but
 * gather-form and deterministic instead of atomicAdd scatter:
 *   grad_guide[b,c,q] = sum_s grad_out[s*B+b, c, q]
 *                     + sum_s grad_out[s*B+b, C+c, (q - s) mod]. */
NSH_API int nsh_pair_gather_backward(const void* grad_out, const int64_t* shifts, int64_t S,
                             int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                             int64_t W, int dtype, void* grad_guide, void* stream);

/* accumulate_uz forward.  Replaces `accumulate_uz_forward(x, weights, shifts)`
 * (csrc/shift_ops.cpp:160-192; kernel csrc/shift_ops_cuda.cu:255-341).
 *   U[p] = sum_s w_s[p] x[(p+s) mod] + sum_{s:inv, box(p-s)} w_s[p-s] x[p-s]
 *   Z[p] = sum_s w_s[p]              + sum_{s:inv, box(p-s)} w_s[p-s]
 * x (B,C,H,W) and weights (S*B,C,H,W) in `dtype`; shifts (S,3);
 * U, Z (B,C,H,W) in the accumulator type.  1 <= S <= 1024. */
NSH_API int nsh_accumulate_uz_forward(const void* x, const void* weights, const int64_t* shifts,
                              int64_t S, int64_t B, int64_t C, int64_t H, int64_t W,
                              int dtype, void* U, void* Z, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* accumulate_uz backward (one fused pass).  Replaces
 * `accumulate_uz_backward(x, weights, grad_U, grad_Z, shifts)`
 * (csrc/shift_ops.cpp:194-212; kernels csrc/shift_ops_cuda.cu:343-458).
 *   gx[q]   = sum_s w_s[(q-s) mod] gU[(q-s) mod] + sum_{inv, box(q+s)} w_s[q] gU[q+s]
 *   gw_s[q] = x[(q+s) mod] gU[q] + gZ[q] + [inv, box(q+s)] (x[q] gU[q+s] + gZ[q+s])
 * grad_U, grad_Z in the accumulator type; grad_x, grad_w in `dtype`. */
NSH_API int nsh_accumulate_uz_backward(const void* x, const void* weights, const void* grad_U,
                               const void* grad_Z, const int64_t* shifts, int64_t S,
                               int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                               void* grad_x, void* grad_w, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* accumulate_uz forward and backward on one horizontal band of a larger
 * image: the building block of a spatial split over several GPUs.  No
 * counterpart in the reference: it is for callers that shard one image by
 * rows, each GPU holding its band plus halo rows above and below (its
 * neighbours' rows, taken around the image at its top and bottom edge).
 * Same arguments and results as nsh_accumulate_uz_forward / _backward, plus
 * row_origin and image_height: local row h of the band is row
 * (row_origin + h) mod image_height of the image, and every box test (a
 * mirror term dropped where its source wraps; row code 4's forward box) is
 * taken on those image rows.  Rows farther than the table's radius from the
 * band's ends then equal the whole-image call's rows (with halos of at least
 * the radius, every row the caller keeps).  The workspace is sized by
 * nsh_accumulate_uz_workspace_bytes for the band's shape.  row_origin = 0
 * and image_height = H is the plain call.  |row_origin| <= 2^30,
 * 1 <= image_height <= 2^30. */
NSH_API int nsh_accumulate_uz_forward_band(const void* x, const void* weights,
                                           const int64_t* shifts, int64_t S, int64_t B,
                                           int64_t C, int64_t H, int64_t W, int64_t row_origin,
                                           int64_t image_height, int dtype, void* U, void* Z,
                                           void* workspace, int64_t workspace_bytes,
                                           void* stream);
NSH_API int nsh_accumulate_uz_backward_band(const void* x, const void* weights,
                                            const void* grad_U, const void* grad_Z,
                                            const int64_t* shifts, int64_t S, int64_t B,
                                            int64_t C, int64_t H, int64_t W, int64_t row_origin,
                                            int64_t image_height, int dtype, void* grad_x,
                                            void* grad_w, void* workspace,
                                            int64_t workspace_bytes, void* stream);

/* Workspace of accumulate_uz forward (backward = 0) or backward (1), in
 * bytes; 0 when the shape does not use one, -1 on invalid arguments.  No
 * counterpart in the reference (whose kernels re-read shifted weights).
 * With a workspace of at least this size (256-byte aligned, device memory,
 * contents irrelevant, not shared with a concurrent call) the calls above
 * read every weight element exactly once: the terms that need a weight at
 * a shifted pixel are scattered through an LDS window per tile, whose
 * border is spilled to the workspace and added by a fix-up kernel.  With a
 * NULL or smaller workspace the calls read shifted weights directly
 * (same results up to summation order). */
NSH_API int64_t nsh_accumulate_uz_workspace_bytes(int64_t S, int64_t B, int64_t C, int64_t H,
                                                  int64_t W, int dtype, int backward);

/* accumulate_uz forward that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as nsh_accumulate_uz_forward
 * without the workspace: the scatter path's workspace is a static device
 * array of NSH_NOALLOC_SCRATCH_BYTES that every GPU the library runs on
 * holds until the process ends (the current device's copy is used; a
 * non-null stream of another device is rejected with NSH_ERR_INVALID).  A
 * shape whose workspace (nsh_accumulate_uz_workspace_bytes) exceeds it is
 * rejected with NSH_ERR_INVALID; shapes that need none run the gather
 * kernels.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams or threads) race, so the caller must
 * serialize them. */
#define NSH_NOALLOC_SCRATCH_BYTES (32ll << 20)
NSH_API int nsh_accumulate_uz_forward_noalloc(const void* x, const void* weights,
                                              const int64_t* shifts, int64_t S, int64_t B,
                                              int64_t C, int64_t H, int64_t W, int dtype,
                                              void* U, void* Z, void* stream);

/* normalized_accumulate_uz forward (online softmax over shifts).  Replaces
 * `normalized_accumulate_uz_forward(x, weights, shifts, log_weights)`
 * (csrc/shift_ops.cpp:218-252; kernel csrc/shift_ops_cuda.cu:474-653).
 *   D = sum_i a_i v_i / sum_i a_i with a_i = w_i / max w (log_weights = 0) or
 *   exp(l_i - max l) (log_weights = 1); log_C = log of the unscaled degree.
 * Masks: w == 0 / l == -inf.  Empty row: D = 0, log_C = -inf.  A NaN, +inf
 * or (positive mode) negative weight makes both outputs NaN.
 * D, log_C in the accumulator type. */
NSH_API int nsh_normalized_accumulate_uz_forward(const void* x, const void* weights,
                                         const int64_t* shifts, int64_t S, int64_t B,
                                         int64_t C, int64_t H, int64_t W, int dtype,
                                         int log_weights, void* D, void* log_C,
                                         void* workspace, int64_t workspace_bytes, void* stream);

/* normalized_accumulate_uz backward.  Replaces
 * `normalized_accumulate_uz_backward(x, weights, D, log_C, grad_D, grad_log_C,
 * shifts, log_weights)` (csrc/shift_ops.cpp:254-280; kernels
 * csrc/shift_ops_cuda.cu:655-791).  D, log_C, grad_D, grad_log_C in the
 * accumulator type; grad_x, grad_w in `dtype`; masked weights get 0. */
NSH_API int nsh_normalized_accumulate_uz_backward(const void* x, const void* weights, const void* D,
                                          const void* log_C, const void* grad_D,
                                          const void* grad_log_C, const int64_t* shifts,
                                          int64_t S, int64_t B, int64_t C, int64_t H,
                                          int64_t W, int dtype, int log_weights,
                                          void* grad_x, void* grad_w, void* workspace,
                                          int64_t workspace_bytes, void* stream);

/* Workspace of normalized_accumulate_uz forward (backward = 0) or backward
 * (1), in bytes; 0 when the shape does not use one, -1 on invalid arguments.
 * No counterpart in the reference (whose kernels re-read shifted weights).
 * With a workspace of at least this size (256-byte aligned device memory,
 * contents irrelevant, not shared with a concurrent call) both calls read
 * every weight element once: the forward merges each mirror term into an
 * LDS window of online-softmax states, the backward scatters the x-gradient
 * term through an LDS window; the windows' borders go to the workspace and
 * a fix-up kernel merges them.  With a NULL or smaller workspace the gather
 * kernels run (same results up to summation order). */
NSH_API int64_t nsh_normalized_workspace_bytes(int64_t S, int64_t B, int64_t C, int64_t H,
                                               int64_t W, int dtype, int backward);

/* normalized_accumulate_uz forward of head-mixed positive weights, no
 * grad.  Replaces the attention installers' head-mixing product followed by
 * the forward (nekde_drunet_attn_patch.py:117-140 `_mix_heads_vec`, then
 * :368-370; shift_ops.cpp:218-252): the weight of channel c at shift s is
 *   w[s*B+b, c] = sum_j mix[c, j] * head_weights[s*B+b, j]
 * formed in the kernel's weight load, so the (S*B, C, H, W) stack is never
 * written (each channel reads the `heads` planes of its shift: C*heads
 * plane reads per shift and pixel against heads + 2C when mixing first).
 * head_weights is (S*B, heads, H, W) in `dtype`; mix is (C, heads) in the
 * accumulator type (fp32, fp64 for fp64); D, log_C as in
 * nsh_normalized_accumulate_uz_forward with log_weights = 0.  dtype may
 * carry NSH_SHIFT_CODES (the forward box, circular mirrors), not
 * NSH_SHARED_WEIGHTS.  The workspace is the forward's
 * (nsh_normalized_workspace_bytes).  Served: 2 <= heads <= 4 on shapes the
 * workspace plan covers; otherwise NSH_ERR_UNSUPPORTED (nothing launched;
 * mix the heads and call nsh_normalized_accumulate_uz_forward). */
NSH_API int nsh_normalized_accumulate_uz_forward_mixed(
    const void* x, const void* head_weights, const void* mix, const int64_t* shifts, int64_t S,
    int64_t B, int64_t C, int64_t H, int64_t W, int64_t heads, int dtype, void* D, void* log_C,
    void* workspace, int64_t workspace_bytes, void* stream);

/* Head mixing and its backward (training path of the same product).
 * Replaces the installers' mixing einsum and its autograd
 * (nekde_drunet_attn_patch.py:117-140 `_mix_heads_vec`, matrix case):
 *   out[n, c, p]  = sum_j mix[c, j] w[n, j, p]
 *   grad_w[n,j,p] = sum_c mix[c, j] grad_out[n, c, p]
 *   grad_mix[c,j] = sum_{n, p} grad_out[n, c, p] w[n, j, p]
 * w, grad_w: (N, heads, P); out, grad_out: (N, C, P), all in `dtype`; mix,
 * grad_mix: (C, heads) in the accumulator type.  Sums in the accumulator
 * type, rounded once; grad_mix is a deterministic two-level reduction
 * through the workspace (nsh_head_mix_workspace_bytes; -1 on invalid
 * arguments).  Served: 2 <= heads <= 4 and C <= 8 (NSH_ERR_UNSUPPORTED
 * otherwise, nothing launched); P * 8 < 2^31. */
NSH_API int nsh_head_mix_forward(const void* w, const void* mix, int64_t N, int64_t heads,
                                 int64_t C, int64_t P, int dtype, void* out, void* stream);
NSH_API int64_t nsh_head_mix_workspace_bytes(int64_t N, int64_t heads, int64_t C, int64_t P,
                                             int dtype);
NSH_API int nsh_head_mix_backward(const void* w, const void* mix, const void* grad_out,
                                  int64_t N, int64_t heads, int64_t C, int64_t P, int dtype,
                                  void* grad_w, void* grad_mix, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/* accumulate_uz_scalar forward (GASD scalar-per-transform weights).
 * Replaces `accumulate_uz_scalar_forward(x, weights, shifts)`
 * (csrc/shift_ops.cpp:289-316; kernel csrc/shift_ops_cuda.cu:806-866).
 *   U[b,c,p] = sum_s w[s,b,c] x[b,c,(p+s) mod],  Z[b,c,p] = sum_s w[s,b,c]
 * weights (S, B, C) in `dtype`; U, Z in the accumulator type. */
NSH_API int nsh_accumulate_uz_scalar_forward(const void* x, const void* weights,
                                     const int64_t* shifts, int64_t S, int64_t shift_cols,
                                     int64_t B, int64_t C, int64_t H, int64_t W, int dtype,
                                     void* U, void* Z, void* stream);

/* accumulate_uz_scalar backward.  Replaces `accumulate_uz_scalar_backward`
 * (csrc/shift_ops.cpp:318-337; kernels csrc/shift_ops_cuda.cu:868-980).
 *   gx[q] = sum_s w[s,b,c] gU[(q-s) mod]
 *   gw[s,b,c] = sum_{h,w} gU[p] x[(p+s) mod] + gZ[p]   (fixed-order tree)
 * grad_w_partial is a caller workspace of S*B*C*nsplit accumulator
 * elements, nsplit = nsh_scalar_backward_splits(H, W). */
NSH_API int nsh_scalar_backward_splits(int64_t H, int64_t W);
NSH_API int nsh_accumulate_uz_scalar_backward(const void* x, const void* weights, const void* grad_U,
                                      const void* grad_Z, const int64_t* shifts, int64_t S,
                                      int64_t shift_cols, int64_t B, int64_t C, int64_t H,
                                      int64_t W, int dtype, void* grad_x, void* grad_w,
                                      void* grad_w_partial, void* stream);

/* Metropolis aggregate (inference).  Replaces
 * `metropolis_aggregate(w_half, img, shifts, use_box, eps=1e-6)`
 * (csrc/metropolis.cpp:29-48; csrc/metropolis_cuda.cu:195-240).
 *   d    = K e      (pass 1, written to `degree`, accumulator type, (B,C,H,W))
 *   wk   = w / max(d_p, d_j, eps) per edge (forward j = p+s, inverse j = p-s
 *          with the circularly shifted forward weight w_s[j])
 *   Wx   = img - d_hat img + K_hat img,  d_hat = K_hat e   (pass 2, fused)
 * w_half (B,S,C,H,W), img (B,C,H,W), Wx and d_hat (B,C,H,W) in `dtype`;
 * shifts (S,3).  use_box != 0 drops wrap-around neighbours.
 * workspace: optional (NULL allowed), see nsh_metropolis_workspace_bytes. */
NSH_API int nsh_metropolis_aggregate(const void* w_half, const void* img, const int64_t* shifts,
                             int64_t B, int64_t S, int64_t C, int64_t H, int64_t W, int dtype,
                             int use_box, double eps, void* Wx, void* d_hat, void* degree,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace of nsh_metropolis_aggregate in bytes; 0 when the shape does not
 * use one, -1 on invalid arguments.  No counterpart in the reference (whose
 * kernels re-read the inverse edge's weight at the shifted pixel).  With a
 * workspace of at least this size (256-byte aligned device memory, contents
 * irrelevant, not shared with a concurrent call) each pass reads every
 * w_half element once: an edge's weight is formed once and added at both
 * ends, the far end through an LDS window whose border is spilled to the
 * workspace and added by a fix-up kernel.  Without it the gather kernels
 * run (same results up to summation order; K_hat exactly symmetric either
 * way). */
NSH_API int64_t nsh_metropolis_workspace_bytes(int64_t B, int64_t S, int64_t C, int64_t H,
                                               int64_t W, int dtype);

/* Metropolis aggregate backward (training).  No counterpart in the
 * reference's native module: the reference trains through its explicit-edge
 * path `metropolis_aggregate_fused` (metropolis.py:117-192, under gradient
 * checkpointing, metropolis.py:229-236), i.e. autograd through 2S-1 edge
 * planes, two accumulate_uz calls and a shift_gather.  This computes the
 * same gradients (torch.maximum's tie split and clamp_min's gate included)
 * in two passes over w_half, from the forward's `degree` buffer and d_hat:
 *   grad_w_half (B,S,C,H,W) and grad_img (B,C,H,W) in `dtype`, from
 *   grad_Wx and grad_d_hat (B,C,H,W) in `dtype`.
 * Requires the shape to have at least 3 tiles of 64 x 32 pixels (32 x 32 for
 * fp64) per direction with edge tiles >= 8 pixels, and a workspace of
 * nsh_metropolis_backward_workspace_bytes (0 = shape not supported). */
NSH_API int nsh_metropolis_aggregate_backward(const void* w_half, const void* img,
                                              const int64_t* shifts, int64_t B, int64_t S,
                                              int64_t C, int64_t H, int64_t W, int dtype,
                                              int use_box, double eps, const void* degree,
                                              const void* d_hat, const void* grad_Wx,
                                              const void* grad_d_hat, void* grad_w_half,
                                              void* grad_img, void* workspace,
                                              int64_t workspace_bytes, void* stream);
NSH_API int64_t nsh_metropolis_backward_workspace_bytes(int64_t B, int64_t S, int64_t C,
                                                        int64_t H, int64_t W, int dtype);

/* Streaming bandwidth probe: the measured HBM ceilings the kernels above are
 * compared against.  Measurement only; no counterpart in the reference.
 * kind NSH_PROBE_READ / _READ_NT: read `bytes` of src (plain or nontemporal
 * 16-byte loads; dst is a sink of at least 4 KiB that is written only on an
 * impossible bit pattern); NSH_PROBE_COPY: src -> dst; NSH_PROBE_FILL: dst.
 * bytes a positive multiple of 16, buffers 16-byte aligned, `workgroups`
 * walk the buffer grid-stride.  Variant bits ORed into the kind:
 * NSH_PROBE_UNROLL(u) loads in flight per lane (u = 4, 8 or 16; default 8),
 * NSH_PROBE_PLAIN_LOADS (copy) / NSH_PROBE_PLAIN_STORES (copy, fill):
 * temporal instead of the default streaming accesses, NSH_PROBE_1024_LANES
 * (workgroups of 1024 lanes instead of 256), NSH_PROBE_RING (copy: a
 * prefetch ring of u loads per lane, one store per step, instead of bursts
 * of u loads then u stores). */
#define NSH_PROBE_READ 0
#define NSH_PROBE_READ_NT 1
#define NSH_PROBE_COPY 2
#define NSH_PROBE_FILL 3
#define NSH_PROBE_KIND_MASK 0xff
#define NSH_PROBE_UNROLL_MASK 0xf00
#define NSH_PROBE_UNROLL(u) (((u) == 4 ? 2 : (u) == 16 ? 4 : 3) << 8)
#define NSH_PROBE_PLAIN_LOADS 0x1000
#define NSH_PROBE_PLAIN_STORES 0x2000
#define NSH_PROBE_1024_LANES 0x4000
#define NSH_PROBE_RING 0x8000
NSH_API int nsh_stream_probe(int kind, const void* src, void* dst, int64_t bytes, int workgroups,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NEURAL_SHIFT_HIP_H */
