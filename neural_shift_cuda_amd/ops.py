"""Public shift-window operators.

    shift_gather(guide, shifts)                       -> (gs_batch, mask)
    pair_gather(guide, shifts)                        -> (pair_batch, mask)
    accumulate_uz(x, weights, shifts)                 -> (U_num, Z)
    normalized_accumulate_uz(x, weights, shifts, *,
        log_weights=False, return_log_degree=False,
        validate=True)                                -> D or (D, log_C)
    accumulate_uz_scalar(x, weights, shifts)          -> (U_num, Z)

Same names, signatures, keyword arguments, return conventions and exception
types as the reference module neural_shift_cuda/ops.py (trishitmg/
neural_shift_cuda, ops.py:576-719).  Dispatch follows the reference too:
tensors on a GPU go through the autograd Functions below into the HIP
library (``_C``); CPU tensors use the pure-PyTorch ``*_reference``
implementations, which are also exported.  A GPU tensor never falls back to
the CPU code: if the library failed to load, the op raises ``RuntimeError``
carrying the original load error.

Conventions (ops.py:580-586 of the reference):
  * gather convention: gs[s*B+b, c, h, w] = guide[b, c, (h+dx) mod H, (w+dy) mod W];
  * weights are shift-major (S*B, C, H, W): plane s*B + b;
  * a shift row is (dx, dy, has_inverse); has_inverse rows add the mirror
    term w_s[p-s] x[p-s], taken only where p-s lies inside the image.

GPU numerics: fp16/bf16/fp32 inputs accumulate in fp32 and fp64 in fp64;
the promotion happens inside the kernels at load time, so a half-precision
weight tensor is read from HBM once, in half precision, and its gradient is
written once in half precision.  U/Z/D/log_C are returned in the
accumulator dtype, as in the reference.
"""
from __future__ import annotations

from typing import List, Tuple

import torch

try:
    from . import _C
    _HAS_CUDA_EXT = True
    _EXT_IMPORT_ERROR = None
except Exception as _exc:  # library not built, or HIP runtime unavailable
    _C = None
    _HAS_CUDA_EXT = False
    _EXT_IMPORT_ERROR = _exc

_NEG_INF = float("-inf")


# ---------------------------------------------------------------------------
# Shared argument handling
# ---------------------------------------------------------------------------

def _wrap_shifts(shifts: torch.Tensor) -> torch.Tensor:
    """(S, 2|3) integer table as int64 (reference ops.py:44-48)."""
    if shifts.dim() != 2 or shifts.size(1) not in (2, 3):
        raise ValueError(f"shifts must be (S, 2) or (S, 3); got {tuple(shifts.shape)}")
    return shifts.to(torch.int64)


def _accumulator_dtype(*tensors: torch.Tensor) -> torch.dtype:
    """fp16/bf16/fp32 accumulate in fp32; any fp64 input makes it fp64
    (reference ops.py:51-64).  Non-floating inputs raise TypeError."""
    for t in tensors:
        if not t.is_floating_point():
            raise TypeError(f"accumulation inputs must be floating point; got {t.dtype}")
    return torch.float64 if any(t.dtype == torch.float64 for t in tensors) else torch.float32


def _promote_accumulation_inputs(x: torch.Tensor, weights: torch.Tensor
                                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Both operands in the accumulator dtype (reference ops.py:67-74)."""
    if x.device != weights.device:
        raise ValueError(
            f"x and weights must share a device; got {x.device} and {weights.device}")
    acc = _accumulator_dtype(x, weights)
    return x.to(dtype=acc), weights.to(dtype=acc)


def _device_operands(x: torch.Tensor, weights: torch.Tensor
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Operands for the HIP kernels.  Same checks as the promotion above, but
    a same-dtype pair is passed through untouched: the kernels promote at
    load time, so no converted copy of the (S*B, C, H, W) weights is made."""
    if x.device != weights.device:
        raise ValueError(
            f"x and weights must share a device; got {x.device} and {weights.device}")
    acc = _accumulator_dtype(x, weights)
    if x.dtype == weights.dtype:
        return x, weights
    return x.to(acc), weights.to(acc)


def _prep_shifts_for_cuda(shifts: torch.Tensor, device: torch.device) -> torch.Tensor:
    """(S, 2|3) int64 contiguous table on `device`; values are never narrowed
    (reference ops.py:397-404)."""
    if shifts.dim() != 2 or shifts.size(1) not in (2, 3):
        raise ValueError(f"shifts must be (S, 2) or (S, 3); got {tuple(shifts.shape)}")
    out = shifts.to(device=device, dtype=torch.int64).contiguous()
    if out is not shifts and not shifts.is_cuda and _HAS_CUDA_EXT:
        # the kernels' launch shape depends on the table's radius: record it
        # from the host copy, so that the device copy is never read back
        _C.remember_table_radius(out, _C.table_radius(shifts))
    return out


def _mirror_table(shifts: torch.Tensor, periodic_inverse: bool,
                  box_forward: bool = False) -> Tuple[torch.Tensor, bool]:
    """(table, row_codes).  Without an extension the caller's table is
    returned unchanged with row_codes False: its third column is the
    reference's has_inverse flag (nonzero = a mirror dropped where its
    source wraps), whatever the value.  When an extension is asked for, the
    third column is rewritten to the row codes the kernels then read (the
    NSH_SHIFT_CODES contract of include/neural_shift_hip.h): 0 no mirror,
    1 the reference's mirror, 2 a circular mirror (`periodic_inverse`), plus
    4 when the forward term is to be dropped where p + s leaves the image
    (`box_forward`: the caller's box mask, applied inside the kernels)."""
    if not (periodic_inverse or box_forward):
        return shifts, False
    t = _wrap_shifts(shifts)
    if t.size(1) != 3:
        raise ValueError("periodic_inverse / box_forward require shifts with shape (S, 3)")
    t = t.clone()
    col = t[:, 2]
    code = torch.where(col != 0, torch.full_like(col, 2 if periodic_inverse else 1),
                       torch.zeros_like(col))
    if box_forward:
        code = code | 4
    t[:, 2] = code
    if _HAS_CUDA_EXT:
        # same (dx, dy) columns: the radius carries over (read once per
        # caller table, not once per rewritten copy)
        r = _C.table_radius(shifts)
        if r is not None:
            _C.remember_table_radius(t, r)
    return t, True


def _row_code(v: int, codes: bool) -> Tuple[int, bool, bool]:
    """(mirror, circular, forward box) of a table's third-column value:
    the reference's flag, or a row code of ``_mirror_table`` when `codes`."""
    if not codes:
        return (1 if v else 0), False, False
    if 0 <= v <= 7:
        mir, fbox = v & 3, bool(v & 4)
    else:
        mir, fbox = 1, False
    return mir, (mir == 2 and not fbox), fbox


def _rows(shifts: torch.Tensor) -> List[List[int]]:
    return _wrap_shifts(shifts).cpu().tolist()


# ---------------------------------------------------------------------------
# CPU reference implementations (pure PyTorch, differentiable)
# ---------------------------------------------------------------------------

def _gather2d(t: torch.Tensor, dx: int, dy: int) -> torch.Tensor:
    """out[..., h, w] = t[..., (h+dx) mod H, (w+dy) mod W]."""
    if dx == 0 and dy == 0:
        return t
    return torch.roll(t, shifts=(-dx, -dy), dims=(-2, -1))


def _box(H: int, W: int, dx: int, dy: int, dtype, device) -> torch.Tensor:
    """(1, 1, H, W) indicator of 0 <= h+dx < H and 0 <= w+dy < W."""
    hs = torch.arange(H, device=device) + dx
    ws = torch.arange(W, device=device) + dy
    rows = (hs >= 0) & (hs < H)
    cols = (ws >= 0) & (ws < W)
    return (rows[:, None] & cols[None, :]).to(dtype).reshape(1, 1, H, W)


def _tree_sum(values: torch.Tensor) -> torch.Tensor:
    """Pairwise sum over dim 0: adjacent pairs per level, an odd last entry
    carried up unchanged.  This is the summation order of the reference CPU
    fallback (ops.py:77-92), kept so fp32 results match it bit for bit."""
    if values.dim() == 0 or values.size(0) == 0:
        raise ValueError("tree reduction requires a non-empty leading dimension")
    level = values
    while level.size(0) > 1:
        n = level.size(0)
        pairs = level[0:n - 1:2] + level[1:n:2]
        level = torch.cat((pairs, level[n - 1:n]), 0) if n % 2 else pairs
    return level[0]


def shift_gather_reference(guide: torch.Tensor, shifts: torch.Tensor
                           ) -> Tuple[torch.Tensor, torch.Tensor]:
    """CPU reference for ``shift_gather`` (reference ops.py:95-135).

    Returns gs (S*B, C, H, W), the circularly shifted guide, and mask
    (S*B, 1, H, W) in the guide dtype, 1 where (h+dx, w+dy) is in bounds.
    """
    rows = _rows(shifts)
    B, C, H, W = guide.shape
    if not rows:
        return guide.new_empty((0, C, H, W)), guide.new_empty((0, 1, H, W))
    gs = torch.cat([_gather2d(guide, r[0], r[1]) for r in rows], 0).contiguous()
    mask = torch.cat([_box(H, W, r[0], r[1], guide.dtype, guide.device).expand(B, 1, H, W)
                      for r in rows], 0).contiguous()
    return gs, mask


def pair_gather_reference(guide: torch.Tensor, shifts: torch.Tensor
                          ) -> Tuple[torch.Tensor, torch.Tensor]:
    """CPU reference for ``pair_gather`` (reference ops.py:138-154):
    pair[s*B+b] = cat(guide[b], gs[s*B+b]) along channels."""
    gs, mask = shift_gather_reference(guide, shifts)
    S = gs.size(0) // max(guide.size(0), 1)
    centre = guide.unsqueeze(0).expand(S, *guide.shape).reshape(gs.shape)
    return torch.cat((centre, gs), 1).contiguous(), mask


def _symmetric_terms(x: torch.Tensor, weights: torch.Tensor, rows, S: int, codes: bool):
    """Yield (weight term, value term, mask or None) in the reference order
    [fwd_0, inv_0?, fwd_1, inv_1?, ...] (reference ops.py:182-203); with
    `codes`, the row codes of ``_mirror_table`` select circular mirrors (no
    mask) and masked forward terms."""
    B, C, H, W = x.shape
    wv = weights.reshape(S, B, C, H, W)
    for s, (dx, dy, v) in enumerate(rows):
        mir, circ, fbox = _row_code(v, codes)
        yield wv[s], _gather2d(x, dx, dy), (_box(H, W, dx, dy, x.dtype, x.device) if fbox
                                            else None)
        if mir:
            box = None if circ else _box(H, W, -dx, -dy, x.dtype, x.device)
            yield _gather2d(wv[s], -dx, -dy), _gather2d(x, -dx, -dy), box


def _check_weights(weights: torch.Tensor, S: int, B: int, C: int, H: int, W: int) -> None:
    if tuple(weights.shape) != (S * B, C, H, W):
        raise ValueError(f"weights must be {(S * B, C, H, W)}; got {tuple(weights.shape)}")


def accumulate_uz_reference(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor, *,
                            periodic_inverse: bool = False,
                            box_forward: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """CPU reference for ``accumulate_uz`` (reference ops.py:157-206).

    U = sum_s w_s x[(p+s) mod] + sum_{inv} (w_s[(p-s) mod] box(p-s)) x[(p-s) mod],
    Z the same without x, each summed by the pairwise tree.  Circular
    mirrors (periodic_inverse) drop box(p-s); box_forward multiplies each
    forward weight by box(p+s).
    """
    x, weights = _promote_accumulation_inputs(x, weights)
    sh, codes = _mirror_table(shifts, periodic_inverse, box_forward)
    sh = _wrap_shifts(sh)
    if sh.size(1) != 3:
        raise ValueError("accumulate_uz requires shifts with shape (S, 3)")
    B, C, H, W = x.shape
    S = sh.size(0)
    if S == 0:
        raise ValueError("at least one shift is required")
    _check_weights(weights, S, B, C, H, W)
    u_terms, z_terms = [], []
    for w_t, v_t, box in _symmetric_terms(x, weights, sh.tolist(), S, codes):
        if box is not None:
            w_t = w_t * box
        u_terms.append(w_t * v_t)
        z_terms.append(w_t)
    return _tree_sum(torch.stack(u_terms)), _tree_sum(torch.stack(z_terms))


def _validate_stable_weights(weights: torch.Tensor, log_weights: bool, *,
                             asynchronous: bool) -> None:
    """Weight contract of the normalized op (reference ops.py:209-224):
    log weights finite or -inf; positive weights finite and >= 0."""
    if log_weights:
        ok = torch.isfinite(weights) | (torch.isinf(weights) & (weights < 0))
        message = "log_weights may be finite or -inf (mask), but not NaN or +inf"
    else:
        ok = torch.isfinite(weights) & (weights >= 0)
        message = "positive weights must be finite and nonnegative"
    allok = ok.all()
    if asynchronous and weights.is_cuda and hasattr(torch, "_assert_async"):
        torch._assert_async(allok, message)
    elif not bool(allok):
        raise ValueError(message)


def _as_log_weights(w: torch.Tensor, log_weights: bool) -> torch.Tensor:
    """Keys of the normalized reduction.  Positive weights map to log w and
    their masks (w <= 0) to -inf.  The log is taken of a masked-safe copy so
    a masked weight receives a zero gradient (the reference GPU kernel's
    rule, shift_ops_cuda.cu:748-751) rather than NaN."""
    if log_weights:
        return w
    pos = w > 0
    safe = torch.where(pos, w, torch.ones_like(w))
    return torch.where(pos, safe.log(), torch.full_like(w, _NEG_INF))


def normalized_accumulate_uz_reference(x: torch.Tensor, weights: torch.Tensor,
                                       shifts: torch.Tensor, *, log_weights: bool = False,
                                       return_log_degree: bool = False, validate: bool = True,
                                       periodic_inverse: bool = False, box_forward: bool = False):
    """Overflow-safe CPU reference for the normalized denoiser
    (reference ops.py:234-320): D = sum a v / sum a with a = exp(key - max key);
    empty rows give D = 0 and log_C = -inf.  Circular mirrors as in
    ``accumulate_uz_reference``."""
    x, weights = _promote_accumulation_inputs(x, weights)
    sh, codes = _mirror_table(shifts, periodic_inverse, box_forward)
    sh = _wrap_shifts(sh)
    if sh.size(1) != 3:
        raise ValueError("normalized_accumulate_uz requires shifts with shape (S, 3)")
    if validate:
        _validate_stable_weights(weights, log_weights, asynchronous=False)
    B, C, H, W = x.shape
    S = sh.size(0)
    if S == 0:
        raise ValueError("at least one shift is required")
    _check_weights(weights, S, B, C, H, W)
    keys, vals = [], []
    for w_t, v_t, box in _symmetric_terms(x, weights, sh.tolist(), S, codes):
        if box is not None:
            if log_weights:
                w_t = torch.where(box > 0, w_t, torch.full_like(w_t, _NEG_INF))
            else:
                w_t = w_t * box
        keys.append(_as_log_weights(w_t, log_weights))
        vals.append(v_t)
    key = torch.stack(keys)
    val = torch.stack(vals)
    m = torch.amax(key, dim=0)
    empty = torch.isinf(m) & (m < 0)
    centred = torch.where(empty.unsqueeze(0), torch.full_like(key, _NEG_INF), key - m.unsqueeze(0))
    a = centred.exp()
    num = _tree_sum(a * val)
    den = _tree_sum(a)
    # Empty rows divide by a safe 1 so their gradients are 0, not 0/0 = NaN
    # (the reference GPU kernels' rule, shift_ops_cuda.cu:517-525).
    den = torch.where(empty, torch.ones_like(den), den)
    D = torch.where(empty, torch.zeros_like(num), num / den)
    log_C = torch.where(empty, torch.full_like(m, _NEG_INF), m + den.log())
    return (D, log_C) if return_log_degree else D


def _broadcast_scalar_weights(weights: torch.Tensor, S: int, B: int, C: int) -> torch.Tensor:
    """(S, B, C) as is, or (S, B) expanded over channels (reference ops.py:323-347)."""
    if weights.dim() == 3:
        if tuple(weights.shape) != (S, B, C):
            raise ValueError(f"weights must be (S, B, C)={(S, B, C)} or (S, B)={(S, B)}; "
                             f"got {tuple(weights.shape)}")
        return weights
    if tuple(weights.shape) != (S, B):
        raise ValueError(f"weights must be (S, B, C)={(S, B, C)} or (S, B)={(S, B)}; "
                         f"got {tuple(weights.shape)}")
    return weights.unsqueeze(-1).expand(S, B, C)


def accumulate_uz_scalar_reference(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor
                                   ) -> Tuple[torch.Tensor, torch.Tensor]:
    """CPU reference for ``accumulate_uz_scalar`` (reference ops.py:350-390):
    U = sum_s w[s,b,c] x[(p+s) mod], Z = sum_s w[s,b,c] broadcast over (H, W);
    no mask and no mirror term."""
    x, weights = _promote_accumulation_inputs(x, weights)
    if shifts.dim() != 2 or shifts.size(1) < 2:
        raise ValueError(f"shifts must be (S, >=2); got {tuple(shifts.shape)}")
    B, C, H, W = x.shape
    rows = shifts[:, :2].to(torch.int64).cpu().tolist()
    S = len(rows)
    weights = _broadcast_scalar_weights(weights, S, B, C)
    u_terms, z_terms = [], []
    for s, (dx, dy) in enumerate(rows):
        ws = weights[s].reshape(B, C, 1, 1)
        u_terms.append(ws * _gather2d(x, dx, dy))
        z_terms.append(ws)
    U = _tree_sum(torch.stack(u_terms))
    Z = _tree_sum(torch.stack(z_terms))
    return U, Z.expand(B, C, H, W)


# ---------------------------------------------------------------------------
# autograd Functions over the HIP library
# ---------------------------------------------------------------------------

class _ShiftGatherFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, guide, shifts):
        shifts_i = _prep_shifts_for_cuda(shifts, guide.device)
        out, mask = _C.shift_gather_forward(guide.contiguous(), shifts_i)
        ctx.save_for_backward(shifts_i)
        ctx.guide_shape = tuple(guide.shape)
        return out, mask

    @staticmethod
    def backward(ctx, grad_out, grad_mask):
        (shifts_i,) = ctx.saved_tensors
        if grad_out is None:
            return None, None
        B, C, H, W = ctx.guide_shape
        return _C.shift_gather_backward(grad_out.contiguous(), shifts_i, B, C, H, W), None


class _PairGatherFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, guide, shifts):
        shifts_i = _prep_shifts_for_cuda(shifts, guide.device)
        out, mask = _C.pair_gather_forward(guide.contiguous(), shifts_i)
        ctx.save_for_backward(shifts_i)
        ctx.guide_shape = tuple(guide.shape)
        return out, mask

    @staticmethod
    def backward(ctx, grad_out, grad_mask):
        (shifts_i,) = ctx.saved_tensors
        if grad_out is None:
            return None, None
        B, C, H, W = ctx.guide_shape
        return _C.pair_gather_backward(grad_out.contiguous(), shifts_i, B, C, H, W), None


def _shared_grad(grad_w: torch.Tensor, shared: bool) -> torch.Tensor:
    """The kernels return the weight gradient per channel; shared weights
    (S*B, 1, H, W) receive its sum over the channels (in the accumulator
    type, rounded once)."""
    if not shared:
        return grad_w
    acc = torch.float64 if grad_w.dtype == torch.float64 else torch.float32
    return grad_w.sum(dim=1, keepdim=True, dtype=acc).to(grad_w.dtype)


def _shared_operand(weights: torch.Tensor, C: int, shared: bool) -> torch.Tensor:
    """Shared weights as the (S*B, C, H, W) view the CPU paths take."""
    if not shared:
        return weights
    if weights.dim() != 4 or weights.size(1) != 1:
        raise ValueError(f"shared weights must be (S*B, 1, H, W); got {tuple(weights.shape)}")
    return weights.expand(weights.size(0), C, weights.size(2), weights.size(3))


class _AccumulateUZFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weights, shifts, row_codes=False, shared=False):
        if shifts.dim() != 2 or shifts.size(1) != 3:
            raise ValueError("accumulate_uz requires shifts of shape (S, 3)")
        shifts_i = _prep_shifts_for_cuda(shifts, x.device)
        x_c, w_c = x.contiguous(), weights.contiguous()
        U, Z = _C.accumulate_uz_forward(x_c, w_c, shifts_i, row_codes=row_codes,
                                        shared_weights=shared)
        ctx.save_for_backward(x_c, w_c, shifts_i)
        ctx.row_codes = row_codes
        ctx.shared = shared
        return U, Z

    @staticmethod
    def backward(ctx, grad_U, grad_Z):
        x, weights, shifts_i = ctx.saved_tensors
        if grad_U is None:
            grad_U = torch.zeros(x.shape, dtype=_C._acc_dtype(x.dtype), device=x.device)
        if grad_Z is None:
            grad_Z = torch.zeros(x.shape, dtype=_C._acc_dtype(x.dtype), device=x.device)
        grad_x, grad_w = _C.accumulate_uz_backward(
            x, weights, grad_U.contiguous(), grad_Z.contiguous(), shifts_i,
            row_codes=ctx.row_codes, shared_weights=ctx.shared)
        return grad_x, _shared_grad(grad_w, ctx.shared), None, None, None


class _HeadMixFn(torch.autograd.Function):
    """sum_j mix[c, j] * w[:, j] through the HIP kernels (head_mix_forward /
    head_mix_backward): the gradients of w and of the matrix in one pass."""

    @staticmethod
    def forward(ctx, w, mix):
        out = _C.head_mix_forward(w, mix)
        ctx.save_for_backward(w, mix)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        w, mix = ctx.saved_tensors
        gw, gm = _C.head_mix_backward(w, mix, grad_out)
        return (gw if ctx.needs_input_grad[0] else None,
                gm.to(mix.dtype) if ctx.needs_input_grad[1] else None)


def mix_head_planes(w: torch.Tensor, mix: torch.Tensor) -> torch.Tensor:
    """(N, C, P) = sum_j mix[c, j] * w[:, j] for per-head planes w (N, h, P)
    and a (C, h) mixing matrix: the attention installers' head-mixing
    product (reference nekde_drunet_attn_patch.py:117-140, an einsum).  On
    the GPU with 2 <= h <= 4 and C <= 8 it runs the HIP kernels (one pass
    each way, the matrix gradient a deterministic reduction); otherwise a
    broadcast product summed over the heads (c3 training shape, C = 3,
    h = 2, N = 976 planes of 256^2 on MI355X: kernels 0.34 ms forward, the
    broadcast form 0.92 ms forward and 2.6 ms forward+backward, the einsum
    3.2 / 16 ms, a batched matmul 3.0 / 50 ms)."""
    N, h, P = w.shape
    C = mix.shape[0]
    if (w.is_cuda and 2 <= h <= 4 and C <= 8 and _HAS_CUDA_EXT
            and hasattr(_C, "head_mix_forward")):
        return _HeadMixFn.apply(w.contiguous(), mix)
    return (mix.to(w.dtype).view(1, C, h, 1) * w.reshape(N, 1, h, P)).sum(2)


class _NormalizedAccumulateUZFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weights, shifts, log_weights, row_codes=False, shared=False):
        if shifts.dim() != 2 or shifts.size(1) != 3:
            raise ValueError("normalized_accumulate_uz requires shifts of shape (S, 3)")
        shifts_i = _prep_shifts_for_cuda(shifts, x.device)
        x_c, w_c = x.contiguous(), weights.contiguous()
        D, log_C = _C.normalized_accumulate_uz_forward(x_c, w_c, shifts_i, bool(log_weights),
                                                       row_codes=row_codes,
                                                       shared_weights=shared)
        ctx.save_for_backward(x_c, w_c, D, log_C, shifts_i)
        ctx.log_weights = bool(log_weights)
        ctx.row_codes = row_codes
        ctx.shared = shared
        ctx.set_materialize_grads(False)
        return D, log_C

    @staticmethod
    def backward(ctx, grad_D, grad_log_C):
        x, weights, D, log_C, shifts_i = ctx.saved_tensors
        if grad_D is None:
            grad_D = torch.zeros_like(D)
        if grad_log_C is None:
            grad_log_C = torch.zeros_like(log_C)
        grad_x, grad_w = _C.normalized_accumulate_uz_backward(
            x, weights, D, log_C, grad_D.contiguous(), grad_log_C.contiguous(), shifts_i,
            ctx.log_weights, row_codes=ctx.row_codes, shared_weights=ctx.shared)
        return grad_x, _shared_grad(grad_w, ctx.shared), None, None, None, None


class _AccumulateUZScalarFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weights, shifts):
        if shifts.dim() != 2 or shifts.size(1) < 2:
            raise ValueError("accumulate_uz_scalar requires shifts of shape (S, >=2)")
        shifts_i = shifts[:, :2].to(device=x.device, dtype=torch.int64).contiguous()
        x_c, w_c = x.contiguous(), weights.contiguous()
        U, Z = _C.accumulate_uz_scalar_forward(x_c, w_c, shifts_i)
        ctx.save_for_backward(x_c, w_c, shifts_i)
        return U, Z

    @staticmethod
    def backward(ctx, grad_U, grad_Z):
        x, weights, shifts_i = ctx.saved_tensors
        acc = _C._acc_dtype(x.dtype)
        if grad_U is None:
            grad_U = torch.zeros(x.shape, dtype=acc, device=x.device)
        if grad_Z is None:
            grad_Z = torch.zeros(x.shape, dtype=acc, device=x.device)
        grad_x, grad_w = _C.accumulate_uz_scalar_backward(
            x, weights, grad_U.contiguous(), grad_Z.contiguous(), shifts_i)
        return grad_x, grad_w, None


# ---------------------------------------------------------------------------
# Extension guards (reference ops.py:494-546)
# ---------------------------------------------------------------------------

def _has_scalar_ext() -> bool:
    """True when the loaded library carries the scalar-accumulate entry points."""
    return _HAS_CUDA_EXT and hasattr(_C, "accumulate_uz_scalar_forward")


def _has_int64_index_ext() -> bool:
    """True only for a library with 64-bit shifts and flattened indices."""
    if not _HAS_CUDA_EXT or not hasattr(_C, "index_width_bits"):
        return False
    try:
        return int(_C.index_width_bits()) == 64
    except Exception:
        return False


def _require_cuda_ext(op_name: str, need_scalar: bool = False,
                      need_normalized: bool = False) -> None:
    """A GPU tensor must reach the HIP library; never the CPU reference."""
    if not _HAS_CUDA_EXT:
        raise RuntimeError(
            f"neural_shift_cuda.{op_name}: input is on the GPU but the HIP library "
            f"`_C` failed to load. Build it in this environment "
            f"(python -m neural_shift_cuda_amd.build).\n"
            f"  Underlying import error: "
            f"{type(_EXT_IMPORT_ERROR).__name__}: {_EXT_IMPORT_ERROR}") from _EXT_IMPORT_ERROR
    if not _has_int64_index_ext():
        raise RuntimeError(
            f"neural_shift_cuda.{op_name}: the loaded `_C` does not advertise 64-bit "
            f"shift/index width; rebuild the library from the current source.")
    if need_scalar and not hasattr(_C, "accumulate_uz_scalar_forward"):
        raise RuntimeError(
            f"neural_shift_cuda.{op_name}: the loaded `_C` has no accumulate_uz_scalar "
            f"entry points; rebuild the library from the current source.")
    if need_normalized and not hasattr(_C, "normalized_accumulate_uz_forward"):
        raise RuntimeError(
            f"neural_shift_cuda.{op_name}: the loaded `_C` has no normalized reduction "
            f"entry points; rebuild the library from the current source.")


# ---------------------------------------------------------------------------
# Public API (reference ops.py:576-719)
# ---------------------------------------------------------------------------

def shift_gather(guide: torch.Tensor, shifts: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Circularly shift `guide` by every (dx, dy) row of `shifts`.

    Returns gs (S*B, C, H, W) and mask (S*B, 1, H, W):
        gs[s*B + b, c, h, w]   = guide[b, c, (h+dx_s) mod H, (w+dy_s) mod W]
        mask[s*B + b, 0, h, w] = 1 iff 0 <= h+dx_s < H and 0 <= w+dy_s < W
    """
    if guide.is_cuda:
        _require_cuda_ext("shift_gather")
        return _ShiftGatherFn.apply(guide, shifts)
    return shift_gather_reference(guide, shifts)


def pair_gather(guide: torch.Tensor, shifts: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``shift_gather`` with the centre guide prepended on channels:
        pair[s*B + b, :C] = guide[b],  pair[s*B + b, C:] = shifted guide."""
    if guide.is_cuda:
        _require_cuda_ext("pair_gather")
        return _PairGatherFn.apply(guide, shifts)
    return pair_gather_reference(guide, shifts)


def accumulate_uz(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor, *,
                  periodic_inverse: bool = False, box_forward: bool = False,
                  shared_weights: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Accumulate U_num and Z over all shifts including the symmetric inverse
    branch.  `weights` (S*B, C, H, W) must already carry the forward box mask.
    Returns (U_num, Z) in the accumulator dtype; the caller forms U_num / Z.
    For very large positive weights prefer ``normalized_accumulate_uz``.

    The mirror term of a has_inverse row is dropped where its source wraps
    around the image (the reference's rule).  ``periodic_inverse=True`` (an
    extension) takes every mirror circularly instead: the fully periodic
    symmetric operator without materialising the rolled mirror planes as
    rows of their own (half the weight bytes).  In the table itself
    has_inverse = 2 selects the circular mirror row by row.
    ``box_forward=True`` (an extension) applies the forward box mask inside
    the kernels, so the weights need not carry it: the same result as
    multiplying each weight plane by its shift's box first, without that
    pass over the weights.  ``shared_weights=True`` (an extension) takes
    weights of shape (S*B, 1, H, W) used for every channel -- the
    single-head weights the reference installers broadcast to the channels
    (nekde_drunet_attn_patch.py:117-140) -- without materialising the
    broadcast copy; their gradient is the sum over the channels."""
    if x.is_cuda:
        table, codes = _mirror_table(shifts, periodic_inverse, box_forward)
        x_d, w_d = _device_operands(x, weights)
        _require_cuda_ext("accumulate_uz")
        return _AccumulateUZFn.apply(x_d, w_d, table, codes, bool(shared_weights))
    weights = _shared_operand(weights, x.shape[1], shared_weights)
    x_acc, w_acc = _promote_accumulation_inputs(x, weights)
    return accumulate_uz_reference(x_acc, w_acc, shifts, periodic_inverse=periodic_inverse,
                                   box_forward=box_forward)


def normalized_accumulate_uz(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor, *,
                             log_weights: bool = False, return_log_degree: bool = False,
                             validate: bool = True, periodic_inverse: bool = False,
                             box_forward: bool = False, shared_weights: bool = False):
    """Normalized denoiser D = K / C without overflow.

    weights: (S*B, C, H, W) positive weights (0 = mask) or, with
    log_weights=True, logits (-inf = mask).  shifts: (S, 3) integer
    (dx, dy, has_inverse).  Returns D, or (D, log_C) with
    return_log_degree=True.  validate checks the weight contract (an
    asynchronous device assertion on the GPU).  periodic_inverse and
    box_forward, shared_weights: as in ``accumulate_uz`` (a dropped forward
    term acts as a masked weight)."""
    x_d, w_d = _device_operands(x, weights)
    if validate:
        _validate_stable_weights(w_d, log_weights, asynchronous=x_d.is_cuda)
    if x_d.is_cuda:
        table, codes = _mirror_table(shifts, periodic_inverse, box_forward)
        _require_cuda_ext("normalized_accumulate_uz", need_normalized=True)
        D, log_C = _NormalizedAccumulateUZFn.apply(x_d, w_d, table, log_weights, codes,
                                                   bool(shared_weights))
    else:
        weights = _shared_operand(weights, x.shape[1], shared_weights)
        x_acc, w_acc = _promote_accumulation_inputs(x, weights)
        D, log_C = normalized_accumulate_uz_reference(
            x_acc, w_acc, shifts, log_weights=log_weights, return_log_degree=True,
            validate=False, periodic_inverse=periodic_inverse, box_forward=box_forward)
    return (D, log_C) if return_log_degree else D


def normalized_accumulate_uz_mixed(x: torch.Tensor, head_weights: torch.Tensor,
                                   head_mix: torch.Tensor, shifts: torch.Tensor, *,
                                   return_log_degree: bool = False,
                                   periodic_inverse: bool = False, box_forward: bool = False):
    """``normalized_accumulate_uz`` of head-mixed positive weights: channel c
    of shift s and batch b weighs sum_j head_mix[c, j] * head_weights[s*B+b, j]
    -- the attention installers' head-mixing product followed by the
    normalized accumulation (reference nekde_drunet_attn_patch.py:117-140,
    then :368-370).

    head_weights: (S*B, h, H, W) positive per-head weights (0 = mask);
    head_mix: (C, h).  On a GPU without autograd the mixing runs in the
    forward kernel's weight load for 2 <= h <= 4 on the shapes its scatter
    path serves: the (S*B, C, H, W) stack is never made, and each channel
    reads its h head planes (C*h plane reads per shift and pixel against
    h + 2C when mixing first).  Otherwise -- a gradient is wanted, another
    head count or shape, the CPU -- the heads are mixed first and
    ``normalized_accumulate_uz`` runs on the result.  The weights are not
    validated (the installers' validate=False)."""
    if head_weights.dim() != 4 or head_mix.dim() != 2:
        raise ValueError("head_weights must be (S*B, h, H, W) and head_mix (C, h)")
    SB, h, H, W = head_weights.shape
    if tuple(head_mix.shape) != (x.shape[1], h):
        raise ValueError(f"head_mix must be (C, h) = ({x.shape[1]}, {h}); "
                         f"got {tuple(head_mix.shape)}")
    wants_grad = torch.is_grad_enabled() and any(
        t.requires_grad for t in (x, head_weights, head_mix))
    if x.is_cuda and not wants_grad:
        x_d, hw_d = _device_operands(x, head_weights)
        table, codes = _mirror_table(shifts, periodic_inverse, box_forward)
        _require_cuda_ext("normalized_accumulate_uz_mixed", need_normalized=True)
        out = _C.normalized_accumulate_uz_forward_mixed(
            x_d.contiguous(), hw_d.contiguous(), head_mix, table, row_codes=codes)
        if out is not None:
            D, log_C = out
            return (D, log_C) if return_log_degree else D
    C = x.shape[1]
    mixed = mix_head_planes(head_weights.reshape(SB, h, H * W), head_mix)
    return normalized_accumulate_uz(x, mixed.view(SB, C, H, W), shifts,
                                    return_log_degree=return_log_degree, validate=False,
                                    periodic_inverse=periodic_inverse, box_forward=box_forward)


def accumulate_uz_scalar(x: torch.Tensor, weights: torch.Tensor, shifts: torch.Tensor
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """GASD scalar-per-transform accumulation:
        U[b, c, h, w] = sum_s w[s, b, c] x[b, c, (h+dx_s) mod H, (w+dy_s) mod W]
        Z[b, c, h, w] = sum_s w[s, b, c]
    weights (S, B, C) or (S, B) (shared over channels); shifts (S, >=2)."""
    if x.is_cuda:
        x_d, w_d = _device_operands(x, weights)
        _require_cuda_ext("accumulate_uz_scalar", need_scalar=True)
        if shifts.dim() != 2 or shifts.size(1) < 2:
            raise ValueError("accumulate_uz_scalar requires shifts of shape (S, >=2)")
        w_d = _broadcast_scalar_weights(w_d, shifts.size(0), x_d.shape[0], x_d.shape[1])
        return _AccumulateUZScalarFn.apply(x_d, w_d, shifts)
    x_acc, w_acc = _promote_accumulation_inputs(x, weights)
    return accumulate_uz_scalar_reference(x_acc, w_acc, shifts)


__all__ = [
    "shift_gather",
    "pair_gather",
    "accumulate_uz",
    "normalized_accumulate_uz",
    "normalized_accumulate_uz_mixed",
    "accumulate_uz_scalar",
    "shift_gather_reference",
    "pair_gather_reference",
    "accumulate_uz_reference",
    "normalized_accumulate_uz_reference",
    "accumulate_uz_scalar_reference",
]
