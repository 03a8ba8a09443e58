"""Metropolis-Hastings aggregation over half-plane shift weights.

    metropolis_aggregate(w_half, img, shifts, use_box, eps=1e-6,
                         checkpoint_train=True) -> (Wx, d_hat)

Same signature, dispatch rules and results as the reference module
neural_shift_cuda/metropolis.py (trishitmg/neural_shift_cuda,
metropolis.py:195-238):

* w_half (B, S, C, H, W): forward weights of the canonical half-plane
  shifts; shifts: a Python list of (dx, dy, has_inverse); use_box drops
  neighbours reached only by wrap-around.
* d = K e; K_hat_ij = w_ij / max(d_i, d_j, eps); d_hat = K_hat e;
  Wx = x - d_hat x + K_hat x.  The inverse edge's weight is the circular
  shift of the forward weight, so K_hat and W are symmetric.
* GPU tensors with autograd disabled run the fused two-pass HIP kernel
  (``_C.metropolis_aggregate``).  With autograd enabled on the GPU, shapes
  the fused backward serves (``_C.metropolis_backward_supported``) run the
  same forward and a fused two-pass HIP backward
  (``_C.metropolis_aggregate_backward``) that yields the gradients of the
  differentiable path below.  Elsewhere the differentiable path runs: it
  expands the half-plane into explicit edges and uses the ``accumulate_uz``
  and ``shift_gather`` ops (HIP kernels on the GPU, the CPU references
  otherwise), under gradient checkpointing by default.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import torch
from torch.autograd.function import once_differentiable
from torch.utils.checkpoint import checkpoint

from .ops import _box, _gather2d, accumulate_uz, shift_gather

try:
    from . import _C as _ext
    _HAS_EXT = (hasattr(_ext, "metropolis_aggregate") and hasattr(_ext, "index_width_bits")
                and int(_ext.index_width_bits()) == 64)
except Exception:  # library not built / no HIP runtime
    _ext = None
    _HAS_EXT = False


def _shifts_to_tensor(shifts: Sequence[Tuple[int, int, bool]], device) -> torch.Tensor:
    rows = [[int(dx), int(dy), int(bool(inv))] for (dx, dy, inv) in shifts]
    table = torch.tensor(rows, dtype=torch.long, device=device)
    if _HAS_EXT and rows:
        # the table's radius, known here, so the library never reads it back
        clamp = 1 << 30
        _ext.remember_table_radius(
            table, max(min(max(abs(dx), abs(dy)), clamp) for dx, dy, _ in rows))
    return table


def metropolis_aggregate_torch(w_half: torch.Tensor, img: torch.Tensor,
                               shifts: Sequence[Tuple[int, int, bool]], use_box: bool,
                               eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """Direct PyTorch statement of the operator (reference metropolis.py:54-114):
    degree pass, then per-edge Metropolis weights, serially over shifts."""
    B, S, C, H, W = w_half.shape
    dev, dt = img.device, img.dtype

    def keep(dx, dy):
        return _box(H, W, dx, dy, dt, dev) if use_box else None

    fwd, inv = [], []
    d = torch.zeros_like(img)
    for s, (dx, dy, has_inv) in enumerate(shifts):
        kf = keep(dx, dy)
        wf = w_half[:, s] if kf is None else w_half[:, s] * kf
        fwd.append(wf)
        d = d + wf
        if has_inv:
            ki = keep(-dx, -dy)
            wi = _gather2d(wf, -dx, -dy)
            wi = wi if ki is None else wi * ki
            inv.append(wi)
            d = d + wi
        else:
            inv.append(None)
    kx = torch.zeros_like(img)
    dh = torch.zeros_like(img)
    for s, (dx, dy, has_inv) in enumerate(shifts):
        wk = fwd[s] / torch.maximum(d, _gather2d(d, dx, dy)).clamp_min(eps)
        kx = kx + wk * _gather2d(img, dx, dy)
        dh = dh + wk
        if has_inv:
            wk = inv[s] / torch.maximum(d, _gather2d(d, -dx, -dy)).clamp_min(eps)
            kx = kx + wk * _gather2d(img, -dx, -dy)
            dh = dh + wk
    return img - dh * img + kx, dh


def metropolis_aggregate_fused(w_half: torch.Tensor, img: torch.Tensor,
                               shifts: Sequence[Tuple[int, int, bool]], use_box: bool,
                               eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """Differentiable path on the shared primitives (reference
    metropolis.py:117-192).  Every half-plane row becomes explicit edges with
    has_inverse = 0: the forward edge (w box(+s)) and, for has_inverse rows,
    the mirror edge whose weight is the circular shift of the forward weight
    by +s, box-masked at -s when use_box.  Then
        d      = Z of accumulate_uz(img, w_edges)
        wk     = w_edges / max(d, shift_gather(d), eps)
        khat_x, d_hat = accumulate_uz(img, wk)."""
    B, S, C, H, W = w_half.shape
    dev, dt = img.device, img.dtype
    edge_w: List[torch.Tensor] = []
    edge_rows: List[List[int]] = []
    for s, (dx, dy, has_inv) in enumerate(shifts):
        wf = w_half[:, s]
        if use_box:
            wf = wf * _box(H, W, dx, dy, dt, dev)
        edge_w.append(wf)
        edge_rows.append([int(dx), int(dy), 0])
        if has_inv:
            wm = torch.roll(wf, shifts=(int(dx), int(dy)), dims=(-2, -1))
            if use_box:
                wm = wm * _box(H, W, -dx, -dy, dt, dev)
            edge_w.append(wm)
            edge_rows.append([-int(dx), -int(dy), 0])
    E = len(edge_rows)
    w_edges = torch.stack(edge_w, 0).reshape(E * B, C, H, W).contiguous()
    table = torch.tensor(edge_rows, dtype=torch.long, device=dev)

    _, d = accumulate_uz(img, w_edges, table)
    d_nb, _ = shift_gather(d, table[:, :2].contiguous())
    denom = torch.maximum(d.repeat(E, 1, 1, 1), d_nb).clamp_min(eps)
    khat_x, d_hat = accumulate_uz(img, w_edges / denom, table)
    return img - d_hat * img + khat_x, d_hat


# Route differentiable GPU calls through the fused backward where the shape
# allows it (False: always the explicit-edge path).
FUSED_BACKWARD = True


class _MetropolisFusedFn(torch.autograd.Function):
    """Fused forward + fused backward.  The gradients equal those of
    ``metropolis_aggregate_fused`` under autograd (torch.maximum's even split
    on ties and clamp_min's gate included); the backward keeps the forward's
    raw degree and d_hat instead of the (2S-1) edge planes."""

    @staticmethod
    def forward(ctx, w_half, img, table, use_box, eps):
        Wx, d_hat, degree = _ext.metropolis_aggregate_with_degree(w_half, img, table, use_box,
                                                                  eps)
        ctx.save_for_backward(w_half, img, table, degree, d_hat)
        ctx.use_box = use_box
        ctx.eps = eps
        return Wx, d_hat

    @staticmethod
    @once_differentiable
    def backward(ctx, gWx, gdh):
        w_half, img, table, degree, d_hat = ctx.saved_tensors
        gw, gx = _ext.metropolis_aggregate_backward(w_half, img, table, ctx.use_box, ctx.eps,
                                                    degree, d_hat, gWx, gdh)
        return (gw if ctx.needs_input_grad[0] else None,
                gx if ctx.needs_input_grad[1] else None, None, None, None)


def _fused_backward_ok(w_half: torch.Tensor, img: torch.Tensor) -> bool:
    return (FUSED_BACKWARD and _HAS_EXT and w_half.is_cuda and img.is_cuda
            and w_half.dtype == img.dtype and w_half.dim() == 5 and img.dim() == 4
            and tuple(img.shape) == (w_half.shape[0],) + tuple(w_half.shape[2:])
            and hasattr(_ext, "metropolis_backward_supported")
            and _ext.metropolis_backward_supported(w_half))


def metropolis_aggregate(w_half: torch.Tensor, img: torch.Tensor,
                         shifts: Sequence[Tuple[int, int, bool]], use_box: bool,
                         eps: float = 1e-6, checkpoint_train: bool = True
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """(Wx, d_hat) with Wx = (1 - d_hat) x + K_hat x and d_hat = K_hat e.

    GPU + no autograd: the fused HIP kernel.  GPU + autograd on a shape the
    fused backward serves: the fused kernel and its fused backward.  Otherwise
    the differentiable edge path, wrapped in gradient checkpointing when
    ``checkpoint_train`` so the (E*B, C, H, W) edge tensors are recomputed in
    backward instead of kept.
    """
    if img.is_cuda and not torch.is_grad_enabled():
        if not _HAS_EXT:
            from .ops import _require_cuda_ext
            _require_cuda_ext("metropolis_aggregate")
        table = _shifts_to_tensor(shifts, img.device)
        Wx, d_hat = _ext.metropolis_aggregate(w_half.contiguous(), img.contiguous(), table,
                                              int(bool(use_box)), float(eps))
        return Wx, d_hat
    needs_grad = torch.is_grad_enabled() and (w_half.requires_grad or img.requires_grad)
    if needs_grad and img.is_cuda and _fused_backward_ok(w_half, img):
        table = _shifts_to_tensor(shifts, img.device)
        return _MetropolisFusedFn.apply(w_half.contiguous(), img.contiguous(), table,
                                        int(bool(use_box)), float(eps))
    if checkpoint_train and needs_grad:
        def _run(w_, x_):
            return metropolis_aggregate_fused(w_, x_, shifts, use_box, eps)
        return checkpoint(_run, w_half, img, use_reentrant=False)
    return metropolis_aggregate_fused(w_half, img, shifts, use_box, eps)


__all__ = [
    "metropolis_aggregate",
    "metropolis_aggregate_torch",
    "metropolis_aggregate_fused",
]
