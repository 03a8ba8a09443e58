"""Metropolis NeKDe installer.

``install_cuda_shift(NeKDeMetropolisDRUNetAttn)`` patches ``forward`` (and
``forward_cached`` when the class has it): GPU inputs build the head-mixed
half-plane weights with the model's own helpers and run the fused
``metropolis_aggregate`` op (symmetric by construction; its fused backward
serves training on the shapes it covers); CPU inputs and
``use_cuda_shift = False`` keep the class's methods.  DSG_NLM and the
laplacian_* methods of these models call ``forward``, so they follow.
Behaviour follows the reference installer (nkd_metropolis_attn_patch.py:
193-255); ``comp_box`` (default True) is passed as ``use_box``.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from ..metropolis import metropolis_aggregate
from ..ops import accumulate_uz
from ._common import (cache_hit, check_cached_weights, mirror_rows, operator_options,
                      signature_default)


def _build_w_half(self, x: torch.Tensor, guide: Optional[torch.Tensor], sig):
    """Head-mixed half-plane forward weights (B, S, C, H, W) and the shift
    list, from the model's _normalise_sigma, pre_activation,
    _halfplane_weights, _head_mix_matrix and _mix_heads."""
    B, C, H, W = x.shape
    R = self.window_rad
    sig = self._normalise_sigma(x, sig)
    z = x if guide is None else guide
    if z.shape != x.shape:
        raise ValueError(
            f"guide must have the same shape as x; got {tuple(z.shape)} and {tuple(x.shape)}.")
    if z.device != x.device or z.dtype != x.dtype:
        raise ValueError("guide and x must share device and dtype.")
    phi = self.pre_activation(z, sigma=sig)
    padded = F.pad(phi, (R, R, R, R), mode="circular")
    shifts = self._collect_shifts()
    per_shift = self._halfplane_weights(phi, padded, sig, shifts)
    mat = self._head_mix_matrix()
    w_half = torch.stack([self._mix_heads(per_shift[i], C, mat) for i in range(len(shifts))],
                         dim=1).contiguous()
    return w_half, shifts


def _forward_cuda(self, x: torch.Tensor, guide: Optional[torch.Tensor] = None,
                  sig: Optional[torch.Tensor] = None, return_D: bool = False):
    """(W x, d_hat) of the model's forward via metropolis_aggregate."""
    if x.dim() != 4:
        raise ValueError(f"x must have shape (B,C,H,W), got {tuple(x.shape)}.")
    w_half, shifts = _build_w_half(self, x, guide, sig)
    eps = max(float(self.metropolis_eps), torch.finfo(x.dtype).tiny)
    Wx, d_hat = metropolis_aggregate(w_half, x, shifts, use_box=bool(getattr(self, "comp_box", True)),
                                     eps=eps)
    return (Wx, d_hat) if return_D else (Wx, None)


def _cached_metropolis_reduction_inputs(self, x: torch.Tensor, cache):
    """Packed (weights, table, op options) of cached Metropolis edges
    (cache.C, cache.shifts, cache.w_hat_fwd_list: the K_hat forward edges,
    cache.comp_box), kept on the model like the other installers' packs."""
    state = getattr(self, "_metropolis_parallel_weight_cache", None)
    if cache_hit(state, cache, x):
        return state[4], state[5], state[6]
    shifts = list(cache.shifts)
    weights = list(cache.w_hat_fwd_list)
    check_cached_weights(x, cache.C, weights, len(shifts), "w_hat_fwd_list")
    w_all = torch.stack(weights, dim=0).reshape(-1, *x.shape[1:]).contiguous()
    table = torch.tensor(mirror_rows(shifts), dtype=torch.int64, device=x.device)
    opts = operator_options(periodic=not bool(cache.comp_box))
    self._metropolis_parallel_weight_cache = (cache, tuple(x.shape), x.device, x.dtype, w_all,
                                              table, opts)
    return w_all, table, opts


def _forward_cached_cuda(self, x: torch.Tensor, cache, return_D: bool = False):
    """Cached W x = x - d_hat x + K_hat x with one accumulation; d_hat is
    cache.degree_hat when present, else the accumulated degree."""
    w_all, table, opts = _cached_metropolis_reduction_inputs(self, x, cache)
    khat_x, d_red = accumulate_uz(x.contiguous(), w_all, table, **opts)
    d_hat = cache.degree_hat if getattr(cache, "degree_hat", None) is not None else d_red
    Wx = x - d_hat * x + khat_x
    return (Wx, d_hat) if return_D else (Wx, None)


def install_cuda_shift(model_cls):
    """Patch a Metropolis NeKDe class (idempotent); returns the class."""
    if getattr(model_cls, "_metropolis_cuda_forward_installed", False):
        return model_cls
    if not hasattr(model_cls, "forward"):
        raise TypeError("model_cls must provide forward(x, guide=None, sig=None).")
    fwd = model_cls.forward
    fwd_has_D, fwd_D = signature_default(fwd, "return_D", False)

    def forward(self, x, guide=None, sig=None, return_D=fwd_D):
        if not hasattr(self, "use_cuda_shift"):
            self.use_cuda_shift = True
        if self.use_cuda_shift and x.is_cuda:
            return _forward_cuda(self, x, guide=guide, sig=sig, return_D=return_D)
        if fwd_has_D:
            return fwd(self, x, guide=guide, sig=sig, return_D=return_D)
        return fwd(self, x, guide=guide, sig=sig)

    model_cls.forward = forward

    cached = getattr(model_cls, "forward_cached", None)
    if cached is not None:
        c_has_D, c_D = signature_default(cached, "return_D", False)

        def forward_cached(self, x, cache, return_D=c_D):
            if not hasattr(self, "use_cuda_shift"):
                self.use_cuda_shift = True
            if getattr(self, "use_cuda_shift", True) and x.is_cuda:
                return _forward_cached_cuda(self, x, cache, return_D=return_D)
            if c_has_D:
                return cached(self, x, cache, return_D=return_D)
            return cached(self, x, cache)

        model_cls.forward_cached = forward_cached

    model_cls._metropolis_cuda_forward_installed = True
    return model_cls
