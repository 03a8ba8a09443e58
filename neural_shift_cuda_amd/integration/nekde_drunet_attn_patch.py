"""NeKDe (half-plane, per-pixel weights, symmetric) installer.

``install_cuda_shift(NeKDeDRUNetAttn)`` patches ``forward``,
``forward_cached`` (when the class has it) and ``_KT_action`` so that GPU
inputs run the shift-window ops of this package; CPU inputs, and instances
with ``use_cuda_shift = False``, keep the class's own methods.  Behaviour
follows the reference installer (nekde_drunet_attn_patch.py:576-662):

* weights: classes with ``_gather_core`` produce them with their own
  ``_halfplane_weights`` (one network pass); older classes go through
  ``shift_gather`` and ``attn_head.logit``/``weight`` per chunk of shifts,
  with a joint softmax over the half-plane;
* heads are mixed to channels (``head_mix_pos_act``; a (C, h) mixing
  matrix is applied in the kernels' weight load when no gradient is
  wanted, ``normalized_accumulate_uz_mixed``), and
* ``comp_box`` (default True) selects the finite-window operator (forward
  edge masked inside the kernels, ``box_forward=True``, instead of a
  multiply over the weights; mirror edge masked by the ops' has_inverse
  rule) or the fully periodic one (circular mirrors, ``periodic_inverse=True``:
  the same operator as the reference's explicit mirror rows from half the
  weight planes);
* the accumulation is one ``normalized_accumulate_uz`` call (overflow-safe
  D = K/C plus log C), ``_KT_action`` one or two ``accumulate_uz`` calls
  (K is symmetric).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint as grad_checkpoint

from ..ops import (accumulate_uz, normalized_accumulate_uz, normalized_accumulate_uz_mixed,
                   shift_gather)
from ._common import (cache_hit, channel_operand, check_cached_weights, head_mix_matrix,
                      mirror_rows, mix_heads, operator_options,
                      normalise_sigma, signature_default)


def _get_shift_tensor(self, device: torch.device) -> torch.Tensor:
    """(S, 3) int64 table of the model's half-plane, cached per device."""
    if (getattr(self, "_cached_shift_tensor", None) is None
            or getattr(self, "_cached_shift_device", None) != device):
        rows = [(int(dx), int(dy), int(bool(inv))) for dx, dy, inv in self._collect_shifts()]
        self._cached_shift_tensor = torch.tensor(rows, dtype=torch.int64, device=device)
        self._cached_shift_device = device
    return self._cached_shift_tensor


def _reduction_operands(w_stack: torch.Tensor, shift_list, use_box: bool, device
                        ) -> Tuple[torch.Tensor, torch.Tensor, dict]:
    """(weights, table, op options) for the accumulation from unmasked
    per-channel weights (S, B, C, H, W).  Finite window: the kernels drop
    the forward edges outside the box (box_forward) and the mirror edges
    whose source wraps; periodic: circular mirrors (periodic_inverse).
    Single-head weights stay one plane per (shift, batch) (shared_weights)."""
    w_all, shared = channel_operand(w_stack)
    table = torch.tensor(mirror_rows(shift_list), dtype=torch.int64, device=device)
    opts = operator_options(periodic=not use_box, box=use_box)
    opts["shared_weights"] = shared
    return w_all, table, opts


def _head_stack(self, x: torch.Tensor, guide, sig):
    """Per-head half-plane weights (S, B, h, H, W), unmasked, the (C, h)
    head-mixing matrix (None without one) and the shift list."""
    B, C, H, W = x.shape
    R = self.window_rad
    phi = self.pre_activation(x if guide is None else guide, sigma=sig).contiguous()
    shift_list = self._collect_shifts()
    mat = head_mix_matrix(self)
    if hasattr(self, "_gather_core"):
        padded = F.pad(phi, (R, R, R, R), mode="circular")
        w = torch.stack(list(self._halfplane_weights(phi, padded, sig, shift_list)), dim=0)
        return w, mat, shift_list

    # older heads: gathered guide features per chunk of shifts
    shifts_xy = _get_shift_tensor(self, x.device)[:, :2].contiguous()
    S = shifts_xy.shape[0]
    chunk = self.max_batch_shifts if self.max_batch_shifts is not None else S
    head = self.attn_head.logit if self.output_activation == "softmax" else self.attn_head.weight
    tiles: List[torch.Tensor] = []
    for start in range(0, S, chunk):
        n = min(chunk, S - start)
        phi_s, _ = shift_gather(phi, shifts_xy[start:start + n])
        phi_c = phi.repeat(n, 1, 1, 1)
        sig_b = sig.repeat(n, 1, 1, 1) if sig is not None else None
        if self.use_grad_checkpoint:
            t = grad_checkpoint(head, phi_c, phi_s, sig_b, use_reentrant=False)
        else:
            t = head(phi_c, phi_s, sig_b)
        tiles.extend(t.split(B, dim=0))
    w = torch.stack(tiles, dim=1)                       # (B, S, h, H, W)
    if self.output_activation == "softmax":
        w = F.softmax(w - w.amax(dim=1, keepdim=True), dim=1)
    return w.permute(1, 0, 2, 3, 4).contiguous(), mat, shift_list


def _weight_stack(self, x: torch.Tensor, guide, sig) -> Tuple[torch.Tensor, list]:
    """Per-channel half-plane weights (S, B, C, H, W), unmasked, and the
    shift list."""
    w, mat, shift_list = _head_stack(self, x, guide, sig)
    return mix_heads(w, x.shape[1], mat), shift_list


def _forward_cuda(self, x: torch.Tensor, guide: Optional[torch.Tensor] = None,
                  sig: Optional[torch.Tensor] = None, return_D: bool = True):
    """(D, Z) of the model's forward: D = Z^-1 K x from one normalized
    accumulation, Z = K e (None unless return_D)."""
    if not self.training:
        self.max_batch_shifts = 10   # the models' test-time chunking
    sig = normalise_sigma(x, sig)
    w_heads, mat, shift_list = _head_stack(self, x, guide, sig)
    use_box = bool(getattr(self, "comp_box", True))
    S, B, h, H, W = w_heads.shape
    if mat is not None and h > 1:
        # the mixing product in the kernels' weight load (without autograd;
        # with it the op mixes first)
        table = torch.tensor(mirror_rows(shift_list), dtype=torch.int64, device=x.device)
        D, log_Z = normalized_accumulate_uz_mixed(
            x.contiguous(), w_heads.reshape(S * B, h, H, W), mat, table,
            return_log_degree=True, **operator_options(periodic=not use_box, box=use_box))
    else:
        w_all, table, opts = _reduction_operands(mix_heads(w_heads, x.shape[1], mat),
                                                 shift_list, use_box, x.device)
        D, log_Z = normalized_accumulate_uz(x.contiguous(), w_all, table,
                                            return_log_degree=True, validate=False, **opts)
    if not self.training:
        self.max_batch_shifts = None
    return (D, log_Z.exp()) if return_D else (D, None)


def _kt_action_cuda(self, y: torch.Tensor, guide=None, sig=None, return_D: bool = False,
                    apply_Dinv: bool = False):
    """K^T y (K is symmetric: the forward accumulation), or K^T D^-1 y with
    apply_Dinv, D = K e from the first accumulation; one network pass."""
    if not self.training:
        self.max_batch_shifts = 10
    sig = normalise_sigma(y, sig)
    w_stack, shift_list = _weight_stack(self, y, guide, sig)
    use_box = bool(getattr(self, "comp_box", True))
    w_all, table, opts = _reduction_operands(w_stack, shift_list, use_box, y.device)
    U, Z = accumulate_uz(y.contiguous(), w_all, table, **opts)
    if apply_Dinv:
        U, _ = accumulate_uz((y / Z.clamp_min(1e-6)).contiguous(), w_all, table, **opts)
    if not self.training:
        self.max_batch_shifts = None
    return (U, Z) if return_D else (U, None)


def _cached_reduction_inputs(self, x: torch.Tensor, cache):
    """Packed (weights, table, op options) of a fixed-guide cache (cache.C,
    cache.shifts, cache.w_fwd_list: final forward edges, cache.comp_box),
    kept on the model as (cache, shape, device, dtype, weights, table,
    options) and reused while the same cache object and input geometry come
    back."""
    state = getattr(self, "_nekde_parallel_weight_cache", None)
    if cache_hit(state, cache, x):
        return state[4], state[5], state[6]
    shifts = list(cache.shifts)
    weights = list(cache.w_fwd_list)
    check_cached_weights(x, cache.C, weights, len(shifts), "w_fwd_list")
    w_all = torch.stack(weights, dim=0).reshape(-1, *x.shape[1:]).contiguous()
    table = torch.tensor(mirror_rows(shifts), dtype=torch.int64, device=x.device)
    opts = operator_options(periodic=not bool(cache.comp_box))
    self._nekde_parallel_weight_cache = (cache, tuple(x.shape), x.device, x.dtype, w_all, table,
                                         opts)
    return w_all, table, opts


def _forward_cached_cuda(self, x: torch.Tensor, cache, return_D: bool = True):
    """Cached-guide forward: one normalized accumulation of the packed cache;
    the degree is cache.D when the cache holds it, else exp(log C)."""
    w_all, table, opts = _cached_reduction_inputs(self, x, cache)
    D, log_Z = normalized_accumulate_uz(x.contiguous(), w_all, table,
                                        return_log_degree=True, validate=False, **opts)
    if not return_D:
        return D, None
    degree = cache.D if getattr(cache, "D", None) is not None else log_Z.exp()
    return D, degree


def _lazy_init(self) -> None:
    if not hasattr(self, "_cached_shift_tensor"):
        self.use_cuda_shift = True
        self._cached_shift_tensor = None
        self._cached_shift_device = None


def install_cuda_shift(model_cls):
    """Patch a NeKDeDRUNetAttn class (idempotent); returns the class."""
    if getattr(model_cls, "_cuda_shift_installed", False):
        return model_cls
    model_cls._get_shift_tensor = _get_shift_tensor
    fwd = model_cls.forward
    fwd_has_D, fwd_D = signature_default(fwd, "return_D", True)

    def forward(self, x, guide=None, sig=None, return_D=fwd_D):
        _lazy_init(self)
        if getattr(self, "use_cuda_shift", True) and x.is_cuda:
            return _forward_cuda(self, x, guide=guide, sig=sig, return_D=return_D)
        if fwd_has_D:
            return fwd(self, x, guide=guide, sig=sig, return_D=return_D)
        return fwd(self, x, guide=guide, sig=sig)

    model_cls.forward = forward

    cached = getattr(model_cls, "forward_cached", None)
    if cached is not None:
        c_has_D, c_D = signature_default(cached, "return_D", True)

        def forward_cached(self, x, cache, return_D=c_D):
            if not hasattr(self, "use_cuda_shift"):
                self.use_cuda_shift = True
            if getattr(self, "use_cuda_shift", True) and x.is_cuda:
                return _forward_cached_cuda(self, x, cache, return_D=return_D)
            if c_has_D:
                return cached(self, x, cache, return_D=return_D)
            return cached(self, x, cache)

        model_cls.forward_cached = forward_cached

    kt = getattr(model_cls, "_KT_action", None)

    def kt_action(self, y, guide=None, sig=None, return_D=False, apply_Dinv=False):
        _lazy_init(self)
        if getattr(self, "use_cuda_shift", True) and y.is_cuda:
            return _kt_action_cuda(self, y, guide=guide, sig=sig, return_D=return_D,
                                   apply_Dinv=apply_Dinv)
        if kt is None:
            raise AttributeError(
                f"{type(self).__name__} has no reference _KT_action; add the arch-level "
                "_KT_action/NLM_transpose before installing.")
        return kt(self, y, guide=guide, sig=sig, return_D=return_D, apply_Dinv=apply_Dinv)

    model_cls._KT_action = kt_action
    model_cls._cuda_shift_installed = True
    return model_cls
