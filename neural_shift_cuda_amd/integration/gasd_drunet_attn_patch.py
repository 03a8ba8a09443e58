"""GASD (full (2R+1)^2 window, per-pixel weights, row-stochastic) installer.

``install_cuda_shift(GASDDRUNetAttn)`` patches ``forward``, the transpose
actions ``_KT_action``, ``NLM_transpose`` and ``laplacian_grw``, and, when
the class has them, the fixed-guide ``forward_cached``, ``_KT_action_cached``
and ``laplacian_grw_cached``; CPU inputs and ``use_cuda_shift = False`` keep
the class's methods.  Behaviour follows the reference installer
(gasd_drunet_attn_patch.py:621-757):

* every window shift is a forward-only row (has_inverse = 0), so
  K x = sum_s w_s (.) x(. + s) and W = Z^-1 K is only row-stochastic;
* ``comp_box`` (default True) multiplies each weight by the finite-window
  mask; False leaves the operator circulant;
* K^T y = sum_s pi_s^-1 (w_s (.) y) = sum_s pi_s^-1(w_s) (.) pi_s^-1(y): the
  weights rolled by their own shift with the shifts negated, i.e. another
  forward accumulation;
* NLM_transpose and laplacian_grw take the degree and the forward from the
  same weight stack, so each costs one network pass.
"""
from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint as grad_checkpoint

from ..ops import (accumulate_uz, normalized_accumulate_uz, normalized_accumulate_uz_mixed,
                   shift_gather)
from ._common import (box_mask_stack, cache_hit, channel_operand, check_cached_weights,
                      head_mix_matrix, mix_heads, normalise_sigma, signature_default)


def _get_shift_tensor(self, device: torch.device) -> torch.Tensor:
    """(S, 3) int64 table of the full window, has_inverse = 0 on every row."""
    if (getattr(self, "_cached_shift_tensor", None) is None
            or getattr(self, "_cached_shift_device", None) != device):
        rows = [(int(dx), int(dy), 0) for dx, dy in self._collect_shifts()]
        self._cached_shift_tensor = torch.tensor(rows, dtype=torch.int64, device=device)
        self._cached_shift_device = device
    return self._cached_shift_tensor


def _get_kt_shift_tensor(self, device: torch.device) -> torch.Tensor:
    """The transpose table: every shift negated, has_inverse = 0."""
    if (getattr(self, "_cached_kt_shift_tensor", None) is None
            or getattr(self, "_cached_kt_shift_device", None) != device):
        rows = [(-int(dx), -int(dy), 0) for dx, dy in self._collect_shifts()]
        self._cached_kt_shift_tensor = torch.tensor(rows, dtype=torch.int64, device=device)
        self._cached_kt_shift_device = device
    return self._cached_kt_shift_tensor


def _roll_each(w_stack: torch.Tensor, shifts_xy) -> torch.Tensor:
    """Slice s of (S, ..., H, W) rolled by its own shift (dx_s, dy_s):
    out[s, ..., h, w] = w[s, ..., (h - dx_s) mod H, (w - dy_s) mod W], as one
    gather over flattened planes."""
    S = w_stack.shape[0]
    H, W = w_stack.shape[-2:]
    dev = w_stack.device
    d = torch.tensor([[int(dx), int(dy)] for dx, dy in shifts_xy], dtype=torch.int64,
                     device=dev)
    src_h = (torch.arange(H, device=dev).view(1, H, 1) - d[:, 0].view(S, 1, 1)) % H
    src_w = (torch.arange(W, device=dev).view(1, 1, W) - d[:, 1].view(S, 1, 1)) % W
    idx = (src_h * W + src_w).view(S, 1, H * W)
    flat = w_stack.reshape(S, -1, H * W)
    return flat.gather(2, idx.expand(S, flat.shape[1], H * W)).view_as(w_stack)


def _head_stack(self, x: torch.Tensor, guide, sig):
    """Per-head weights (S, B, h, H, W) of every window shift, unmasked, and
    the (C, h) head-mixing matrix (None without one)."""
    B, C, H, W = x.shape
    R = self.window_rad
    phi = self.pre_activation(x if guide is None else guide, sigma=sig).contiguous()
    shift_list = self._collect_shifts()
    mat = head_mix_matrix(self)
    if hasattr(self, "_gather_core"):
        padded = F.pad(phi, (R, R, R, R), mode="circular")
        return torch.stack(list(self._all_shift_weights(phi, padded, sig, shift_list)),
                           dim=0), mat
    else:
        shifts_xy = _get_shift_tensor(self, x.device)[:, :2].contiguous()
        S = shifts_xy.shape[0]
        chunk = self.max_batch_shifts if self.max_batch_shifts is not None else S
        head = (self.attn_head.logit if self.output_activation == "softmax"
                else self.attn_head.weight)
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
        w = torch.stack(tiles, dim=1)                   # (B, S, h, H, W)
        if self.output_activation == "softmax":
            # joint softmax over the window; the mask is applied after it
            w = F.softmax(w - w.amax(dim=1, keepdim=True), dim=1)
        return w.permute(1, 0, 2, 3, 4).contiguous(), mat


def _weight_stack(self, x: torch.Tensor, guide, sig, apply_box: bool = True) -> torch.Tensor:
    """Per-channel weights (S, B, C, H, W) of every window shift, with the
    finite-window mask applied when comp_box and `apply_box`."""
    B, C, H, W = x.shape
    w, mat = _head_stack(self, x, guide, sig)
    w = mix_heads(w, C, mat)
    if apply_box and bool(getattr(self, "comp_box", True)):
        w = w * box_mask_stack(self._collect_shifts(), H, W, x.device, w.dtype)
    return w


def _begin(self):
    if not self.training:
        self.max_batch_shifts = 10   # the models' test-time chunking


def _end(self):
    if not self.training:
        self.max_batch_shifts = None


def _forward_cuda(self, x: torch.Tensor, guide: Optional[torch.Tensor] = None,
                  sig: Optional[torch.Tensor] = None, return_D: bool = True):
    """(Z^-1 K x, Z) from one normalized accumulation (Z None unless return_D)."""
    _begin(self)
    sig = normalise_sigma(x, sig)
    # the kernels apply the comp_box mask to the forward terms (box_forward),
    # single-head weights stay one plane per (shift, batch), and a (C, h)
    # mixing matrix is applied in the kernels' weight load when no gradient
    # is wanted (normalized_accumulate_uz_mixed; with one, the op mixes first)
    w_heads, mat = _head_stack(self, x, guide, sig)
    box = bool(getattr(self, "comp_box", True))
    table = _get_shift_tensor(self, x.device)
    S, B, h, H, W = w_heads.shape
    if mat is not None and h > 1:
        D, log_Z = normalized_accumulate_uz_mixed(
            x.contiguous(), w_heads.reshape(S * B, h, H, W), mat, table,
            return_log_degree=True, box_forward=box)
    else:
        w_all, shared = channel_operand(mix_heads(w_heads, x.shape[1], mat))
        D, log_Z = normalized_accumulate_uz(x.contiguous(), w_all, table,
                                            return_log_degree=True, validate=False,
                                            box_forward=box, shared_weights=shared)
    _end(self)
    return (D, log_Z.exp()) if return_D else (D, None)


def _transpose_weights(self, w: torch.Tensor) -> torch.Tensor:
    S, B, C, H, W = w.shape
    return _roll_each(w, self._collect_shifts()).reshape(S * B, C, H, W).contiguous()


def _kt_action_cuda(self, y: torch.Tensor, guide=None, sig=None) -> torch.Tensor:
    """K^T y."""
    _begin(self)
    sig = normalise_sigma(y, sig)
    w = _weight_stack(self, y, guide, sig)
    KT, _ = accumulate_uz(y.contiguous(), _transpose_weights(self, w),
                          _get_kt_shift_tensor(self, y.device))
    _end(self)
    return KT


def _nlm_transpose_cuda(self, x: torch.Tensor, guide=None, sig=None, return_D: bool = False):
    """W^T x = K^T D^-1 x with D = sum_s w_s (the forward degree), one
    network pass."""
    _begin(self)
    sig = normalise_sigma(x, sig)
    w = _weight_stack(self, x, x if guide is None else guide, sig)
    D = w.sum(dim=0)
    WT, _ = accumulate_uz((x / D.clamp_min(1e-6)).contiguous(), _transpose_weights(self, w),
                          _get_kt_shift_tensor(self, x.device))
    _end(self)
    return (WT, D) if return_D else (WT, None)


def _laplacian_grw_cuda(self, x: torch.Tensor, guide, sig=None, eps=1e-10) -> torch.Tensor:
    """L^T L x with L = I - D^-1 K, from one weight stack: z = x - Wx, then
    z - K^T (z / max(D, 1e-6)), the floor applied in log space."""
    _begin(self)
    sig = normalise_sigma(x, sig)
    w = _weight_stack(self, x, x if guide is None else guide, sig)
    S, B, C, H, W = w.shape
    Wx, log_Z = normalized_accumulate_uz(x.contiguous(), w.reshape(S * B, C, H, W).contiguous(),
                                         _get_shift_tensor(self, x.device),
                                         return_log_degree=True, validate=False)
    z = x - Wx
    dz = z * (-torch.maximum(log_Z, log_Z.new_tensor(1e-6).log())).exp()
    KT, _ = accumulate_uz(dz.contiguous(), _transpose_weights(self, w),
                          _get_kt_shift_tensor(self, x.device))
    _end(self)
    return z - KT


# ---- fixed-guide cache (cache.C, cache.shifts, cache.w_list, cache.Z) ------

def _cached_gasd_reduction_inputs(self, x: torch.Tensor, cache):
    """Packed (weights, table) of a GASD weight cache, kept on the model as
    (cache, shape, device, dtype, weights, table); a new pack drops the
    transpose pack."""
    state = getattr(self, "_gasd_parallel_weight_cache", None)
    if cache_hit(state, cache, x):
        return state[4], state[5]
    shifts = list(cache.shifts)
    weights = list(cache.w_list)
    check_cached_weights(x, cache.C, weights, len(shifts), "w_list")
    w_all = torch.stack(weights, dim=0).reshape(-1, *x.shape[1:]).contiguous()
    table = torch.tensor([(int(dx), int(dy), 0) for dx, dy in shifts], dtype=torch.int64,
                         device=x.device)
    self._gasd_parallel_weight_cache = (cache, tuple(x.shape), x.device, x.dtype, w_all, table)
    self._gasd_parallel_transpose_cache = None
    return w_all, table


def _cached_gasd_transpose_inputs(self, x: torch.Tensor, cache):
    """Packed transpose operands (rolled weights, negated table), built on
    first use."""
    w_all, _ = _cached_gasd_reduction_inputs(self, x, cache)
    state = getattr(self, "_gasd_parallel_transpose_cache", None)
    if cache_hit(state, cache, x):
        return state[4], state[5]
    shifts = list(cache.shifts)
    S = len(shifts)
    w_t = _roll_each(w_all.view(S, *x.shape), shifts).reshape(-1, *x.shape[1:]).contiguous()
    table = torch.tensor([(-int(dx), -int(dy), 0) for dx, dy in shifts], dtype=torch.int64,
                         device=x.device)
    self._gasd_parallel_transpose_cache = (cache, tuple(x.shape), x.device, x.dtype, w_t, table)
    return w_t, table


def _forward_cached_cuda(self, x: torch.Tensor, cache, return_D: bool = True):
    """Cached Z^-1 K x; the degree is cache.Z when present, else exp(log C)."""
    w_all, table = _cached_gasd_reduction_inputs(self, x, cache)
    D, log_Z = normalized_accumulate_uz(x.contiguous(), w_all, table,
                                        return_log_degree=True, validate=False)
    if not return_D:
        return D, None
    return D, (cache.Z if getattr(cache, "Z", None) is not None else log_Z.exp())


def _kt_action_cached_cuda(self, y: torch.Tensor, cache) -> torch.Tensor:
    """Cached raw K^T y (unnormalized: a row-normalized transpose would be a
    different operator)."""
    w_t, table = _cached_gasd_transpose_inputs(self, y, cache)
    KT, _ = accumulate_uz(y.contiguous(), w_t, table)
    return KT


def _laplacian_grw_cached_cuda(self, x: torch.Tensor, cache, eps=1e-10) -> torch.Tensor:
    """Cached L^T L x (normalized forward, raw transpose, degree floor 1e-6)."""
    w_all, table = _cached_gasd_reduction_inputs(self, x, cache)
    Wx, log_Z = normalized_accumulate_uz(x.contiguous(), w_all, table,
                                         return_log_degree=True, validate=False)
    z = x - Wx
    dz = z * (-torch.maximum(log_Z, log_Z.new_tensor(1e-6).log())).exp()
    return z - _kt_action_cached_cuda(self, dz, cache)


def _lazy_init(self) -> None:
    if not hasattr(self, "_cached_shift_tensor"):
        self.use_cuda_shift = True
        self._cached_shift_tensor = None
        self._cached_shift_device = None


def _on_gpu(self, t: torch.Tensor) -> bool:
    return bool(getattr(self, "use_cuda_shift", True)) and t.is_cuda


def install_cuda_shift(model_cls):
    """Patch a GASDDRUNetAttn class (idempotent); returns the class."""
    if getattr(model_cls, "_cuda_shift_installed", False):
        return model_cls
    model_cls._get_shift_tensor = _get_shift_tensor
    fwd = model_cls.forward
    fwd_has_D, fwd_D = signature_default(fwd, "return_D", True)

    def forward(self, x, guide=None, sig=None, return_D=fwd_D):
        _lazy_init(self)
        if _on_gpu(self, x):
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
            if _on_gpu(self, x):
                return _forward_cached_cuda(self, x, cache, return_D=return_D)
            if c_has_D:
                return cached(self, x, cache, return_D=return_D)
            return cached(self, x, cache)

        model_cls.forward_cached = forward_cached

    kt_cached = getattr(model_cls, "_KT_action_cached", None)
    if kt_cached is not None:
        def kt_action_cached(self, y, cache):
            if not hasattr(self, "use_cuda_shift"):
                self.use_cuda_shift = True
            if _on_gpu(self, y):
                return _kt_action_cached_cuda(self, y, cache)
            return kt_cached(self, y, cache)

        model_cls._KT_action_cached = kt_action_cached

    lap_cached = getattr(model_cls, "laplacian_grw_cached", None)
    if lap_cached is not None:
        def laplacian_grw_cached(self, x, cache, eps=1e-10):
            if not hasattr(self, "use_cuda_shift"):
                self.use_cuda_shift = True
            if _on_gpu(self, x):
                return _laplacian_grw_cached_cuda(self, x, cache, eps=eps)
            return lap_cached(self, x, cache, eps=eps)

        model_cls.laplacian_grw_cached = laplacian_grw_cached

    kt = getattr(model_cls, "_KT_action", None)
    nlm_t = getattr(model_cls, "NLM_transpose", None)
    lap = getattr(model_cls, "laplacian_grw", None)

    def _missing(self, name):
        return AttributeError(
            f"{type(self).__name__} has no reference {name}; add the arch-level methods "
            "before installing.")

    def kt_action(self, y, guide=None, sig=None):
        _lazy_init(self)
        if _on_gpu(self, y):
            return _kt_action_cuda(self, y, guide=guide, sig=sig)
        if kt is None:
            raise _missing(self, "_KT_action")
        return kt(self, y, guide=guide, sig=sig)

    def nlm_transpose(self, x, guide=None, sig=None, return_D=False):
        _lazy_init(self)
        if _on_gpu(self, x):
            return _nlm_transpose_cuda(self, x, guide=guide, sig=sig, return_D=return_D)
        if nlm_t is None:
            raise _missing(self, "NLM_transpose")
        return nlm_t(self, x, guide=guide, sig=sig, return_D=return_D)

    def laplacian_grw(self, x, guide, sig=None, eps=1e-10):
        _lazy_init(self)
        if _on_gpu(self, x):
            return _laplacian_grw_cuda(self, x, guide, sig=sig, eps=eps)
        if lap is None:
            raise _missing(self, "laplacian_grw")
        return lap(self, x, guide, sig=sig, eps=eps)

    model_cls._KT_action = kt_action
    model_cls.NLM_transpose = nlm_transpose
    model_cls.laplacian_grw = laplacian_grw
    model_cls._cuda_shift_installed = True
    return model_cls
