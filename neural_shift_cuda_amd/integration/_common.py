"""Pieces shared by the model installers: sigma normalisation, head mixing,
the finite-window (comp_box) mask, periodic mirror rows and the patched-method
plumbing.  Behaviour follows the reference installers
(neural_shift_cuda/integration/nekde_drunet_attn_patch.py:103-140,
gasd_drunet_attn_patch.py:103-143)."""
from __future__ import annotations

import inspect
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from ..ops import mix_head_planes


def normalise_sigma(x: torch.Tensor, sig):
    """sig as a (B, 1, 1, 1)-broadcastable tensor: a Python number becomes a
    (B, 1, 1, 1) tensor, a 0-d tensor is expanded, a batch-1 tensor is
    expanded to B; anything else is returned as given."""
    if sig is None:
        return None
    B = x.shape[0]
    if not torch.is_tensor(sig):
        return x.new_full((B, 1, 1, 1), float(sig))
    if sig.dim() == 0:
        return sig.view(1, 1, 1, 1).expand(B, 1, 1, 1)
    if sig.shape[0] == 1 and B > 1:
        return sig.expand(B, *sig.shape[1:])
    return sig


def head_mix_matrix(model) -> Optional[torch.Tensor]:
    """(C, n_heads) mixing matrix from the model's raw_head_mix, with the
    model's positivity map head_mix_pos_act ('softmax' over heads by default,
    'softplus', otherwise relu); None without raw_head_mix."""
    raw = getattr(model, "raw_head_mix", None)
    if raw is None:
        return None
    act = getattr(model, "head_mix_pos_act", "softmax")
    if act == "softmax":
        return F.softmax(raw, dim=1)
    if act == "softplus":
        return F.softplus(raw)
    return F.relu(raw)


def mix_planes(mat: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """sum_j mat[c, j] * w[:, j] for w (N, h, P) and mat (C, h): (N, C, P)
    (ops.mix_head_planes: the HIP kernels on the GPU, a broadcast product
    summed over the heads otherwise)."""
    return mix_head_planes(w, mat)


def mix_heads(w_stack: torch.Tensor, C: int, mat: Optional[torch.Tensor]) -> torch.Tensor:
    """Per-head weights (S, B, h, H, W) to per-channel weights (S, B, C, H, W):
    one head is broadcast, a mixing matrix is applied over the head axis, C
    heads are used as they are, otherwise the head mean is broadcast."""
    S, B, h, H, W = w_stack.shape
    if h == 1:
        return w_stack.expand(S, B, C, H, W)
    if mat is not None:
        out = mix_planes(mat.to(w_stack.dtype), w_stack.reshape(S * B, h, H * W))
        return out.view(S, B, C, H, W)
    if h == C:
        return w_stack
    return w_stack.mean(dim=2, keepdim=True).expand(S, B, C, H, W)


def box_mask_stack(shifts_xy: Sequence[Tuple[int, int]], H: int, W: int, device,
                   dtype) -> torch.Tensor:
    """(S, 1, 1, H, W) finite-window mask: 1 where the gathered neighbour
    (h + dx, w + dy) lies inside the image (the zero-padded ones box of the
    models, sliced at the shift)."""
    d = torch.tensor([[int(dx), int(dy)] for dx, dy in shifts_xy], dtype=torch.int64,
                     device=device)
    S = d.shape[0]
    hh = torch.arange(H, device=device).view(1, H, 1) + d[:, 0].view(S, 1, 1)
    ww = torch.arange(W, device=device).view(1, 1, W) + d[:, 1].view(S, 1, 1)
    ok = (hh >= 0) & (hh < H) & (ww >= 0) & (ww < W)
    return ok.to(dtype).view(S, 1, 1, H, W)


def channel_operand(w_stack: torch.Tensor) -> Tuple[torch.Tensor, bool]:
    """(weights, shared) for the ops from per-channel weights (S, B, C, H, W).
    A stack broadcast over the channels (one head, or the head mean: stride
    0 on the channel axis) goes to the ops as its single (S*B, 1, H, W)
    plane with shared_weights=True, so the kernels read it for every channel
    instead of a materialised copy per channel; any other stack is made
    contiguous as (S*B, C, H, W)."""
    S, B, C, H, W = w_stack.shape
    if C > 1 and w_stack.stride(2) == 0:
        return w_stack[:, :, :1].reshape(S * B, 1, H, W).contiguous(), True
    return w_stack.reshape(S * B, C, H, W).contiguous(), False


def mirror_rows(shift_list) -> List[Tuple[int, int, int]]:
    """(dx, dy, has_inverse) rows of a half-plane for the accumulations."""
    return [(int(dx), int(dy), int(bool(inv))) for dx, dy, inv in shift_list]


def operator_options(periodic: bool, box: bool = False) -> dict:
    """Keyword options of accumulate_uz / normalized_accumulate_uz for a
    half-plane operator: the fully periodic one takes every mirror
    circularly (periodic_inverse) and `box` lets the kernels apply the
    forward box mask to the unmasked weights (box_forward).  The reference
    installers express the periodic operator with explicit mirror rows whose
    weights are the rolled forward weights (nekde_drunet_attn_patch.py:350-366)
    and multiply the weights by the box beforehand (:337-345); these options
    compute the same operators from the half-plane weights alone, without
    either pass over them."""
    return {"periodic_inverse": bool(periodic), "box_forward": bool(box)}


def signature_default(fn, name: str, fallback):
    """(accepts `name`, its default or `fallback`) for a wrapped method."""
    params = inspect.signature(fn).parameters
    if name in params:
        return True, params[name].default
    return False, fallback


def check_cached_weights(x: torch.Tensor, C: int, weights, n_shifts: int, what: str) -> None:
    """The checks every cached-guide path makes before packing."""
    if x.dim() != 4:
        raise ValueError(f"x must have shape (B,C,H,W), got {tuple(x.shape)}.")
    if x.size(1) != C:
        raise ValueError(
            f"cached weights have C={C} channels but x has {x.size(1)}; rebuild the "
            "cache for this channel count.")
    if len(weights) != n_shifts or not weights:
        raise ValueError(f"cached {what} must contain one tensor per cached shift.")
    for w in weights:
        if tuple(w.shape) != tuple(x.shape):
            raise ValueError(
                "cached weights and x must have identical (B,C,H,W) shapes; got "
                f"{tuple(w.shape)} and {tuple(x.shape)}.")
        if w.device != x.device or w.dtype != x.dtype:
            raise ValueError("cached weights and x must share device and dtype.")


def cache_hit(state, cache, x: torch.Tensor) -> bool:
    """A packed state (cache, shape, device, dtype, ...) is valid for x."""
    return (state is not None and state[0] is cache and state[1] == tuple(x.shape)
            and state[2] == x.device and state[3] == x.dtype)
