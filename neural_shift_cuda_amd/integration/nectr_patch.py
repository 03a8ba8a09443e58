"""NECTR installer (the official NECTR_denoiser and the legacy batched nekre).

``install_cuda_shift(cls)`` recognises the forward contract from the
signature:

* official: ``forward(x, reference=None, sig=None, cache=None,
  store_cache=False)`` (models/NECTR_models1.py:154, NECTR_models2.py);
* legacy: ``forward(x, guide=None, sig=None, batched=...)``.

With ``use_cuda_shift`` (default True) and ``model_type == 'concat'`` the
patched forward gathers (centre, shifted) guide pairs for the whole
half-plane with ``pair_gather`` (or ``shift_gather`` plus a concatenation when
``use_cuda_pair_gather`` is False), runs the model's unchanged head on the
batch, masks the wrapped neighbours, and aggregates once: positive weights
and the 'exp' head (kept as logits, so it cannot overflow before
normalization) through ``normalized_accumulate_uz``, other activations
through ``accumulate_uz`` and U/Z.  The degree comes back in float64 when it
is formed from log C.  Behaviour follows the reference installer
(nectr_patch.py:248-299); it applies to tensors on any device (the ops have
CPU paths).
"""
from __future__ import annotations

import functools
import inspect
from typing import Iterable, List, Tuple

import torch

from ..ops import accumulate_uz, normalized_accumulate_uz, pair_gather, shift_gather

Shift = Tuple[int, int, bool]
_UNSET = object()


class _NECTRWeightCache(dict):
    """Per-shift weight cache {(dx, dy): (B, C, H, W)} of the patched
    forward, tagged with its representation ('positive', 'log' or 'raw')."""

    def __init__(self, *args, weight_kind: str = "positive", **kwargs):
        super().__init__(*args, **kwargs)
        self.weight_kind = weight_kind


def _lazy_init(self) -> None:
    if not hasattr(self, "use_cuda_shift"):
        self.use_cuda_shift = True
    if not hasattr(self, "use_cuda_pair_gather"):
        self.use_cuda_pair_gather = True
    if not hasattr(self, "_nectr_cached_shift_tensor"):
        self._nectr_cached_shift_tensor = None
        self._nectr_cached_shift_key = None


def _collect_shifts(self) -> List[Shift]:
    """The model's half-plane (its own _collect_shifts when it has one): rows
    (dx in [-R, R], dy in [1, R], mirrored), then (dx in [0, R], 0), mirrored
    except (0, 0)."""
    own = getattr(self, "_collect_shifts", None)
    if callable(own):
        return [(int(dx), int(dy), bool(inv)) for dx, dy, inv in own()]
    R = int(self.window_rad)
    rows: List[Shift] = [(dx, dy, True) for dx in range(-R, R + 1) for dy in range(1, R + 1)]
    rows += [(dx, 0, dx != 0) for dx in range(0, R + 1)]
    return rows


def _get_shift_tensor(self, device: torch.device):
    shifts = _collect_shifts(self)
    key = (device.type, device.index, int(self.window_rad), tuple(shifts))
    if self._nectr_cached_shift_tensor is None or self._nectr_cached_shift_key != key:
        self._nectr_cached_shift_tensor = torch.tensor(
            [(dx, dy, int(inv)) for dx, dy, inv in shifts], dtype=torch.int64, device=device)
        self._nectr_cached_shift_key = key
    return shifts, self._nectr_cached_shift_tensor


def _is_model2(self) -> bool:
    return hasattr(self, "unet") and hasattr(self, "layer_norm")


def _channels_last(layer, t: torch.Tensor) -> torch.Tensor:
    return layer(t.permute(0, 2, 3, 1)).permute(0, 3, 1, 2)


def _head(self, pairs: torch.Tensor) -> Tuple[torch.Tensor, str]:
    """The model's head on concatenated (centre, shifted) pairs; returns the
    values and their kind: 'positive' weights, 'log' weights (the 'exp'
    activation before its exponential) or 'raw' values."""
    if _is_model2(self):
        v = self.out(_channels_last(self.layer_norm, self.unet(pairs)))
        if self.output_activation == "control_sigmoid":
            k, a, b = torch.chunk(v, 3, dim=1)
            return self.controlled_sigmoid(k, a, b) + 1e-8, "positive"
        return v, "raw"
    if self.output_activation == "sig":
        # the released 'sig' branch is the model's own business: call it
        Cg = pairs.shape[1] // 2
        fn = getattr(self, "N_theta", None) or self.compute_weights
        return fn(pairs[:, :Cg], pairs[:, Cg:]), "raw"
    v = pairs
    for block in self.proj:
        for i, layer in enumerate(block):
            v = _channels_last(layer, v) if i == 1 else layer(v)   # index 1: LayerNorm
    v = self.out(v)
    if self.output_activation == "exp":
        return v / self.sigma ** 2, "log"
    if self.output_activation == "control_sigmoid":
        k, a, b = torch.chunk(v, 3, dim=1)
        return self.controlled_sigmoid(k, a, b) + 1e-8, "positive"
    return v, "raw"


def _gather_and_weight(self, guide: torch.Tensor, table: torch.Tensor):
    """Masked weights (S*B, C, H, W) of every half-plane row and their kind."""
    guide = guide.contiguous()
    if getattr(self, "use_cuda_pair_gather", True):
        pairs, mask = pair_gather(guide, table)
    else:
        shifted, mask = shift_gather(guide, table)
        S = table.size(0)
        centre = guide.unsqueeze(0).expand(S, *guide.shape).reshape(-1, *guide.shape[1:])
        pairs = torch.cat((centre, shifted), dim=1)
    v, kind = _head(self, pairs)
    if kind == "log":
        v = torch.where(mask > 0, v, torch.full_like(v, -torch.inf))
    else:
        v = v * mask
    return v.contiguous(), kind


def _plain_cache_kind(self) -> str:
    """Kind of the values in a cache written by the unpatched forward."""
    if _is_model2(self):
        return "positive" if self.output_activation == "control_sigmoid" else "raw"
    if self.output_activation == "exp":
        return "exp-positive"
    if self.output_activation == "control_sigmoid":
        return "positive"
    return "raw"


def _weights_from_cache(self, cache, shifts: Iterable[Shift]):
    v = torch.cat([cache[(dx, dy)] for dx, dy, _ in shifts], dim=0)
    if isinstance(cache, _NECTRWeightCache):
        return v.contiguous(), cache.weight_kind
    kind = _plain_cache_kind(self)
    if kind == "exp-positive":
        # exponentiated weights of the unpatched 'exp' head: back to logits
        v = torch.where(v > 0, v.log(), torch.full_like(v, -torch.inf))
        kind = "log"
    return v.contiguous(), kind


def _store_cache(values: torch.Tensor, shifts: Iterable[Shift], B: int,
                 kind: str) -> _NECTRWeightCache:
    cache = _NECTRWeightCache(weight_kind=kind)
    for (dx, dy, _), v in zip(shifts, values.split(B, dim=0)):
        cache[(dx, dy)] = v
    return cache


def _aggregate(x: torch.Tensor, values: torch.Tensor, table: torch.Tensor, kind: str):
    """(U / Z, Z) for the given weights."""
    if kind in ("positive", "log"):
        D, log_Z = normalized_accumulate_uz(x.contiguous(), values, table,
                                            log_weights=(kind == "log"),
                                            return_log_degree=True, validate=True)
        return D, log_Z.to(torch.float64).exp()
    U, Z = accumulate_uz(x.contiguous(), values, table)
    return U / Z, Z


def _forward_official(self, x, reference=None, sig=None, cache=None, store_cache=False):
    guide = self.pre_activation(x if reference is None else reference, sigma=sig)
    shifts, table = _get_shift_tensor(self, x.device)
    if cache is None:
        values, kind = _gather_and_weight(self, guide, table)
        held = _store_cache(values, shifts, x.shape[0], kind) if store_cache else None
    else:
        values, kind = _weights_from_cache(self, cache, shifts)
        held = {} if store_cache else None
    D, Z = _aggregate(x, values, table, kind)
    return (D, Z, held) if store_cache else (D, Z)


def _forward_legacy(self, x, guide=None, sig=None):
    feats = self.pre_activation(x if guide is None else guide, sigma=sig)
    _, table = _get_shift_tensor(self, x.device)
    values, kind = _gather_and_weight(self, feats, table)
    return _aggregate(x, values, table, kind)


def install_cuda_shift(nectr_cls):
    """Patch an official NECTR_denoiser or a legacy batched nekre class
    (idempotent); returns the class.  ``instance.use_cuda_shift = False``
    routes back through the class's own forward."""
    if hasattr(nectr_cls, "_neural_shift_nectr_original_forward"):
        return nectr_cls
    fwd = nectr_cls.forward
    nectr_cls._neural_shift_nectr_original_forward = fwd
    params = inspect.signature(fwd).parameters

    if "batched" in params:
        dflt = params["batched"].default
        dflt = False if dflt is inspect.Parameter.empty else dflt

        @functools.wraps(fwd)
        def forward(self, x, guide=None, sig=None, batched=_UNSET):
            _lazy_init(self)
            b = dflt if batched is _UNSET else batched
            if (bool(b) and getattr(self, "use_cuda_shift", False)
                    and getattr(self, "model_type", "concat") == "concat"):
                return _forward_legacy(self, x, guide=guide, sig=sig)
            return fwd(self, x, guide=guide, sig=sig, batched=b)
    else:
        if not {"reference", "cache", "store_cache"}.issubset(params):
            raise TypeError(
                "NECTR patch expected either the legacy batched forward or the official "
                "reference/cache/store_cache forward contract")

        @functools.wraps(fwd)
        def forward(self, x, reference=None, sig=None, cache=None, store_cache=False):
            _lazy_init(self)
            if (getattr(self, "use_cuda_shift", False)
                    and getattr(self, "model_type", "concat") == "concat"):
                return _forward_official(self, x, reference=reference, sig=sig, cache=cache,
                                         store_cache=store_cache)
            return fwd(self, x, reference=reference, sig=sig, cache=cache,
                       store_cache=store_cache)

    nectr_cls.forward = forward
    return nectr_cls
