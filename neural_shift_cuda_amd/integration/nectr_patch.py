"""NECTR installer: the official ``NECTR_denoiser`` and the legacy batched
``nekre`` (reference neural_shift_cuda/integration/nectr_patch.py:248-299).

``install_cuda_shift(cls)`` reads the forward contract from the signature:

* official: ``forward(x, reference=None, sig=None, cache=None,
  store_cache=False)`` (models/NECTR_models1.py:154, NECTR_models2.py);
* legacy: ``forward(x, guide=None, sig=None, batched=...)``, patched only
  when called batched.

The patched forward runs in three stages, whatever the contract:

1. weights - every half-plane (centre, shifted) guide pair goes through the
   model's own head in one batch (``pair_gather``, or ``shift_gather`` and
   a concatenation when ``use_cuda_pair_gather`` is False), or the weights
   come from a cache;
2. masking - neighbours reached only by wrap-around are dropped (a -inf
   logit, or a zero weight);
3. reduction - one ``normalized_accumulate_uz`` for positive weights and
   for the 'exp' head, which is kept as its logits so that nothing can
   overflow before normalization (the degree comes back in float64 from
   log C), or ``accumulate_uz`` and U / Z for any other activation.

It applies while ``use_cuda_shift`` (default True) is set and
``model_type == 'concat'``, on tensors on any device (the ops have CPU
paths).  Kept as interface: the forward signatures, the two flags above and
the ``weight_kind`` tag ('positive', 'log' or 'raw') of the caches the
patched forward returns.
"""
from __future__ import annotations

import functools
import inspect
from typing import Dict, List, Optional, Tuple

import torch

from ..ops import accumulate_uz, normalized_accumulate_uz, pair_gather, shift_gather
from ._common import mirror_rows

Row = Tuple[int, int, bool]
POSITIVE, LOG, RAW = "positive", "log", "raw"
_NOT_GIVEN = object()


class NECTRWeightCache(dict):
    """{(dx, dy): masked weights (B, C, H, W)} with the representation of
    the values in ``weight_kind``."""

    def __init__(self, *args, weight_kind: str = POSITIVE, **kwargs):
        super().__init__(*args, **kwargs)
        self.weight_kind = weight_kind


# the name under which earlier releases of this package exported the class
_NECTRWeightCache = NECTRWeightCache


# ---------------------------------------------------------------------------
# Per-instance state: the half-plane and its device tables
# ---------------------------------------------------------------------------

class _ShiftPlan:
    """The model's half-plane rows and one int64 table per device."""

    __slots__ = ("rows", "_tables")

    def __init__(self, rows: Tuple[Row, ...]):
        self.rows = rows
        self._tables: Dict[torch.device, torch.Tensor] = {}

    def table(self, device: torch.device) -> torch.Tensor:
        t = self._tables.get(device)
        if t is None:
            t = torch.tensor(mirror_rows(self.rows), dtype=torch.int64, device=device)
            self._tables[device] = t
        return t


def _halfplane(model) -> Tuple[Row, ...]:
    """The model's own enumeration when it has one, else the canonical
    half-plane of radius window_rad: (dx, dy >= 1) mirrored, then (dx >= 0,
    0) mirrored except (0, 0) (models/NECTR_models1.py:166-232)."""
    own = getattr(model, "_collect_shifts", None)
    if callable(own):
        return tuple((int(a), int(b), bool(c)) for a, b, c in own())
    R = int(model.window_rad)
    upper = [(dx, dy, True) for dx in range(-R, R + 1) for dy in range(1, R + 1)]
    axis = [(dx, 0, dx != 0) for dx in range(R + 1)]
    return tuple(upper + axis)


def _plan(model) -> _ShiftPlan:
    rows = _halfplane(model)
    plan = model.__dict__.get("_nsh_nectr_plan")
    if plan is None or plan.rows != rows:
        plan = _ShiftPlan(rows)
        model.__dict__["_nsh_nectr_plan"] = plan
    return plan


def _flags(model) -> None:
    for name in ("use_cuda_shift", "use_cuda_pair_gather"):
        if not hasattr(model, name):
            setattr(model, name, True)


# ---------------------------------------------------------------------------
# Stage 1: weights
# ---------------------------------------------------------------------------

def _is_unet_head(model) -> bool:
    """NECTR_models2: a U-Net head with a channels-last layer norm."""
    return hasattr(model, "unet") and hasattr(model, "layer_norm")


def _native_kind(model) -> str:
    """Representation the head's activation produces: 'exp' is handled as
    its logits; 'exp-positive' marks the exponentiated values the unpatched
    forward caches for it."""
    act = model.output_activation
    if act == "control_sigmoid":
        return POSITIVE
    if act == "exp" and not _is_unet_head(model):
        return LOG
    return RAW


def _norm_last(layer, t: torch.Tensor) -> torch.Tensor:
    """A channels-last layer (LayerNorm) on an NCHW tensor."""
    return layer(t.permute(0, 2, 3, 1)).permute(0, 3, 1, 2)


def _positive_head(model, v: torch.Tensor) -> torch.Tensor:
    k, a, b = torch.chunk(v, 3, dim=1)
    return model.controlled_sigmoid(k, a, b) + 1e-8


def _head(model, pairs: torch.Tensor) -> torch.Tensor:
    """The head's values for a batch of concatenated (centre, shifted) guide
    features, in the representation _native_kind names."""
    if _is_unet_head(model):
        v = model.out(_norm_last(model.layer_norm, model.unet(pairs)))
        return _positive_head(model, v) if _native_kind(model) == POSITIVE else v
    if model.output_activation == "sig":
        # The released 'sig' branch belongs to the model: call its own
        # weight function on the two halves of the pair.
        half = pairs.shape[1] // 2
        fn = getattr(model, "N_theta", None) or model.compute_weights
        return fn(pairs[:, :half], pairs[:, half:])
    v = pairs
    for block in model.proj:          # (conv, channels-last norm, activation)
        for i, layer in enumerate(block):
            v = _norm_last(layer, v) if i == 1 else layer(v)
    v = model.out(v)
    kind = _native_kind(model)
    if kind == LOG:
        return v / model.sigma ** 2
    if kind == POSITIVE:
        return _positive_head(model, v)
    return v


def _pairs(model, guide: torch.Tensor, table: torch.Tensor):
    """(pairs (S*B, 2C, H, W), wrap mask (S*B, 1, H, W)) of the half-plane."""
    if getattr(model, "use_cuda_pair_gather", True):
        return pair_gather(guide, table)
    shifted, mask = shift_gather(guide, table)
    reps = table.size(0)
    centre = guide.repeat(reps, 1, 1, 1)
    return torch.cat((centre, shifted), dim=1), mask


def _masked(values: torch.Tensor, mask: torch.Tensor, kind: str) -> torch.Tensor:
    """Stage 2: drop the wrapped neighbours (-inf logits, zero weights)."""
    if kind == LOG:
        return values.masked_fill(mask <= 0, float("-inf"))
    return values * mask


def _weights_from_head(model, guide: torch.Tensor, table: torch.Tensor):
    pairs, mask = _pairs(model, guide.contiguous(), table)
    kind = _native_kind(model)
    return _masked(_head(model, pairs), mask, kind).contiguous(), kind


def _weights_from_cache(model, cache, rows):
    """Weights of a cache: this installer's own (tagged) or one written by
    the class's unpatched forward (exponentiated for the 'exp' head, turned
    back into logits here)."""
    stacked = torch.cat([cache[(dx, dy)] for dx, dy, _ in rows], dim=0).contiguous()
    kind = getattr(cache, "weight_kind", None)
    if kind is not None:
        return stacked, kind
    kind = _native_kind(model)
    if kind == LOG:
        positive = stacked > 0
        safe = torch.where(positive, stacked, torch.ones_like(stacked))
        stacked = torch.where(positive, safe.log(), torch.full_like(stacked, float("-inf")))
    return stacked, kind


def _cache_of(values: torch.Tensor, rows, batch: int, kind: str) -> NECTRWeightCache:
    cache = NECTRWeightCache(weight_kind=kind)
    for (dx, dy, _), block in zip(rows, values.split(batch, dim=0)):
        cache[(dx, dy)] = block
    return cache


# ---------------------------------------------------------------------------
# Stage 3: reduction
# ---------------------------------------------------------------------------

def _reduce(x: torch.Tensor, values: torch.Tensor, table: torch.Tensor, kind: str):
    """(U / Z, Z): normalized for positive weights and logits, plain U / Z
    for anything else (a softmax over weights of either sign is not
    defined)."""
    if kind == RAW:
        U, Z = accumulate_uz(x.contiguous(), values, table)
        return U / Z, Z
    D, log_Z = normalized_accumulate_uz(x.contiguous(), values, table,
                                        log_weights=(kind == LOG), return_log_degree=True,
                                        validate=True)
    # the official API returns the degree itself: exponentiate in float64 so
    # that a degree beyond the float32 range survives
    return D, log_Z.to(torch.float64).exp()


def _denoise(model, x, guide_input, sig, cache=None, keep_cache=False):
    """(D, Z, cache or None) of the patched forward."""
    plan = _plan(model)
    table = plan.table(x.device)
    # the guide features are formed first even when a cache is given, as the
    # class's own forward does (its sigma checks raise the same errors)
    guide = model.pre_activation(guide_input, sigma=sig)
    if cache is None:
        values, kind = _weights_from_head(model, guide, table)
        held = _cache_of(values, plan.rows, x.shape[0], kind) if keep_cache else None
    else:
        values, kind = _weights_from_cache(model, cache, plan.rows)
        held = {} if keep_cache else None
    D, Z = _reduce(x, values, table, kind)
    return D, Z, held


def _active(model) -> bool:
    return bool(getattr(model, "use_cuda_shift", False)) and \
        getattr(model, "model_type", "concat") == "concat"


# ---------------------------------------------------------------------------
# Installation
# ---------------------------------------------------------------------------

def _official(original):
    @functools.wraps(original)
    def forward(self, x, reference=None, sig=None, cache=None, store_cache=False):
        _flags(self)
        if not _active(self):
            return original(self, x, reference=reference, sig=sig, cache=cache,
                            store_cache=store_cache)
        D, Z, held = _denoise(self, x, x if reference is None else reference, sig,
                              cache=cache, keep_cache=store_cache)
        return (D, Z, held) if store_cache else (D, Z)
    return forward


def _legacy(original, batched_default):
    @functools.wraps(original)
    def forward(self, x, guide=None, sig=None, batched=_NOT_GIVEN):
        _flags(self)
        run_batched = batched_default if batched is _NOT_GIVEN else batched
        if not (run_batched and _active(self)):
            return original(self, x, guide=guide, sig=sig, batched=run_batched)
        D, Z, _ = _denoise(self, x, x if guide is None else guide, sig)
        return D, Z
    return forward


def install_cuda_shift(nectr_cls):
    """Patch an official NECTR_denoiser or a legacy batched nekre class
    (idempotent); returns the class.  ``instance.use_cuda_shift = False``
    routes back through the class's own forward."""
    if nectr_cls.__dict__.get("_nsh_nectr_installed", False):
        return nectr_cls
    original = nectr_cls.forward
    params = inspect.signature(original).parameters
    if "batched" in params:
        default = params["batched"].default
        patched = _legacy(original, False if default is inspect.Parameter.empty else default)
    elif {"reference", "cache", "store_cache"} <= set(params):
        patched = _official(original)
    else:
        raise TypeError("install_cuda_shift_nectr: the class's forward has neither the legacy "
                        "batched contract nor the official reference/cache/store_cache forward "
                        "contract")
    nectr_cls.forward = patched
    nectr_cls._nsh_nectr_installed = True
    return nectr_cls
