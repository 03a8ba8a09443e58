"""MI355X (gfx950) implementation of the neural_shift_cuda shift-window ops.

The public surface mirrors the reference package neural_shift_cuda
(trishitmg/neural_shift_cuda, __init__.py:1-28); the ``neural_shift_cuda``
package in this repository re-exports this one under that name so existing
callers import it unchanged.
"""
from .ops import (
    accumulate_uz,
    accumulate_uz_reference,
    accumulate_uz_scalar,
    accumulate_uz_scalar_reference,
    normalized_accumulate_uz,
    normalized_accumulate_uz_reference,
    pair_gather,
    pair_gather_reference,
    shift_gather,
    shift_gather_reference,
)
from .metropolis import metropolis_aggregate

__version__ = "0.12.0"
__all__ = [
    "shift_gather",
    "pair_gather",
    "accumulate_uz",
    "normalized_accumulate_uz",
    "accumulate_uz_scalar",
    "shift_gather_reference",
    "pair_gather_reference",
    "accumulate_uz_reference",
    "normalized_accumulate_uz_reference",
    "accumulate_uz_scalar_reference",
    "metropolis_aggregate",
]
