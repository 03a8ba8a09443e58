"""The degree-tie rule of the Metropolis backward's edge pass in its clamped
form (``tie_shares`` in csrc/metropolis.hip), checked on the CPU in exact
arithmetic.

d(loss)/d(max(d_q, d_j)) goes wholly to the larger degree and half to each
on a tie (torch.maximum's rule, reference metropolis.py:117-192 through
autograd).  On tiles whose degrees are all at least kMinEps the kernel forms
the two shares as clamp((d_q - d_j) * 2^K + 1/2, 0, 1) and clamp((d_q - d_j)
* -2^K + 1/2, 0, 1) with one rounded subtraction and two FMAs (K = 126 for
fp32, 1022 for fp64).  This emulates those steps (the subtraction rounded to
the kernel's type, the FMA's single rounding, the clamp) and checks that the
shares are exactly 1, 1/2 or 0 as the rule says, across binades, on
neighbouring floats and at the kMinEps gate, and that the form is wrong
below the gate (why the kernel keeps the compare-and-select form there).
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

# (dtype, K, kMinEps) as csrc/metropolis.hip's TieScale states them
CASES = [(np.float32, 126, 2.0 ** -104), (np.float64, 1022, 2.0 ** -970)]


def _fma_round(dtype, d, scale_exp, sign):
    """d * (sign * 2^scale_exp) + 1/2 with one rounding to dtype (exact
    rational arithmetic, round to nearest even; overflow to +-inf)."""
    exact = Fraction(float(d)) * Fraction(2) ** scale_exp * sign + Fraction(1, 2)
    finfo = np.finfo(dtype)
    if abs(exact) > Fraction(float(finfo.max)):
        # beyond the largest finite value by more than half an ulp: the
        # clamp only needs the sign, and such values round to +-inf
        return dtype(np.inf) if exact > 0 else dtype(-np.inf)
    # float() of a Fraction rounds correctly to binary64; one more rounding to
    # binary32 cannot cross a clamp boundary for the values that matter here
    # (|exact| >= 1 or <= 0 stays so, and exact 1/2 is representable)
    return dtype(float(exact))


def _shares(dtype, K, mine, other):
    d = dtype(mine) - dtype(other)  # the kernel's rounded subtraction
    sq = _fma_round(dtype, d, K, +1)
    sj = _fma_round(dtype, d, K, -1)
    clamp = lambda v: min(max(v, dtype(0)), dtype(1))  # noqa: E731
    return clamp(sq), clamp(sj)


def _rule(mine, other):
    return 1.0 if mine > other else (0.5 if mine == other else 0.0)


def _pairs(dtype, eps, rng):
    eps = dtype(eps)
    out = []
    # neighbouring floats across binades from the gate upward
    for e in list(range(int(np.log2(float(eps))), 40, 7)) + [0, 1, 20]:
        v = dtype(2.0 ** e)
        if v < eps:
            continue
        for a in (v, np.nextafter(v, dtype(np.inf)), np.nextafter(v, dtype(0))):
            if a < eps:
                continue
            b = np.nextafter(a, dtype(np.inf))
            out += [(a, b), (b, a), (a, a)]
    out += [(eps, np.nextafter(eps, dtype(np.inf))), (eps, eps)]
    # wide ratios and random pairs
    big = np.finfo(dtype).max
    out += [(big, eps), (eps, big), (big, np.nextafter(big, dtype(0))), (big, big)]
    lo, hi = np.log2(float(eps)), min(100.0, np.log2(float(big)) - 1)
    for _ in range(2000):
        a, b = (dtype(2.0 ** rng.uniform(lo, hi)) for _ in range(2))
        out.append((max(a, eps), max(b, eps)))
    return out


@pytest.mark.parametrize("dtype,K,min_eps", CASES, ids=["fp32", "fp64"])
def test_clamped_shares_follow_the_tie_rule(dtype, K, min_eps):
    rng = np.random.default_rng(11)
    for mine, other in _pairs(dtype, min_eps, rng):
        sq, sj = _shares(dtype, K, mine, other)
        want = _rule(mine, other)
        assert float(sq) == want and float(sj) == 1.0 - want, (mine, other, sq, sj)


@pytest.mark.parametrize("dtype,K,min_eps", CASES, ids=["fp32", "fp64"])
def test_clamped_shares_fail_below_the_gate(dtype, K, min_eps):
    """Far enough below kMinEps, neighbouring degrees differ by less than
    2^-(K+1): the scaled difference stays inside (-1/2, 1/2) and the shares
    come out strictly between 0 and 1, which the rule never gives."""
    tiny = np.nextafter(dtype(0), dtype(1))  # smallest subnormal
    a, b = tiny, dtype(2) * tiny
    sq, _ = _shares(dtype, K, b, a)
    assert 0.5 < float(sq) < 1.0
