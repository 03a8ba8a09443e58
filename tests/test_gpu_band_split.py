"""One GPU's share of a spatially sharded accumulate_uz, emulated on one GPU.

A large image shards into horizontal bands of Hb rows per GPU; each GPU runs
the op on its band padded with R halo rows above and below (the rows its
neighbours own) and keeps the band's own Hb rows.  Every term that reaches an
output row of the band (forward: w_s[p] x[p+s] and the mirror w_s[p-s]
x[p-s]; backward: the same pairs through gU, gZ) lies within R rows of it, so
it is inside the padded band, and the band's own wrap-around links halo rows
only to halo rows.  The kept rows therefore equal the whole-image result up to
the order of summation (the tile borders differ).

Bands away from the image's top and bottom edge are exact under the
reference's mirror rule (a mirror term is dropped where its source wraps the
image); a band at the edge would need the image's global row origin for that
rule, so with the reference rule only interior bands are compared.  With
circular mirrors (periodic_inverse) no term depends on the image edge and
every band, the edge ones with wrapped halos included, must agree.

Tolerance: two results that each carry the accumulation error bound, so
2 * rtol of the per-element absolute-value sum (the same op on |x|, |w|,
|gU|, |gZ|).
"""
from __future__ import annotations

import sys

import pytest
import torch

from helpers import assert_bound, rtol_for
from neural_shift_cuda import accumulate_uz
from neural_shift_cuda_amd.workloads import (box_stack, halfplane_shifts, softplus_weights,
                                             synthetic_image)

HAS_GPU = torch.cuda.is_available()
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _run(x, w, sh, gU, gZ, periodic):
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV), periodic_inverse=periodic)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    torch.cuda.synchronize()
    return U.detach().cpu(), Z.detach().cpu(), xd.grad.cpu(), wd.grad.cpu()


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("periodic", [False, True])
def test_gpu_band_split(periodic):
    # 4 bands of 64 rows, R = 6 (S = 85): padded bands of 76 rows take the
    # scatter path (3 tile rows, the last one 12 rows), like the whole image
    R, n, Hb, W = 6, 4, 64, 256
    H = n * Hb
    sh = halfplane_shifts(R)
    S = sh.size(0)
    x = synthetic_image(1, 1, H, W, seed=7)
    w = softplus_weights((S, 1, H, W), seed=8)
    if not periodic:
        w = w * box_stack(sh, 1, H, W)
    g = torch.Generator().manual_seed(9)
    gU = torch.randn(1, 1, H, W, generator=g)
    gZ = torch.randn(1, 1, H, W, generator=g)
    _case(f"band split periodic={periodic}: whole image 1x1x{H}x{W}, S={S}")
    full = _run(x, w, sh, gU, gZ, periodic)
    scale = _run(x.abs(), w.abs(), sh, gU.abs(), gZ.abs(), periodic)
    rt = 2 * rtol_for(torch.float32)
    for b in (range(n) if periodic else range(1, n - 1)):
        rows = torch.arange(b * Hb - R, (b + 1) * Hb + R) % H
        _case(f"band split periodic={periodic}: band {b}, rows {b * Hb}..{(b + 1) * Hb - 1} "
              f"padded to {rows.numel()}")
        out = _run(x[:, :, rows], w[:, :, rows], sh, gU[:, :, rows], gZ[:, :, rows], periodic)
        keep = slice(R, R + Hb)
        mine = slice(b * Hb, (b + 1) * Hb)
        for name, a, e, s in zip(("U", "Z", "grad_x", "grad_w"), out, full, scale):
            assert_bound(a[:, :, keep], e[:, :, mine], s[:, :, mine], rt, f"band {b} {name}")
