"""One GPU's share of a spatially sharded accumulate_uz, emulated on one GPU.

A large image shards into horizontal bands of Hb rows per GPU; each GPU runs
the op on its band padded with R halo rows above and below (the rows its
neighbours own, taken around the image at its top and bottom edge) and keeps
the band's own Hb rows.  Every term that reaches an output row of the band
(forward: w_s[p] x[p+s] and the mirror w_s[p-s] x[p-s]; backward: the same
pairs through gU, gZ) lies within R rows of it, so it is inside the padded
band.  The box tests (a mirror term dropped where its source wraps the image,
row code 4's forward box) need the rows' place in the image: the band entry
points (nsh_accumulate_uz_{forward,backward}_band) take the band's first
row, row_origin = b * Hb - R (negative for the top band, whose halo holds the
image's last rows), and the image height.  Then every band, the edge bands
included, reproduces the whole-image rows it keeps, up to the order of
summation (the tile borders differ).

Cases: the reference mirror rule, circular mirrors, the forward box applied
in the kernels (row codes), a table beyond the 8-pixel tile border (the
gather form inside the scatter launch), a radius-10 table on the 16-pixel
border tiles, and bands small enough for the gather kernels.

Tolerance: two results that each carry the accumulation error bound, so
2 * rtol of the per-element absolute-value sum (the same call on |x|, |w|,
|gU|, |gZ|).
"""
from __future__ import annotations

import sys

import pytest
import torch

from helpers import assert_bound, rtol_for
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import box_stack, halfplane_shifts, synthetic_image

HAS_GPU = torch.cuda.is_available()
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _table(name):
    if name == "far12":
        return torch.tensor([[0, 1, 1], [12, -3, 1], [-9, 2, 1], [3, 11, 0], [1, 0, 1],
                             [-12, -12, 1]])
    return halfplane_shifts(int(name[4:]))


def _run(x, w, sh, gU, gZ, codes, band=None):
    U, Z = _C.accumulate_uz_forward(x, w, sh, row_codes=codes, band=band)
    gx, gw = _C.accumulate_uz_backward(x, w, gU, gZ, sh, row_codes=codes, band=band)
    return U, Z, gx, gw


# (table, mode, bands n, own rows Hb, width W)
CASES = [
    ("half6", "reference", 4, 64, 256),     # scatter path (128 x 32 tiles)
    ("half6", "circular", 4, 64, 256),
    ("half6", "forward box", 4, 64, 256),
    ("far12", "reference", 3, 48, 256),     # radius 12: gather form inside the launch
    ("half10", "reference", 4, 236, 4096),  # 16-pixel tile border (NSH_WIDE_HALO)
    ("half2", "reference", 4, 16, 40),      # bands on the gather kernels
]


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("table,mode,n,Hb,W", CASES)
def test_gpu_band_split(table, mode, n, Hb, W):
    sh = _table(table)
    R = int(sh[:, :2].abs().max())
    H = n * Hb
    S = sh.size(0)
    codes = mode != "reference"
    if mode == "circular":
        sh = sh.clone()
        sh[:, 2] *= 2            # row code 2: circular mirror
    elif mode == "forward box":
        sh = sh.clone()
        sh[:, 2] = sh[:, 2] | 4  # row codes 1 | 4 and 0 | 4: the box in the kernels
    x = synthetic_image(1, 1, H, W, seed=7).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(8)
    w = torch.nn.functional.softplus(torch.randn(S, 1, H, W, generator=g, device=DEV))
    w = w * torch.where(torch.rand(S, 1, H, W, generator=g, device=DEV) < 0.5, -1.0, 1.0)
    if mode == "reference":
        w = w * box_stack(sh, 1, H, W, device=DEV)
    gU = torch.randn(1, 1, H, W, generator=g, device=DEV)
    gZ = torch.randn(1, 1, H, W, generator=g, device=DEV)
    shd = sh.to(DEV)
    _case(f"band split {table} {mode}: whole image 1x1x{H}x{W}, S={S}, R={R}")
    full = _run(x, w, shd, gU, gZ, codes)
    scale = _run(x.abs(), w.abs(), shd, gU.abs(), gZ.abs(), codes)
    rt = 2 * rtol_for(torch.float32)
    for b in range(n):
        rows = (torch.arange(b * Hb - R, (b + 1) * Hb + R, device=DEV) % H)
        _case(f"band split {table} {mode}: band {b}, image rows {b * Hb}..{(b + 1) * Hb - 1} "
              f"padded to {rows.numel()}, row_origin {b * Hb - R}")
        band = (b * Hb - R, H)
        out = _run(x[:, :, rows].contiguous(), w[:, :, rows].contiguous(), shd,
                   gU[:, :, rows].contiguous(), gZ[:, :, rows].contiguous(), codes, band)
        keep = slice(R, R + Hb)
        mine = slice(b * Hb, (b + 1) * Hb)
        for name, a, e, s in zip(("U", "Z", "grad_x", "grad_w"), out, full, scale):
            assert_bound(a[:, :, keep], e[:, :, mine].double(), s[:, :, mine], rt,
                         f"band {b} {name}")
        del out
    torch.cuda.empty_cache()


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
def test_gpu_band_whole_image_is_plain_call():
    """row_origin 0 and image_height H is the plain call, bit for bit."""
    _case("band call with the whole image")
    sh = halfplane_shifts(4).to(DEV)
    H, W = 136, 264
    x = synthetic_image(1, 1, H, W, seed=3).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(4)
    w = torch.rand(sh.size(0), 1, H, W, generator=g, device=DEV) * \
        box_stack(sh.cpu(), 1, H, W, device=DEV)
    gU = torch.randn(1, 1, H, W, generator=g, device=DEV)
    gZ = torch.randn(1, 1, H, W, generator=g, device=DEV)
    a = _run(x, w, sh, gU, gZ, False)
    b = _run(x, w, sh, gU, gZ, False, (0, H))
    for u, v in zip(a, b):
        assert torch.equal(u, v)
