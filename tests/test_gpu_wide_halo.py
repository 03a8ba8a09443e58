"""accumulate_uz on the scatter path with a 16- or 24-pixel tile border
(NSH_WIDE_HALO, NSH_WIDER_HALO), against the CPU oracle.

Tables of radius 9..16 reach beyond the 8-pixel border of the default
scatter tiles; the library then stages a 16-pixel border (forward tiles
128 x 32, backward 128 x 16), and for radius 17..24 a 24-pixel border
(64 x 32 tiles in both passes), so that every weight element is still
read once.  The flags are hints that the Python layer sets from the table's
radius (`_C.table_radius`); the kernels check the radius themselves, so a
hint on a table of smaller radius (wide border, narrow table), on one above
the border or above the narrowest tile (the gather form inside the launch)
must give the same results as well.

Shapes: fp32-class types with 4-pixel lanes (the wide tiles), partial edge
tiles exactly 16 pixels wide/high, 2 x 2 tiles per plane (the neighbour on
either side is the same tile), 16-bit types (fp32 gx partials rounded once
by the fix-up), several planes.  Tolerance as for every accumulation: 1e-5
of the per-element term scale (helpers.assert_bound) plus output rounding
for 16-bit gradients.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, out_ulp_for, rtol_for
from neural_shift_cuda import accumulate_uz
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import box_stack, halfplane_shifts, window_shifts

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEV = torch.device("cuda:0")
_CODE = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3, torch.float64: 4}


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()
    yield
    torch.cuda.empty_cache()


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _table(name):
    return {
        "half10": halfplane_shifts(10),
        "win12": window_shifts(12),
        # radius exactly 16 in every direction (corners included), mirrored
        # and not, a (0, 0) mirror row, and some short rows
        "ring16": torch.tensor([[16, 16, 1], [-16, 16, 1], [16, -16, 0], [0, 16, 1], [16, 0, 1],
                                [-16, 0, 0], [3, -5, 1], [0, 0, 1], [9, 12, 1], [-13, 7, 1],
                                [-16, -16, 1], [1, 1, 0]]),
        "half6": halfplane_shifts(6),
        "half18": halfplane_shifts(18),
        # radius exactly 24 (corners included) and 22 (the R = 22 half-plane's
        # reach), mirrored and not, plus short rows
        "ring24": torch.tensor([[24, 24, 1], [-24, 24, 1], [24, -24, 0], [0, 24, 1], [24, 0, 1],
                                [-24, 0, 0], [22, -22, 1], [0, 0, 1], [17, 3, 1], [-5, 19, 1],
                                [-24, -24, 1], [1, 1, 0], [2, -1, 1]]),
        # beyond the 16-pixel border: the gather form inside the launch
        "far20": torch.tensor([[0, 0, 0], [9, 3, 1], [-20, 11, 1], [2, -10, 1], [17, -7, 1]]),
    }[name]


def _inputs(dtype, shape, sh, seed, masked=True):
    B, C, H, W = shape
    S = sh.size(0)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = torch.nn.functional.softplus(torch.randn(S * B, C, H, W, generator=g))
    w = w * torch.where(torch.rand(w.shape, generator=g) < 0.5, -1.0, 1.0)
    if masked:
        w = w * box_stack(sh, B, H, W)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    gU = torch.randn(B, C, H, W, generator=g).to(acc)
    gZ = torch.randn(B, C, H, W, generator=g).to(acc)
    return x, w.to(dtype), gU, gZ


def _raw(dtype, x, w, gU, gZ, sh, flags):
    """Forward and backward through the C ABI with `flags` ORed into the
    dtype code (workspace sized by the same query)."""
    B, C, H, W = x.shape
    S = sh.size(0)
    code = _CODE[dtype] | flags
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    xd, wd, shd = x.to(DEV), w.to(DEV), sh.to(DEV)
    gUd, gZd = gU.to(DEV), gZ.to(DEV)
    U = torch.empty(x.shape, dtype=acc, device=DEV)
    Z = torch.empty_like(U)
    gx = torch.empty_like(xd)
    gw = torch.empty_like(wd)
    st = torch.cuda.current_stream().cuda_stream
    nf = int(_C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, code, 0))
    nb = int(_C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, code, 1))
    assert nf > 0 and nb > 0, "the shape must take the scatter path"
    wsf = torch.empty(nf, dtype=torch.uint8, device=DEV)
    wsb = torch.empty(nb, dtype=torch.uint8, device=DEV)
    assert _C._lib.nsh_accumulate_uz_forward(xd.data_ptr(), wd.data_ptr(), shd.data_ptr(), S, B,
                                             C, H, W, code, U.data_ptr(), Z.data_ptr(),
                                             wsf.data_ptr(), nf, st) == 0
    assert _C._lib.nsh_accumulate_uz_backward(xd.data_ptr(), wd.data_ptr(), gUd.data_ptr(),
                                              gZd.data_ptr(), shd.data_ptr(), S, B, C, H, W,
                                              code, gx.data_ptr(), gw.data_ptr(),
                                              wsb.data_ptr(), nb, st) == 0
    torch.cuda.synchronize()
    return U, Z, gx, gw


def _check(dtype, x, w, gU, gZ, sh, outs):
    U, Z, gx, gw = outs
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    del Uo, Zo, Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    ou = out_ulp_for(dtype)
    assert_bound(gx, gxo, gxs, rt, "grad_x", ou)
    assert_bound(gw, gwo, gws, rt, "grad_w", ou)


def _workspace_grows(dtype, shape, S):
    B, C, H, W = shape
    for bwd in (0, 1):
        n8 = int(_C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, _CODE[dtype], bwd))
        n16 = int(_C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W,
                                                             _CODE[dtype] | _C.NSH_WIDE_HALO,
                                                             bwd))
        assert n16 > n8 > 0, (bwd, n8, n16)


# (dtype, shape): every one takes the 16-pixel-border tiles in both passes,
# with the partial last tiles at least 16 wide and high (a radius above the
# narrowest tile runs the gather form, see the hint test)
SHAPES = [
    (torch.float32, (1, 1, 1040, 1040)),   # last forward tiles exactly 16 x 16
    (torch.float32, (64, 1, 64, 256)),     # 2 x 2 forward tiles (2 x 4 backward)
    (torch.float32, (160, 1, 48, 144)),    # last tiles 16 wide / high in both passes
    (torch.float16, (1, 1, 1072, 4112)),   # fp32 gx partials, one rounding in the fix-up
    (torch.bfloat16, (2, 1, 1040, 1040)),  # forward 4-pixel lanes need 2^21 16-bit pixels
]


@pytest.mark.parametrize("dtype,shape", SHAPES)
def test_wide_halo_radius16(dtype, shape):
    _case(f"wide halo ring16 {dtype} {shape}")
    sh = _table("ring16")
    _workspace_grows(dtype, shape, sh.size(0))
    x, w, gU, gZ = _inputs(dtype, shape, sh, 21)
    _check(dtype, x, w, gU, gZ, sh, _raw(dtype, x, w, gU, gZ, sh, _C.NSH_WIDE_HALO))


# the 24-pixel border: 64 x 32 tiles, so images whose last tiles are at
# least 24 pixels (1056 = 33 x 32)
SHAPES24 = [
    (torch.float32, (1, 1, 1056, 1024)),
    (torch.float32, (96, 1, 96, 128)),     # 2 tiles across, 3 down
    (torch.float16, (2, 1, 1056, 1024)),   # fp32 gx partials, one rounding in the fix-up
    (torch.bfloat16, (2, 1, 1056, 1024)),
]


@pytest.mark.parametrize("dtype,shape", SHAPES24)
def test_wider_halo_radius24(dtype, shape):
    _case(f"wider halo ring24 {dtype} {shape}")
    sh = _table("ring24")
    B, C, H, W = shape
    for bwd in (0, 1):
        n8 = int(_C._lib.nsh_accumulate_uz_workspace_bytes(sh.size(0), B, C, H, W, _CODE[dtype],
                                                            bwd))
        n24 = int(_C._lib.nsh_accumulate_uz_workspace_bytes(
            sh.size(0), B, C, H, W, _CODE[dtype] | _C.NSH_WIDER_HALO, bwd))
        assert n24 > n8 > 0, (bwd, n8, n24)
    x, w, gU, gZ = _inputs(dtype, shape, sh, 25)
    _check(dtype, x, w, gU, gZ, sh, _raw(dtype, x, w, gU, gZ, sh, _C.NSH_WIDER_HALO))


@pytest.mark.parametrize("table", ["half10", "win12", "half18"])
def test_wide_halo_full_tables(table):
    """Whole half-planes (R = 10, 221 rows; R = 18, 685 rows, on the
    24-pixel border) and a full window (R = 12, 625 rows), through the
    package op: the hint comes from the table's radius."""
    _case(f"wide halo {table}")
    sh = _table(table)
    shape = (1, 1, 1056, 1024) if table == "half18" else (1, 1, 1040, 1040)
    x, w, gU, gZ = _inputs(torch.float32, shape, sh, 22, masked=table != "win12")
    shd = sh.to(DEV)
    assert _C._halo_flag(shd) == (_C.NSH_WIDER_HALO if table == "half18" else _C.NSH_WIDE_HALO)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, shd)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    _check(torch.float32, x, w, gU, gZ, sh, (U, Z, xd.grad, wd.grad))


@pytest.mark.parametrize("table,shape,flag", [
    ("half6", (1, 1, 1040, 1040), "wide"),
    ("far20", (1, 1, 1040, 1040), "wide"),
    ("ring16", (1, 1, 1033, 1036), "wide"),
    ("half6", (1, 1, 1056, 1024), "wider"),
    ("ring24", (1, 1, 1040, 1040), "wider"),
    ("ring24", (1, 1, 1056, 1024), "wide"),
])
def test_wide_halo_hint_outside_its_range(table, shape, flag):
    """A hint that does not fit the table: radius 6 on the 16- and 24-pixel
    borders (wide border, narrow table); radius 20 and 24 on the 16-pixel
    border (beyond it); radius 16 on an image whose last tiles are 12 and 9
    pixels and radius 24 on one whose last forward tiles are 16 (narrower
    than the radius).  Those beyond run the gather form inside the launch.
    All exact."""
    _case(f"wide halo hint {flag} on {table} {shape}")
    sh = _table(table)
    dtype = torch.float32
    x, w, gU, gZ = _inputs(dtype, shape, sh, 23, masked=table != "far20")
    f = _C.NSH_WIDE_HALO if flag == "wide" else _C.NSH_WIDER_HALO
    _check(dtype, x, w, gU, gZ, sh, _raw(dtype, x, w, gU, gZ, sh, f))


def test_wide_halo_deterministic_and_matches_gather():
    """Run-twice bitwise determinism on the wide border, and agreement with
    the gather form (no hint: radius 16 is beyond the default border)."""
    _case("wide halo determinism")
    sh = _table("ring16")
    dtype, shape = torch.float32, (1, 1, 1040, 1040)
    x, w, gU, gZ = _inputs(dtype, shape, sh, 24)
    a = _raw(dtype, x, w, gU, gZ, sh, _C.NSH_WIDE_HALO)
    b = _raw(dtype, x, w, gU, gZ, sh, _C.NSH_WIDE_HALO)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    c = _raw(dtype, x, w, gU, gZ, sh, 0)
    assert torch.equal(a[3], c[3])  # grad_w: same terms, same order in both forms
    xa, wa = x.abs(), w.abs()
    Us, Zs = oracle.accumulate_uz(xa, wa, sh)
    gxs, _ = oracle.accumulate_uz_bwd(xa, wa, gU.abs(), gZ.abs(), sh)
    for i, (name, scale) in enumerate((("U", Us), ("Z", Zs), ("grad_x", gxs))):
        assert_bound(a[i], c[i].double(), scale, 2e-5, name)
