"""accumulate_uz on shapes that take the scatter path (every weight element
read once; mirror / x terms scattered through an LDS window whose border is
spilled and added back by a fix-up kernel), against the CPU oracle.

The library picks the path from the shape: a vector width VEC (4 elements,
2 for fp64, narrower when the image has fewer than 2^19 * VEC pixels) and
tiles of 32*VEC x 32 (fp32-class with VEC 4) or 16*VEC x 32 pixels, with
at least 2 tiles per direction and edge tiles at least 8 pixels wide.  The shapes below cover
every vector width of every dtype, partial edge tiles in both directions,
several (b, c) planes, tables of radius 1..8 (box-masked mirrors, full
windows, explicit mirrors) and a table beyond radius 8, which the same
launch serves with the gather algorithm.  Tolerances as elsewhere:
the error-bound rule, rtol 1e-5 of the term scale (fp16/bf16/fp32 inputs,
fp32 accumulation) or 1e-12 (fp64), plus output rounding for 16-bit
gradients.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, out_ulp_for, rtol_for
from neural_shift_cuda import accumulate_uz
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import (box_stack, explicit_mirror_shifts, halfplane_shifts,
                                             window_shifts)

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
        "half2": halfplane_shifts(2),
        "half6": halfplane_shifts(6),
        "half8": halfplane_shifts(8),
        "win2": window_shifts(2),
        "mirror3": explicit_mirror_shifts(halfplane_shifts(3)),
        "far": torch.tensor([[0, 0, 0], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0]]),
        "selfinv": torch.tensor([[0, 0, 1], [1, 0, 1], [0, 1, 1], [-1, 2, 0]]),
    }[name]


# (dtype, shape) pairs: each takes the scatter path with the noted vector width
SCATTER_SHAPES = [
    (torch.float32, (1, 2, 1033, 1036)),   # VEC 4, 128x32 tiles, partial edges
    (torch.float32, (2, 2, 105, 204)),     # VEC 1, 16x32 tiles
    (torch.float64, (1, 1, 1033, 1034)),   # VEC 2, 32x16 tiles
    (torch.float16, (1, 1, 1049, 4104)),   # VEC 4 (fp32 gx partials, one rounding)
    (torch.bfloat16, (1, 1, 1049, 4104)),  # VEC 4
    (torch.float16, (2, 1, 136, 216)),     # VEC 1
    (torch.float32, (32, 1, 256, 256)),    # VEC 4, 128x32 tiles, 2 per row (both passes)
    (torch.float32, (64, 1, 64, 256)),     # VEC 4, 128x32 tiles: 2 tiles in each direction
    (torch.float32, (64, 1, 40, 200)),     # 2 x 2 tiles with partial second tiles (8 rows, 72 cols)
    (torch.float32, (168, 1, 64, 100)),    # VEC 4 on the second-choice 64x32 tiles (64 + 36 cols)
    # 16-bit backward (fp32 gx partials, the rounding fix-up over every
    # pixel) on 2 x 2 tiles of 128 x 32: the left/right and upper/lower
    # neighbours are the same tile
    (torch.float16, (128, 1, 64, 256)),    # backward VEC 4, 128x32 tiles, 2 x 2 per plane
    (torch.bfloat16, (160, 1, 40, 200)),   # backward VEC 4, 2 x 2 with partial second tiles
]


def _uses_workspace(dtype, shape, S, backward):
    B, C, H, W = shape
    return int(_C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, _CODE[dtype],
                                                         int(backward))) > 0


def _run_and_check(dtype, shape, sh, seed, masked=True):
    B, C, H, W = shape
    S = sh.size(0)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = torch.nn.functional.softplus(torch.randn(S * B, C, H, W, generator=g))
    w = w * torch.where(torch.rand(w.shape, generator=g) < 0.5, -1.0, 1.0)
    if masked:
        w = w * box_stack(sh, B, H, W)
    w = w.to(dtype)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    gU = torch.randn(B, C, H, W, generator=g).to(acc)
    gZ = torch.randn(B, C, H, W, generator=g).to(acc)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    torch.cuda.synchronize()
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    del Uo, Zo, Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    ou = out_ulp_for(dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou)
    assert_bound(wd.grad, gwo, gws, rt, "grad_w", ou)
    return U, Z, xd.grad, wd.grad


@pytest.mark.parametrize("dtype,shape", SCATTER_SHAPES)
@pytest.mark.parametrize("table", ["half2", "half6"])
def test_scatter_path_vs_oracle(dtype, shape, table):
    _case(f"scatter {dtype} {shape} {table}")
    sh = _table(table)
    assert _uses_workspace(dtype, shape, sh.size(0), False)
    assert _uses_workspace(dtype, shape, sh.size(0), True)
    _run_and_check(dtype, shape, sh, seed=7)


@pytest.mark.parametrize("table", ["half8", "win2", "mirror3", "far", "selfinv"])
def test_scatter_tables(table):
    """Radius 8 (the window limit), full windows (no mirror rows: the
    forward needs no window, the backward scatters every row), explicit
    mirror rows, a radius beyond the window (gather inside the launch), and
    a (0, 0) inverse row (window radius 0: its mirror term lands on the pixel
    itself)."""
    _case(f"scatter table {table}")
    sh = _table(table)
    masked = table != "far"
    _run_and_check(torch.float32, (2, 1, 1033, 1036), sh, seed=9, masked=masked)


def test_scatter_deterministic():
    _case("scatter determinism")
    sh = _table("half6")
    first = _run_and_check(torch.float32, (1, 1, 1033, 1036), sh, seed=3)
    second = _run_and_check(torch.float32, (1, 1, 1033, 1036), sh, seed=3)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_scatter_matches_gather_path():
    """The same inputs through the scatter launch and through the gather
    kernels (no workspace) agree to the accumulation tolerance."""
    _case("scatter vs gather path")
    B, C, H, W = 1, 1, 1033, 1036
    sh = _table("half6").to(DEV)
    S = sh.size(0)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, C, H, W, generator=g).to(DEV)
    w = (torch.rand(S * B, C, H, W, generator=g) * box_stack(sh.cpu(), B, H, W)).to(DEV)
    gU = torch.randn(B, C, H, W, generator=g).to(DEV)
    gZ = torch.randn(B, C, H, W, generator=g).to(DEV)
    st = torch.cuda.current_stream().cuda_stream
    out = {}
    for name in ("scatter", "gather"):
        U = torch.empty_like(x)
        Z = torch.empty_like(x)
        gx = torch.empty_like(x)
        gw = torch.empty_like(w)
        ws_f = _C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, 3, 0)
        ws_b = _C._lib.nsh_accumulate_uz_workspace_bytes(S, B, C, H, W, 3, 1)
        assert ws_f > 0 and ws_b > 0
        wsf = torch.empty(ws_f, dtype=torch.uint8, device=DEV) if name == "scatter" else None
        wsb = torch.empty(ws_b, dtype=torch.uint8, device=DEV) if name == "scatter" else None
        rc = _C._lib.nsh_accumulate_uz_forward(
            x.data_ptr(), w.data_ptr(), sh.data_ptr(), S, B, C, H, W, 3, U.data_ptr(),
            Z.data_ptr(), wsf.data_ptr() if wsf is not None else None,
            ws_f if wsf is not None else 0, st)
        assert rc == 0
        rc = _C._lib.nsh_accumulate_uz_backward(
            x.data_ptr(), w.data_ptr(), gU.data_ptr(), gZ.data_ptr(), sh.data_ptr(), S, B, C, H,
            W, 3, gx.data_ptr(), gw.data_ptr(), wsb.data_ptr() if wsb is not None else None,
            ws_b if wsb is not None else 0, st)
        assert rc == 0
        torch.cuda.synchronize()
        out[name] = (U, Z, gx, gw)
    # gw is computed identically by both paths
    assert torch.equal(out["scatter"][3], out["gather"][3])
    xa, wa = x.abs().cpu(), w.abs().cpu()
    Us, Zs = oracle.accumulate_uz(xa, wa, sh.cpu())
    gxs, _ = oracle.accumulate_uz_bwd(xa, wa, gU.abs().cpu(), gZ.abs().cpu(), sh.cpu())
    for i, (name, scale) in enumerate((("U", Us), ("Z", Zs), ("gx", gxs))):
        assert_bound(out["scatter"][i], out["gather"][i].double(), scale, 2e-5, name)
