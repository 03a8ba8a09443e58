"""metropolis_aggregate on shapes that take the scatter path (each pass reads
every w_half element once; an edge's weight is formed once and added at both
ends, the far end through an LDS window whose border a fix-up adds back),
against the CPU oracle, against the library's own gather kernels (the C ABI
called without a workspace), for exact symmetry of W across tile borders
and image wrap-around, and for bitwise determinism.

The scatter path needs, for both passes' tiles (128 x 32 pixels for
fp32-class types, 32 x 32 for fp64), at least 3 tiles per direction with
edge tiles at least 8 pixels.  The shapes below
have partial edge tiles in both directions (one with W not a multiple of 4)
and several (b, c) planes; the tables cover radius 1..8 with inverse rows,
explicit mirrors (no inverse rows), a (0, 0) inverse row (window radius 0),
and rows beyond radius 8
(served by the gather form inside the same kernels).  Tolerance: the
error-bound rule, rtol 1e-5 (fp16/fp32 inputs, fp32 accumulation) or 1e-12
(fp64), plus output rounding for fp16.
"""
from __future__ import annotations

import ctypes
import sys

import pytest
import torch

import oracle
from helpers import assert_bound, out_ulp_for, rtol_for
from neural_shift_cuda import metropolis_aggregate
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import explicit_mirror_shifts, halfplane_shifts, window_shifts

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
        "half1": halfplane_shifts(1),
        "half3": halfplane_shifts(3),
        "half6": halfplane_shifts(6),
        "half8": halfplane_shifts(8),
        "mirror3": explicit_mirror_shifts(halfplane_shifts(3)),
        "win2": window_shifts(2),
        "far": torch.tensor([[0, 1, 1], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0],
                             [2, 2, 1], [-12, 0, 0]]),
        "selfinv": torch.tensor([[0, 0, 1], [1, 0, 1], [0, 1, 1], [-1, 2, 0]]),
    }[name]


def _inputs(B, C, H, W, sh, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    S = sh.size(0)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, generator=g)).to(dtype)
    img = torch.randn(B, C, H, W, generator=g).to(dtype)
    return wh, img


def _shift_list(sh):
    return [(dx, dy, bool(inv)) for dx, dy, inv in sh.tolist()]


def _gather_path(wh, img, sh, use_box, eps=1e-6):
    """The library's gather kernels: the C ABI called without a workspace."""
    B, S, C, H, W = wh.shape
    Wx = torch.empty_like(img)
    dh = torch.empty_like(img)
    acc = torch.float64 if img.dtype == torch.float64 else torch.float32
    deg = torch.empty(img.shape, dtype=acc, device=img.device)
    shd = sh.to(img.device).contiguous()
    rc = _C._lib.nsh_metropolis_aggregate(
        wh.data_ptr(), img.data_ptr(), shd.data_ptr(), B, S, C, H, W, _CODE[img.dtype],
        int(use_box), ctypes.c_double(eps), Wx.data_ptr(), dh.data_ptr(), deg.data_ptr(), None,
        0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _C._lib.nsh_last_error().decode()
    return Wx, dh


def _uses_scatter(shape, dtype, S):
    B, C, H, W = shape
    return _C._lib.nsh_metropolis_workspace_bytes(B, S, C, H, W, _CODE[dtype]) > 0


SHAPES = [
    (torch.float32, (1, 2, 200, 264)),
    (torch.float32, (1, 1, 200, 266)),
    (torch.float32, (2, 1, 104, 392)),
    (torch.float16, (1, 1, 136, 264)),
    (torch.float64, (1, 2, 136, 104)),
]


@pytest.mark.parametrize("dtype,shape", SHAPES)
@pytest.mark.parametrize("table", ["half1", "half6", "half8", "mirror3", "far", "selfinv"])
@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_scatter_vs_oracle(dtype, shape, table, use_box):
    _case(f"metropolis scatter {dtype} {shape} {table} box={use_box}")
    sh = _table(table)
    assert _uses_scatter(shape, dtype, sh.size(0))
    B, C, H, W = shape
    wh, img = _inputs(B, C, H, W, sh, dtype, 71)
    with torch.no_grad():
        Wx, dh = metropolis_aggregate(wh.to(DEV), img.to(DEV), _shift_list(sh), use_box)
    Wo, do = oracle.metropolis(wh, img, sh, use_box)
    Ws, _ = oracle.metropolis(wh, img.abs(), sh, use_box)
    scale = Ws.abs() + 2 * img.double().abs() * (1 + do.abs())
    rt, ou = rtol_for(dtype), out_ulp_for(dtype)
    assert_bound(Wx, Wo, scale, rt, "Wx", ou)
    assert_bound(dh, do, do.abs(), rt, "d_hat", ou)
    # the gather kernels agree within the same bound (summation order only)
    Wg, dg = _gather_path(wh.to(DEV), img.to(DEV), sh, use_box)
    assert_bound(Wx, Wg.double().cpu(), scale, 2 * rt, "Wx vs gather", 2 * ou)
    assert_bound(dh, dg.double().cpu(), do.abs(), 2 * rt, "d_hat vs gather", 2 * ou)


def test_metropolis_scatter_window_table():
    """A full window without inverse rows (R = 0: no LDS window, no fix-up)."""
    _case("metropolis scatter win2")
    sh = _table("win2")
    B, C, H, W = 1, 1, 200, 264
    wh, img = _inputs(B, C, H, W, sh, torch.float32, 72)
    with torch.no_grad():
        Wx, dh = metropolis_aggregate(wh.to(DEV), img.to(DEV), _shift_list(sh), True)
    Wo, do = oracle.metropolis(wh, img, sh, True)
    Ws, _ = oracle.metropolis(wh, img.abs(), sh, True)
    scale = Ws.abs() + 2 * img.double().abs() * (1 + do.abs())
    assert_bound(Wx, Wo, scale, 1e-5, "Wx")
    assert_bound(dh, do, do.abs(), 1e-5, "d_hat")


@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_scatter_exact_symmetry(use_box):
    """(W e_j)_i == (W e_i)_j bitwise, for neighbour pairs inside a tile,
    across tile borders in both directions, and across the image edges
    (wrap-around edges exist only without the box)."""
    _case(f"metropolis scatter symmetry box={use_box}")
    sh = halfplane_shifts(3)
    B, C, H, W = 1, 1, 200, 264
    wh, _ = _inputs(B, C, H, W, sh, torch.float32, 73)
    wh = wh.to(DEV)
    pairs = [((10, 10), (12, 11)), ((63, 30), (65, 32)), ((31, 63), (33, 64)),
             ((10, 127), (12, 129)), ((31, 126), (32, 131)),
             ((64, 64), (61, 66)), ((0, 0), (2, 263)), ((199, 5), (1, 3)),
             ((199, 263), (0, 0)), ((100, 255), (100, 257))]
    with torch.no_grad():
        for i, j in pairs:
            ei = torch.zeros(B, C, H, W, device=DEV)
            ej = torch.zeros(B, C, H, W, device=DEV)
            ei[0, 0, i[0], i[1]] = 1
            ej[0, 0, j[0], j[1]] = 1
            Wej, _ = metropolis_aggregate(wh, ej, _shift_list(sh), use_box)
            Wei, _ = metropolis_aggregate(wh, ei, _shift_list(sh), use_box)
            a = Wej[0, 0, i[0], i[1]].item()
            b = Wei[0, 0, j[0], j[1]].item()
            assert a == b, f"W not symmetric at {i},{j}: {a} vs {b}"


def test_metropolis_scatter_deterministic():
    _case("metropolis scatter determinism")
    sh = halfplane_shifts(6)
    B, C, H, W = 1, 2, 200, 264
    wh, img = _inputs(B, C, H, W, sh, torch.float32, 74)
    wh, img = wh.to(DEV), img.to(DEV)
    with torch.no_grad():
        a = metropolis_aggregate(wh, img, _shift_list(sh), False)
        b = metropolis_aggregate(wh, img, _shift_list(sh), False)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
