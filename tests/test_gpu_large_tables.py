"""The top of the reference's table-size contract on the GPU.

The reference accepts any shift table with 1 <= S <= 1024 rows
(csrc/shift_ops.cpp:178-179, shift_ops_cuda.cu:43-49): a half-plane up to
R = 22 (S = 1013) or a full window up to R = 15 (S = 961).  Radii above the
8-pixel LDS halo take other code paths in every kernel (the shifts beyond
the halo read their operands from L2, and the tile's staged shift table
grows to 16 KB of LDS), so every op is checked here, forward and backward,
against the CPU oracle at three tables:

* half22: the R = 22 half-plane, 1013 rows, mirror terms on 1012 of them;
* win15: the R = 15 full window, 961 rows, no mirror terms;
* s1024: half22 plus 11 rows out to |dx| = 199 and |dy| = 295 (mirrored
  and not), exactly S = 1024;

on 200 x 296 images (two channels; several tiles per direction with ragged
last tiles) in fp32 and fp64, at the same tolerances as every other parity
test (helpers.assert_bound: 1e-5 of the per-element term scale for fp32
accumulation, 1e-12 for fp64; gathers bit-exact).
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import (assert_bound, metropolis_grad_abs, metropolis_torch_ordered,
                     normalized_bwd_cond, rtol_for)
from neural_shift_cuda import (accumulate_uz, accumulate_uz_scalar, metropolis_aggregate,
                               normalized_accumulate_uz, pair_gather, shift_gather)
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import box_stack, halfplane_shifts, window_shifts

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEV = torch.device("cuda:0")
SHAPE = (1, 2, 200, 296)
DTYPES = [torch.float32, torch.float64]
TABLES = ["half22", "win15", "s1024"]
FAR_ROWS = [(31, -7, 1), (-45, 3, 1), (0, 40, 1), (25, 25, 0), (-60, -90, 1), (100, 1, 1),
            (7, 150, 1), (-199, 0, 1), (3, -295, 1), (50, 50, 1), (1, 23, 0)]


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()
    yield
    torch.cuda.empty_cache()


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _table(name):
    if name == "half22":
        t = halfplane_shifts(22)
    elif name == "win15":
        t = window_shifts(15)
    else:
        t = torch.cat([halfplane_shifts(22), torch.tensor(FAR_ROWS, dtype=torch.int64)])
    assert t.size(0) == {"half22": 1013, "win15": 961, "s1024": 1024}[name]
    return t


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("table", TABLES)
def test_accumulate_uz_large_table(table, dtype):
    _case(f"accumulate_uz {table} {dtype}")
    B, C, H, W = SHAPE
    sh = _table(table)
    S = sh.size(0)
    g = torch.Generator().manual_seed(1001)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = torch.nn.functional.softplus(torch.randn(S * B, C, H, W, generator=g))
    w = (w * box_stack(sh, B, H, W)).to(dtype)
    gU = torch.randn(B, C, H, W, generator=g).to(dtype)
    gZ = torch.randn(B, C, H, W, generator=g).to(dtype)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    del Uo, Zo, Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x")
    assert_bound(wd.grad, gwo, gws, rt, "grad_w")


@pytest.mark.parametrize("log_weights", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("table", TABLES)
def test_normalized_large_table(table, dtype, log_weights):
    _case(f"normalized {table} {dtype} log={log_weights}")
    B, C, H, W = SHAPE
    sh = _table(table)
    S = sh.size(0)
    g = torch.Generator().manual_seed(1002)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    raw = torch.randn(S * B, C, H, W, generator=g)
    w = (2 * raw) if log_weights else raw.exp()
    pick = torch.rand(w.shape, generator=g)
    w = torch.where(pick < 0.1, torch.full_like(w, float("-inf") if log_weights else 0.0), w)
    if log_weights:
        w = torch.where(pick > 0.99, 80.0 * torch.sign(raw), w)  # +-80 outliers
    w = w.to(dtype)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=log_weights,
                                    return_log_degree=True, validate=False)
    gD = torch.randn(B, C, H, W, generator=g).to(D.dtype)
    gL = torch.randn(B, C, H, W, generator=g).to(D.dtype)
    torch.autograd.backward([D, L], [gD.to(DEV), gL.to(DEV)])
    rt = rtol_for(dtype)
    Do, Lo = oracle.normalized(x, w, sh, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), w, sh, log_weights=log_weights, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
    gxo, gwo = oracle.normalized_bwd(x, w, Do, Lo, gD, gL, sh, log_weights=log_weights)
    gxs, gws = oracle.normalized_bwd(x.abs(), w, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=log_weights)
    gxc, gwc = normalized_bwd_cond(x, w, Lo, gD, gL, Ds, sh, log_weights=log_weights,
                                   acc_dtype=dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", extra=gxc)
    assert_bound(wd.grad, gwo, gws, rt, "grad_w", extra=gwc)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("table", TABLES)
def test_gathers_large_table(table, dtype):
    _case(f"gathers {table} {dtype}")
    B, C, H, W = SHAPE
    sh = _table(table)
    g = torch.Generator().manual_seed(1003)
    guide = torch.randn(B, C, H, W, generator=g).to(dtype)
    for pair in (False, True):
        gd = guide.to(DEV).requires_grad_(True)
        out, mask = (pair_gather if pair else shift_gather)(gd, sh.to(DEV))
        eo, em = (oracle.pair_gather if pair else oracle.shift_gather)(guide, sh)
        assert torch.equal(out.detach().cpu(), eo), f"pair={pair}: stack not bit-exact"
        assert torch.equal(mask.cpu(), em), f"pair={pair}: mask not bit-exact"
        del eo, em
        gout = torch.randn(out.shape, generator=g).to(dtype)
        out.backward(gout.to(DEV))
        bw = oracle.pair_gather_bwd if pair else oracle.shift_gather_bwd
        ref = bw(gout, sh, B, C, H, W)
        scale = bw(gout.abs(), sh, B, C, H, W)
        assert_bound(gd.grad, ref, scale, rtol_for(dtype), f"grad guide pair={pair}")
        del out, mask, gout, gd


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("table", TABLES)
def test_scalar_large_table(table, dtype):
    _case(f"accumulate_uz_scalar {table} {dtype}")
    B, C, H, W = SHAPE
    sh = _table(table)[:, :2].contiguous()
    S = sh.size(0)
    g = torch.Generator().manual_seed(1004)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = (torch.rand(S, B, C, generator=g) + 0.1).to(dtype)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz_scalar(xd, wd, sh.to(DEV))
    gU = torch.randn(B, C, H, W, generator=g).to(U.dtype)
    gZ = torch.randn(B, C, H, W, generator=g).to(U.dtype)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz_scalar(x, w, sh)
    Us, Zs = oracle.accumulate_uz_scalar(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    gxo, gwo = oracle.accumulate_uz_scalar_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_scalar_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x")
    assert_bound(wd.grad, gwo, gws, rt, "grad_w")


# Metropolis: 104 x 272 keeps three tiles per direction in both forward
# passes (128 x 32 tiles), so the fused backward serves the shape.
M_SHAPE = (1, 1, 104, 272)


@pytest.mark.parametrize("use_box", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("table", TABLES)
def test_metropolis_large_table(table, dtype, use_box):
    _case(f"metropolis {table} {dtype} box={use_box}")
    B, C, H, W = M_SHAPE
    sh = _table(table)
    rows = [(int(dx), int(dy), bool(inv)) for dx, dy, inv in sh.tolist()]
    S = len(rows)
    g = torch.Generator().manual_seed(1005)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, generator=g)).to(dtype)
    img = torch.randn(B, C, H, W, generator=g).to(dtype)
    gWx = torch.randn(B, C, H, W, generator=g).to(dtype)
    gdh = torch.randn(B, C, H, W, generator=g).to(dtype)
    rt = rtol_for(dtype)
    # forward against the C oracle
    with torch.no_grad():
        Wx, dh, deg = _C.metropolis_aggregate_with_degree(wh.to(DEV), img.to(DEV), sh.to(DEV),
                                                          int(use_box), 1e-6)
    Wo, do = oracle.metropolis(wh, img, sh, use_box)
    Ws, _ = oracle.metropolis(wh, img.abs(), sh, use_box)
    scale = Ws.abs() + 2 * img.double().abs() * (1 + do.abs())
    assert_bound(Wx, Wo, scale, rt, "Wx")
    assert_bound(dh, do, do.abs(), rt, "d_hat")
    # backward (fused) against fp64 autograd with the kernel's degree ordering
    assert _C.metropolis_backward_supported(wh.to(DEV))
    w = wh.to(DEV).requires_grad_(True)
    x = img.to(DEV).requires_grad_(True)
    Wg, dg = metropolis_aggregate(w, x, rows, use_box)
    assert type(Wg.grad_fn).__name__.startswith("_MetropolisFusedFn")
    torch.autograd.backward([Wg, dg], [gWx.to(DEV), gdh.to(DEV)])
    wr = wh.double().requires_grad_(True)
    xr = img.double().requires_grad_(True)
    Wr, dr = metropolis_torch_ordered(wr, xr, rows, use_box, deg.double().cpu())
    torch.autograd.backward([Wr, dr], [gWx.double(), gdh.double()])
    sw, sx = metropolis_grad_abs(wh, img, gWx, gdh, rows, use_box)
    assert_bound(w.grad, wr.grad, sw, rt, "grad w_half")
    assert_bound(x.grad, xr.grad, sx, rt, "grad img")
