"""normalized_accumulate_uz on shapes that take the scatter path (every
weight element read once: the forward merges each mirror term into an LDS
window of online-softmax states, the backward scatters the x-gradient term;
window borders go through the workspace and a fix-up kernel), against the
CPU oracle (reference GPU policy), against the library's own gather kernels
(the C ABI called without a workspace), and for bitwise determinism.

The scatter path needs at least 2 tiles per direction (forward tiles of
64 x 32 pixels; fp32 backward 128 x 32, 16-bit backward 64 x 32, fp64
forward 32 x 16, fp64 backward 32 x 32) with edge tiles at least 8 pixels.  The shapes
below have partial edge tiles in both directions and several (b, c)
planes; the tables cover radius 1..8 with inverse rows, full windows,
explicit mirrors, a (0, 0) inverse row, and rows beyond radius 8 (served by
the gather form inside the same kernels).  Weights include masked entries
(0 / -inf), a fully masked row and, for logits, +-80 outliers.

Tolerance (the error-bound rule of tests/helpers.py): rtol 1e-5 of the term
scale for fp32-accumulated inputs, 1e-12 for fp64, plus output rounding of
16-bit gradients; gradients add the per-element term of
helpers.normalized_bwd_cond (the error of exp(l - log C) propagated from the
forward's log C, up to |l - log C| ~ 160 with +-80 logits).
"""
from __future__ import annotations

import ctypes
import sys

import pytest
import torch

import oracle
from helpers import assert_bound, normalized_bwd_cond, out_ulp_for, rtol_for
from neural_shift_cuda import normalized_accumulate_uz
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
        "half6": halfplane_shifts(6),
        "half8": halfplane_shifts(8),
        "win2": window_shifts(2),
        "mirror3": explicit_mirror_shifts(halfplane_shifts(3)),
        "selfinv": torch.tensor([[0, 0, 1], [1, 0, 1], [0, 1, 1], [-1, 2, 0]]),
        "far": torch.tensor([[0, 1, 1], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0],
                             [2, 2, 1], [-12, 0, 0]]),
    }[name]


def _weights(shape, log_weights, g):
    raw = torch.randn(*shape, generator=g)
    w = (2 * raw) if log_weights else raw.exp()
    pick = torch.rand(shape, generator=g)
    w = torch.where(pick < 0.1, torch.full_like(w, float("-inf") if log_weights else 0.0), w)
    if log_weights:
        w = torch.where(pick > 0.99, 80.0 * torch.sign(raw), w)  # +-80 outliers
    w[:, 0, 3, 4] = float("-inf") if log_weights else 0.0      # an empty row
    return w


def _uses_scatter(shape, dtype, S):
    B, C, H, W = shape
    lib = _C._lib
    return (lib.nsh_normalized_workspace_bytes(S, B, C, H, W, _CODE[dtype], 0) > 0
            and lib.nsh_normalized_workspace_bytes(S, B, C, H, W, _CODE[dtype], 1) > 0)


def _gather_path(x, w, sh, log_weights, gD, gL):
    """The library's gather kernels: the C ABI called without a workspace."""
    B, C, H, W = x.shape
    S = sh.size(0)
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    D = torch.empty(x.shape, dtype=acc, device=DEV)
    L = torch.empty_like(D)
    shd = sh.to(DEV).contiguous()
    st = torch.cuda.current_stream().cuda_stream
    lib = _C._lib
    rc = lib.nsh_normalized_accumulate_uz_forward(
        x.data_ptr(), w.data_ptr(), shd.data_ptr(), S, B, C, H, W, _CODE[x.dtype],
        int(log_weights), D.data_ptr(), L.data_ptr(), None, 0, st)
    assert rc == 0, lib.nsh_last_error().decode()
    gx = torch.empty_like(x)
    gw = torch.empty_like(w)
    rc = lib.nsh_normalized_accumulate_uz_backward(
        x.data_ptr(), w.data_ptr(), D.data_ptr(), L.data_ptr(), gD.data_ptr(), gL.data_ptr(),
        shd.data_ptr(), S, B, C, H, W, _CODE[x.dtype], int(log_weights), gx.data_ptr(),
        gw.data_ptr(), None, 0, st)
    assert rc == 0, lib.nsh_last_error().decode()
    return D, L, gx, gw


SHAPES = [
    (torch.float32, (1, 2, 72, 200)),
    (torch.float32, (2, 1, 64, 256)),    # 2 x 2 backward tiles: the window wraps onto the other tile
    (torch.float32, (2, 1, 104, 138)),
    (torch.float16, (2, 1, 104, 136)),
    (torch.bfloat16, (1, 1, 80, 140)),
    (torch.float64, (1, 2, 72, 76)),
]


def _run(dtype, shape, sh, log_weights, seed):
    B, C, H, W = shape
    S = sh.size(0)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = _weights((S * B, C, H, W), log_weights, g).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=log_weights,
                                    return_log_degree=True, validate=False)
    gD = torch.randn(B, C, H, W, generator=g).to(D.dtype)
    gL = torch.randn(B, C, H, W, generator=g).to(D.dtype)
    torch.autograd.backward([D, L], [gD.to(DEV), gL.to(DEV)])
    torch.cuda.synchronize()
    return x, w, gD, gL, D, L, xd.grad, wd.grad


@pytest.mark.parametrize("dtype,shape", SHAPES)
@pytest.mark.parametrize("table", ["half1", "half6", "half8", "win2", "mirror3", "selfinv", "far"])
@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_scatter_vs_oracle(dtype, shape, table, log_weights):
    _case(f"normalized scatter {dtype} {shape} {table} log={log_weights}")
    sh = _table(table)
    assert _uses_scatter(shape, dtype, sh.size(0))
    x, w, gD, gL, D, L, gx, gw = _run(dtype, shape, sh, log_weights, 31)
    rt = rtol_for(dtype)
    Do, Lo = oracle.normalized(x, w, sh, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), w, sh, log_weights=log_weights, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
    gxo, gwo = oracle.normalized_bwd(x, w, Do, Lo, gD, gL, sh, log_weights=log_weights)
    # x[p+s] - D enters each weight gradient: D's own error (<= rtol * Ds)
    # propagates, so the scale takes Ds = sum w|x| / C >= |D| in D's place
    gxs, gws = oracle.normalized_bwd(x.abs(), w, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=log_weights)
    ou = out_ulp_for(dtype)
    gxc, gwc = normalized_bwd_cond(x, w, Lo, gD, gL, Ds, sh, log_weights=log_weights,
                                   acc_dtype=dtype)
    assert_bound(gx, gxo, gxs, rt, "grad_x", ou, extra=gxc)
    assert_bound(gw, gwo, gws, rt, "grad_w", ou, extra=gwc)
    # the gather kernels agree within the sum of both bounds (summation order only)
    Dg, Lg, gxg, gwg = _gather_path(x.to(DEV), w.to(DEV), sh, log_weights, gD.to(DEV),
                                    gL.to(DEV))
    assert_bound(D, Dg.double().cpu(), Ds, 2 * rt, "D vs gather")
    assert_bound(gx, gxg.double().cpu(), gxs, 2 * rt, "grad_x vs gather", 2 * ou, extra=2 * gxc)
    assert_bound(gw, gwg.double().cpu(), gws, 2 * rt, "grad_w vs gather", 2 * ou, extra=2 * gwc)


@pytest.mark.parametrize("table", ["half8", "far"])
@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_fp64_backward_narrow_hint_on_far_tables(monkeypatch, table, log_weights):
    """The 6-pixel border hint (NSH_NARROW_HALO) forced on for tables that
    reach 8 and 12 pixels: the fp64 backward runs on the narrow border
    (32 x 16 tiles), its rows beyond 6 pixels in the gather form of the same
    launch, and matches the oracle as the 8-pixel border does."""
    monkeypatch.setattr(_C, "table_radius", lambda t: 0)
    _case(f"normalized fp64 backward {table} narrow hint forced log={log_weights}")
    dtype, shape = torch.float64, (1, 2, 72, 76)
    sh = _table(table)
    x, w, gD, gL, D, L, gx, gw = _run(dtype, shape, sh, log_weights, 33)
    rt = rtol_for(dtype)
    Do, Lo = oracle.normalized(x, w, sh, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), w, sh, log_weights=log_weights, policy="gpu")
    gxo, gwo = oracle.normalized_bwd(x, w, Do, Lo, gD, gL, sh, log_weights=log_weights)
    gxs, gws = oracle.normalized_bwd(x.abs(), w, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=log_weights)
    gxc, gwc = normalized_bwd_cond(x, w, Lo, gD, gL, Ds, sh, log_weights=log_weights,
                                   acc_dtype=dtype)
    assert_bound(gx, gxo, gxs, rt, "grad_x", 0.0, extra=gxc)
    assert_bound(gw, gwo, gws, rt, "grad_w", 0.0, extra=gwc)


def test_normalized_fp64_backward_narrow_workspace_fallback():
    """The fp64 backward with the 6-pixel border hint and a workspace sized
    without it (smaller than the narrow plan's at this shape) runs the
    8-pixel border; with the hinted size, the narrow one.  Both agree with
    the unhinted call to fp64 summation-order rounding."""
    _case("normalized fp64 backward narrow hint, workspace fallback")
    B, C, H, W = 2, 3, 256, 256
    sh = window_shifts(5)
    S = sh.size(0)
    g = torch.Generator().manual_seed(41)
    x = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(DEV)
    w = torch.randn(S * B, C, H, W, generator=g, dtype=torch.float64).exp().to(DEV)
    lib = _C._lib
    st = torch.cuda.current_stream().cuda_stream
    shd = sh.to(DEV).contiguous()
    D = torch.empty(B, C, H, W, dtype=torch.float64, device=DEV)
    L = torch.empty_like(D)
    nf = lib.nsh_normalized_workspace_bytes(S, B, C, H, W, 4, 0)
    wsf = torch.empty(nf, dtype=torch.uint8, device=DEV)
    rc = lib.nsh_normalized_accumulate_uz_forward(
        x.data_ptr(), w.data_ptr(), shd.data_ptr(), S, B, C, H, W, 4, 0, D.data_ptr(),
        L.data_ptr(), wsf.data_ptr(), nf, st)
    assert rc == 0, lib.nsh_last_error().decode()
    gD = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(DEV)
    gL = torch.randn(B, C, H, W, generator=g, dtype=torch.float64).to(DEV)
    plain = lib.nsh_normalized_workspace_bytes(S, B, C, H, W, 4, 1)
    hinted = lib.nsh_normalized_workspace_bytes(S, B, C, H, W, 4 | 0x1000, 1)
    assert hinted > plain > 0

    def bwd(code, nbytes):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        gx, gw = torch.empty_like(x), torch.empty_like(w)
        rc = lib.nsh_normalized_accumulate_uz_backward(
            x.data_ptr(), w.data_ptr(), D.data_ptr(), L.data_ptr(), gD.data_ptr(),
            gL.data_ptr(), shd.data_ptr(), S, B, C, H, W, code, 0, gx.data_ptr(),
            gw.data_ptr(), ws.data_ptr(), nbytes, st)
        assert rc == 0, lib.nsh_last_error().decode()
        torch.cuda.synchronize()
        return gx.cpu(), gw.cpu()

    ref = bwd(4, plain)
    for got in (bwd(4 | 0x1000, plain), bwd(4 | 0x1000, hinted)):
        for a, b in zip(got, ref):
            assert torch.allclose(a, b, rtol=1e-12, atol=1e-12 * b.abs().max().item())


def test_normalized_scatter_deterministic():
    _case("normalized scatter determinism")
    sh = _table("half6")
    first = _run(torch.float32, (1, 2, 72, 200), sh, True, 5)[4:]
    second = _run(torch.float32, (1, 2, 72, 200), sh, True, 5)[4:]
    for a, b in zip(first, second):
        assert torch.equal(a.nan_to_num(), b.nan_to_num())


@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_scatter_bad_keys(log_weights):
    """Bad keys on the scatter path: +inf or NaN logits (log mode), negative,
    +inf or NaN weights (positive mode) make exactly the pixels whose rows
    hold them NaN in D and log C, through the forward term and the mirror
    term alike (reference GPU policy); every other pixel matches the
    oracle."""
    _case(f"normalized scatter bad keys log={log_weights}")
    from neural_shift_cuda import normalized_accumulate_uz
    shape = (1, 2, 72, 200)
    sh = _table("half6")
    S = sh.size(0)
    B, C, H, W = shape
    assert _uses_scatter(shape, torch.float32, S)
    g = torch.Generator().manual_seed(47)
    x = torch.randn(*shape, generator=g)
    w = _weights((S * B, C, H, W), log_weights, g)
    bad = [float("inf"), float("nan")] if log_weights else [-1.0, float("inf"), float("nan")]
    n = 40
    planes = torch.randint(0, S * B, (n,), generator=g)
    chans = torch.randint(0, C, (n,), generator=g)
    hs = torch.randint(0, H, (n,), generator=g)
    ws_ = torch.randint(0, W, (n,), generator=g)
    for i in range(n):
        w[planes[i], chans[i], hs[i], ws_[i]] = bad[i % len(bad)]
    D, L = normalized_accumulate_uz(x.to(DEV), w.to(DEV), sh.to(DEV), log_weights=log_weights,
                                    validate=False, return_log_degree=True)
    D, L = D.double().cpu(), L.double().cpu()
    Do, Lo = oracle.normalized(x, w, sh, log_weights=log_weights, policy="gpu")
    assert torch.isnan(Do).any()
    assert torch.equal(torch.isnan(D), torch.isnan(Do))
    assert torch.equal(torch.isnan(L), torch.isnan(Lo))
    ok = ~torch.isnan(Do)
    Ds, _ = oracle.normalized(x.abs(), w, sh, log_weights=log_weights, policy="gpu")
    rt = rtol_for(torch.float32)
    assert_bound(D[ok], Do[ok], Ds[ok], rt, "D")
    assert_bound(L[ok], Lo[ok], Lo[ok].abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
