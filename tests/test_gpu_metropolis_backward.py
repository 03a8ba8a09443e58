"""Fused Metropolis backward (``_C.metropolis_aggregate_backward``, reached
through ``metropolis_aggregate`` with autograd on a GPU shape it serves).

Pins, each independent of the HIP backward:

* torch autograd in fp64 on the CPU through ``metropolis_aggregate_torch``,
  the direct statement of the operator (its forward is checked against the
  C oracle by the CPU suite), including torch.maximum's even split on ties
  (the (0, 0) self edge of the "selfinv" table ties on every pixel);
* the gradients of the reference's own differentiable path
  (``metropolis_aggregate_fused``, metropolis.py:117-192) run on this
  library's GPU ops under autograd;
* central differences of the fused GPU forward in fp64 along a random
  direction (the forward itself is pinned against the oracle).

Tolerance: every gradient element is a sum of edge terms, so the bound is
rtol * (|ref| + scale) with the per-element scale from
helpers.metropolis_grad_abs (the same gradient expressions evaluated with
the absolute value of every factor and contribution), rtol 1e-5 for fp32
accumulation (fp16, bf16 and fp32 inputs) and 1e-12 for fp64, plus the
output's own rounding for fp16/bf16.  No element is left out.

Degree ordering: d(loss)/d(max(d_q, d_j)) goes wholly to the larger degree,
so where two degrees are closer than their rounding a kernel that compares
its own degrees can give an edge's term to the other end than an exact
evaluation would.  The fp64 reference is therefore the operator with every
edge's max routed by the kernel's own degree (returned by its forward,
helpers.metropolis_torch_ordered): the values are the exact fp64 ones, the
ordering is the kernel's, and where the orderings agree (all but a few
edges per 10^4) it is the plain operator.  Its gradients equal plain
autograd's when the ordering is the fp64 degree's own
(tests/test_oracle.py pins that on the CPU).

16-bit inputs: grad img = grad_Wx (1 - d_hat) + ... reads the forward's
d_hat, which the reference's autograd holds rounded to the input dtype (as
the fused backward does): that moves each element by up to half an ulp of
d_hat times |grad_Wx|, an `extra` term of |grad_Wx| |d_hat| 2^-11 (fp16) or
2^-8 (bf16) per element (out_ulp_for gives twice that).
"""
from __future__ import annotations

import sys

import pytest
import torch

from helpers import (assert_bound, metropolis_grad_abs, metropolis_torch_ordered, out_ulp_for,
                     rtol_for)
from neural_shift_cuda import metropolis as metro
from neural_shift_cuda import metropolis_aggregate
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import explicit_mirror_shifts, halfplane_shifts, window_shifts

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _table(name):
    t = {
        "half1": halfplane_shifts(1),
        "half3": halfplane_shifts(3),
        "half8": halfplane_shifts(8),
        "mirror3": explicit_mirror_shifts(halfplane_shifts(3)),
        "win2": window_shifts(2),
        "far": torch.tensor([[0, 1, 1], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0],
                             [2, 2, 1], [-12, 0, 0]]),
        "selfinv": torch.tensor([[0, 0, 1], [1, 0, 1], [0, 1, 1], [-1, 2, 0]]),
    }[name]
    return [(int(dx), int(dy), bool(inv)) for dx, dy, inv in t.tolist()]


def _inputs(B, C, H, W, S, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, generator=g)).to(dtype)
    img = torch.randn(B, C, H, W, generator=g).to(dtype)
    gWx = torch.randn(B, C, H, W, generator=g).to(dtype)
    gdh = torch.randn(B, C, H, W, generator=g).to(dtype)
    return wh, img, gWx, gdh


def _grads_gpu(wh, img, gWx, gdh, shifts, use_box, fn=None):
    w = wh.to(DEV).requires_grad_(True)
    x = img.to(DEV).requires_grad_(True)
    if fn is None:
        Wx, dh = metropolis_aggregate(w, x, shifts, use_box)
        assert type(Wx.grad_fn).__name__.startswith("_MetropolisFusedFn"), type(Wx.grad_fn)
    else:
        Wx, dh = fn(w, x, shifts, use_box)
    torch.autograd.backward([Wx, dh], [gWx.to(DEV), gdh.to(DEV)])
    return w.grad, x.grad


def _kernel_degree(wh, img, shifts, use_box):
    """The degree d = K e as the kernel's forward computes it (accumulator
    dtype), which orders the degrees in its backward."""
    table = torch.tensor([[dx, dy, int(inv)] for dx, dy, inv in shifts], device=DEV)
    with torch.no_grad():
        return _C.metropolis_aggregate_with_degree(wh.to(DEV), img.to(DEV), table, int(use_box),
                                                   1e-6)[2].double().cpu()


def _grads_ref(wh, img, gWx, gdh, shifts, use_box):
    """fp64 autograd on the CPU through the operator with the kernel's own
    degree ordering (see above), and the per-element scales (w_half, img)
    of the same gradients."""
    order = _kernel_degree(wh, img, shifts, use_box)
    w = wh.double().requires_grad_(True)
    x = img.double().requires_grad_(True)
    Wx, dh = metropolis_torch_ordered(w, x, shifts, use_box, order)
    torch.autograd.backward([Wx, dh], [gWx.double(), gdh.double()])
    sw, sx = metropolis_grad_abs(wh, img, gWx, gdh, shifts, use_box)
    return w.grad, x.grad, sw, sx


def _check(got, ref, scale, rtol, what, out_ulp=0.0, extra=None):
    assert_bound(got, ref, scale, rtol, what, out_ulp, extra=extra)


def _degree64(wh, shifts, use_box):
    """d = K e in fp64: every kept edge weight at both of its ends."""
    B, S, C, H, W = wh.shape
    w = wh.double()
    d = torch.zeros(B, C, H, W, dtype=torch.float64)
    for s, (dx, dy, inv) in enumerate(shifts):
        k = metro._box(H, W, dx, dy, torch.float64, "cpu") if use_box else 1.0
        o = w[:, s] * k
        d = d + o + (torch.roll(o, (dx, dy), (-2, -1)) if inv else 0)
    return d


# The odd width (2 * 128 + 9) still gives three forward tiles, with a
# partial last tile column in every pass.
SHAPES = [
    (torch.float32, (1, 2, 104, 200)),
    (torch.float32, (1, 1, 104, 266)),
    (torch.float32, (2, 1, 72, 136)),
    (torch.float32, (1, 1, 104, 265)),
    (torch.float64, (1, 2, 104, 104)),
]


@pytest.mark.parametrize("dtype,shape", SHAPES)
@pytest.mark.parametrize("table", ["half1", "half3", "mirror3", "far", "selfinv"])
@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_backward_vs_autograd(dtype, shape, table, use_box):
    _case(f"metropolis backward {dtype} {shape} {table} box={use_box}")
    shifts = _table(table)
    B, C, H, W = shape
    wh, img, gWx, gdh = _inputs(B, C, H, W, len(shifts), dtype, 81)
    assert _C.metropolis_backward_supported(wh.to(DEV))
    gw, gx = _grads_gpu(wh, img, gWx, gdh, shifts, use_box)
    rw, rx, sw, sx = _grads_ref(wh, img, gWx, gdh, shifts, use_box)
    rt = rtol_for(dtype)
    _check(gw, rw, sw, rt, "grad w_half")
    _check(gx, rx, sx, rt, "grad img")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_metropolis_backward_below_tie_gate(dtype):
    """eps below the clamped tie form's gate (2^-104 fp32, 2^-970 fp64):
    every tile, interior ones included, takes the masked loop and its
    compare-and-select tie split.  The degrees (softplus sums, far above
    eps) and so the operator are those of eps = 1e-6; the "selfinv" table
    ties on every pixel."""
    eps = 1e-33 if dtype == torch.float32 else 1e-300
    for table in ("half3", "selfinv"):
        _case(f"metropolis backward {dtype} {table} eps={eps}")
        shifts = _table(table)
        wh, img, gWx, gdh = _inputs(1, 2, 104, 200, len(shifts), dtype, 85)
        w = wh.to(DEV).requires_grad_(True)
        x = img.to(DEV).requires_grad_(True)
        Wx, dh = metropolis_aggregate(w, x, shifts, True, eps=eps)
        assert type(Wx.grad_fn).__name__.startswith("_MetropolisFusedFn"), type(Wx.grad_fn)
        torch.autograd.backward([Wx, dh], [gWx.to(DEV), gdh.to(DEV)])
        order = _kernel_degree(wh, img, shifts, True)
        wr = wh.double().requires_grad_(True)
        xr = img.double().requires_grad_(True)
        Wr, dr = metropolis_torch_ordered(wr, xr, shifts, True, order, eps=eps)
        torch.autograd.backward([Wr, dr], [gWx.double(), gdh.double()])
        sw, sx = metropolis_grad_abs(wh, img, gWx, gdh, shifts, True, eps=eps)
        rt = rtol_for(dtype)
        _check(w.grad, wr.grad, sw, rt, f"grad w_half {table}")
        _check(x.grad, xr.grad, sx, rt, f"grad img {table}")


def test_metropolis_backward_narrow_hint_on_far_tables(monkeypatch):
    """The 6-pixel border hint (NSH_NARROW_HALO) forced on for tables that
    reach 8 and 12 pixels: the rows beyond the border take the gather form
    in the same launch, so the gradients are those of the plain operator."""
    monkeypatch.setattr(_C, "table_radius", lambda t: 0)
    for table in ("half8", "far"):
        _case(f"metropolis backward fp32 {table} narrow hint forced")
        shifts = _table(table)
        wh, img, gWx, gdh = _inputs(1, 1, 136, 200, len(shifts), torch.float32, 86)
        for use_box in (True, False):
            gw, gx = _grads_gpu(wh, img, gWx, gdh, shifts, use_box)
            rw, rx, sw, sx = _grads_ref(wh, img, gWx, gdh, shifts, use_box)
            _check(gw, rw, sw, 1e-5, f"grad w_half {table} box={use_box}")
            _check(gx, rx, sx, 1e-5, f"grad img {table} box={use_box}")


@pytest.mark.parametrize("table", ["half8", "win2"])
def test_metropolis_backward_wide_tables(table):
    """Radius 8 (the full LDS halo) and a window table without inverse rows."""
    _case(f"metropolis backward fp32 {table}")
    shifts = _table(table)
    wh, img, gWx, gdh = _inputs(1, 1, 136, 200, len(shifts), torch.float32, 82)
    for use_box in (True, False):
        gw, gx = _grads_gpu(wh, img, gWx, gdh, shifts, use_box)
        rw, rx, sw, sx = _grads_ref(wh, img, gWx, gdh, shifts, use_box)
        _check(gw, rw, sw, 1e-5, f"grad w_half box={use_box}")
        _check(gx, rx, sx, 1e-5, f"grad img box={use_box}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_metropolis_backward_half(dtype):
    _case(f"metropolis backward {dtype}")
    shifts = _table("half3")
    wh, img, gWx, gdh = _inputs(1, 2, 104, 200, len(shifts), dtype, 83)
    gw, gx = _grads_gpu(wh, img, gWx, gdh, shifts, True)
    assert gw.dtype == dtype and gx.dtype == dtype
    rw, rx, sw, sx = _grads_ref(wh, img, gWx, gdh, shifts, True)
    ou = out_ulp_for(dtype)
    _check(gw, rw, sw, 1e-5, "grad w_half", ou)
    # the forward's d_hat, rounded to the input dtype, enters grad img
    with torch.no_grad():
        _, dh = metropolis_aggregate(wh.to(DEV), img.to(DEV), shifts, True)
    dh_extra = ou * gWx.double().abs() * dh.double().cpu().abs()
    _check(gx, rx, sx, 1e-5, "grad img", ou, extra=dh_extra)


@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_backward_vs_edge_path(use_box):
    """Same gradients as autograd through the reference's explicit-edge path
    (two accumulate_uz calls and a shift_gather, here on the GPU ops)."""
    _case(f"metropolis backward vs edge path box={use_box}")
    shifts = _table("half3")
    wh, img, gWx, gdh = _inputs(1, 2, 104, 136, len(shifts), torch.float64, 84)
    gw, gx = _grads_gpu(wh, img, gWx, gdh, shifts, use_box)
    ew, ex = _grads_gpu(wh, img, gWx, gdh, shifts, use_box, fn=metro.metropolis_aggregate_fused)
    rw, rx, sw, sx = _grads_ref(wh, img, gWx, gdh, shifts, use_box)
    _check(ew, rw, sw, 1e-12, "edge path grad w_half")
    _check(gw, rw, sw, 1e-12, "grad w_half")
    _check(gx, rx, sx, 1e-12, "grad img")
    _check(gw, ew.double().cpu(), sw, 2e-12, "grad w_half vs edge path")
    _check(gx, ex.double().cpu(), sx, 2e-12, "grad img vs edge path")


def test_metropolis_backward_directional_derivative():
    """<grad, v> equals the central difference of the fused fp64 forward."""
    _case("metropolis backward directional derivative")
    shifts = _table("half3")
    B, C, H, W = 1, 1, 104, 136
    wh, img, gWx, gdh = _inputs(B, C, H, W, len(shifts), torch.float64, 85)
    g = torch.Generator().manual_seed(86)
    vw = torch.randn(wh.shape, generator=g, dtype=torch.float64)
    vx = torch.randn(img.shape, generator=g, dtype=torch.float64)
    for use_box in (True, False):
        gw, gx = _grads_gpu(wh, img, gWx, gdh, shifts, use_box)
        lin = (gw.cpu() * vw).sum().item() + (gx.cpu() * vx).sum().item()

        def f(t):
            with torch.no_grad():
                Wx, dh = metropolis_aggregate((wh + t * vw).to(DEV), (img + t * vx).to(DEV),
                                              shifts, use_box)
            return ((Wx.cpu() * gWx).sum() + (dh.cpu() * gdh).sum()).item()

        # max(d_q, d_j) has kinks: the step is small enough that no edge's
        # degree ordering changes between the two evaluation points
        eps = 1e-7
        dp = _degree64(wh + eps * vw, shifts, use_box)
        dm = _degree64(wh - eps * vw, shifts, use_box)
        for dx, dy, _ in shifts:
            assert torch.equal(torch.sign(dp - torch.roll(dp, (-dx, -dy), (-2, -1))),
                               torch.sign(dm - torch.roll(dm, (-dx, -dy), (-2, -1))))
        fd = (f(eps) - f(-eps)) / (2 * eps)
        assert abs(fd - lin) <= 1e-5 * (abs(lin) + 1.0), (use_box, fd, lin)


def test_metropolis_backward_one_input():
    """Gradient for img only (w_half frozen), and for w_half only."""
    _case("metropolis backward one input")
    shifts = _table("half1")
    wh, img, gWx, gdh = _inputs(1, 1, 104, 200, len(shifts), torch.float32, 87)
    rw, rx, sw, sx = _grads_ref(wh, img, gWx, gdh, shifts, False)
    x = img.to(DEV).requires_grad_(True)
    Wx, dh = metropolis_aggregate(wh.to(DEV), x, shifts, False)
    assert type(Wx.grad_fn).__name__.startswith("_MetropolisFusedFn")
    Wx.backward(gWx.to(DEV))  # d_hat unused: its gradient is zero
    _, rx_only, _, sx_only = _grads_ref(wh, img, gWx, torch.zeros_like(gdh), shifts, False)
    _check(x.grad, rx_only, sx_only, 1e-5, "grad img (Wx only)")
    w = wh.to(DEV).requires_grad_(True)
    Wx, dh = metropolis_aggregate(w, img.to(DEV), shifts, False)
    torch.autograd.backward([Wx, dh], [gWx.to(DEV), gdh.to(DEV)])
    _check(w.grad, rw, sw, 1e-5, "grad w_half (w only)")


def test_metropolis_backward_deterministic():
    _case("metropolis backward determinism")
    shifts = _table("half3")
    wh, img, gWx, gdh = _inputs(1, 2, 104, 200, len(shifts), torch.float32, 88)
    a = _grads_gpu(wh, img, gWx, gdh, shifts, False)
    b = _grads_gpu(wh, img, gWx, gdh, shifts, False)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_metropolis_backward_small_shape_uses_edge_path():
    """Shapes below 3 tiles per direction keep the explicit-edge path."""
    _case("metropolis backward small shape")
    shifts = _table("half1")
    wh, img, gWx, gdh = _inputs(1, 1, 40, 48, len(shifts), torch.float64, 89)
    assert not _C.metropolis_backward_supported(wh.to(DEV))
    table = torch.tensor([[dx, dy, int(inv)] for dx, dy, inv in shifts], device=DEV)
    with pytest.raises(RuntimeError, match="not supported"):
        _C.metropolis_aggregate_backward(
            wh.to(DEV), img.to(DEV), table, 1, 1e-6, torch.zeros_like(img.to(DEV)), img.to(DEV),
            gWx.to(DEV), gdh.to(DEV))
    w = wh.to(DEV).requires_grad_(True)
    Wx, dh = metropolis_aggregate(w, img.to(DEV), shifts, True)
    assert not type(Wx.grad_fn).__name__.startswith("_MetropolisFusedFn")
    torch.autograd.backward([Wx, dh], [gWx.to(DEV), gdh.to(DEV)])
    rw, _, sw, _ = _grads_ref(wh, img, gWx, gdh, shifts, True)
    _check(w.grad, rw, sw, 1e-12, "grad w_half (edge path)")
