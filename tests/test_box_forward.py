"""Forward box applied inside the kernels (``box_forward=True``; bit 4 of the
table's third column).

The reference's callers multiply every weight plane by its shift's box
(1 where (h + dx, w + dy) lies inside the image) before accumulate_uz /
normalized_accumulate_uz (nekde_drunet_attn_patch.py:337-345).  With
box_forward the kernels apply that mask to the forward term as they read
the weights.  Pinned against the C oracle run on pre-masked weights: values
must agree (same error-bound rule as the other accumulation tests), the
x-gradient too, and the weight gradient is the oracle's times the box (a
dropped weight has no gradient).  The CPU paths are checked the same way in
fp64.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, normalized_bwd_cond, out_ulp_for, rtol_for
from neural_shift_cuda import accumulate_uz, normalized_accumulate_uz
from neural_shift_cuda_amd.workloads import box_stack, halfplane_shifts, window_shifts

HAS_GPU = torch.cuda.is_available()
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()


def _table(name):
    return {
        "half2": halfplane_shifts(2),
        "half6": halfplane_shifts(6),
        "win2": window_shifts(2),
        "far": torch.tensor([[0, 0, 0], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0]]),
    }[name]


def _inputs(B, C, H, W, S, dtype, seed, log_weights=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    if log_weights is None:
        w = torch.randn(S * B, C, H, W, generator=g)
    elif log_weights:
        w = 2 * torch.randn(S * B, C, H, W, generator=g)
    else:
        w = torch.nn.functional.softplus(torch.randn(S * B, C, H, W, generator=g))
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    g1 = torch.randn(B, C, H, W, generator=g).to(acc)
    g2 = torch.randn(B, C, H, W, generator=g).to(acc)
    return x, w.to(dtype), g1, g2


def _premask(w, sh, B, H, W, log_weights):
    box = box_stack(sh, B, H, W).to(w.dtype)
    if log_weights:
        return torch.where(box > 0, w, torch.full_like(w, -float("inf"))), box
    return w * box, box


@pytest.mark.parametrize("table", ["half2", "win2", "far"])
def test_cpu_box_forward_matches_premasked(table):
    sh = _table(table)
    B, C, H, W = 2, 2, 11, 13
    x, w, gU, gZ = _inputs(B, C, H, W, sh.size(0), torch.float64, 5)
    wm, box = _premask(w, sh, B, H, W, False)
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    U, Z = accumulate_uz(xr, wr, sh, box_forward=True)
    torch.autograd.backward([U, Z], [gU, gZ])
    xe, we = x.clone().requires_grad_(True), wm.clone().requires_grad_(True)
    Ue, Ze = accumulate_uz(xe, we, sh)
    torch.autograd.backward([Ue, Ze], [gU, gZ])
    torch.testing.assert_close(U, Ue, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(Z, Ze, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(xr.grad, xe.grad, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(wr.grad, we.grad * box, rtol=1e-12, atol=1e-12)
    assert not torch.allclose(accumulate_uz(x, w, sh)[0], Ue.detach())
    for log_weights in (False, True):
        _, wn, _, _ = _inputs(B, C, H, W, sh.size(0), torch.float64, 6, log_weights)
        wnm, _ = _premask(wn, sh, B, H, W, log_weights)
        D, L = normalized_accumulate_uz(x, wn, sh, log_weights=log_weights,
                                        return_log_degree=True, box_forward=True)
        De, Le = normalized_accumulate_uz(x, wnm, sh, log_weights=log_weights,
                                          return_log_degree=True)
        torch.testing.assert_close(D, De, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(L, Le, rtol=1e-12, atol=1e-12)
    # with the forward box, a circular mirror is the reference's one
    U2, _ = accumulate_uz(x, w, sh, box_forward=True, periodic_inverse=True)
    torch.testing.assert_close(U2, Ue.detach(), rtol=1e-12, atol=1e-12)


SHAPES = [
    (torch.float32, (1, 2, 1033, 1036)),   # scatter path
    (torch.float64, (1, 1, 1033, 1034)),   # scatter path, fp64 tiles
    (torch.float16, (2, 1, 136, 264)),     # scatter path, 16-bit
    (torch.float32, (1, 1, 40, 52)),       # gather kernels
]


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("dtype,shape", SHAPES)
@pytest.mark.parametrize("table", ["half6", "win2", "far"])
def test_gpu_accumulate_box_forward_vs_oracle(dtype, shape, table):
    _case(f"accumulate box_forward {dtype} {shape} {table}")
    sh = _table(table)
    B, C, H, W = shape
    x, w, gU, gZ = _inputs(B, C, H, W, sh.size(0), dtype, 31)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV), box_forward=True)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    torch.cuda.synchronize()
    wm, box = _premask(w, sh, B, H, W, False)
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz(x, wm, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), wm.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    del Uo, Zo, Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, wm, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), wm.abs(), gU.abs(), gZ.abs(), sh)
    ou = out_ulp_for(dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou)
    bx = box.double()
    assert_bound(wd.grad, gwo * bx, gws * bx, rt, "grad_w", ou)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("dtype,shape", [(torch.float32, (1, 2, 72, 200)),
                                         (torch.float64, (1, 1, 104, 104)),
                                         (torch.float32, (1, 1, 30, 44))])
@pytest.mark.parametrize("table", ["half6", "far"])
@pytest.mark.parametrize("log_weights", [False, True])
def test_gpu_normalized_box_forward_vs_oracle(dtype, shape, table, log_weights):
    _case(f"normalized box_forward {dtype} {shape} {table} log={log_weights}")
    sh = _table(table)
    B, C, H, W = shape
    x, w, gD, gL = _inputs(B, C, H, W, sh.size(0), dtype, 32, log_weights)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=log_weights,
                                    return_log_degree=True, validate=False, box_forward=True)
    torch.autograd.backward([D, L], [gD.to(D.dtype).to(DEV), gL.to(D.dtype).to(DEV)])
    torch.cuda.synchronize()
    wm, box = _premask(w, sh, B, H, W, log_weights)
    rt = rtol_for(dtype)
    Do, Lo = oracle.normalized(x, wm, sh, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), wm, sh, log_weights=log_weights, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
    gxo, gwo = oracle.normalized_bwd(x, wm, Do, Lo, gD, gL, sh, log_weights=log_weights)
    gxs, gws = oracle.normalized_bwd(x.abs(), wm, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=log_weights)
    ou = out_ulp_for(dtype)
    gxc, gwc = normalized_bwd_cond(x, wm, Lo, gD, gL, Ds, sh, log_weights=log_weights,
                                   acc_dtype=dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou, extra=gxc)
    bx = box.double()
    assert_bound(wd.grad, gwo * bx, gws * bx, rt, "grad_w", ou, extra=gwc * bx)
