"""The HIP kernels against the golden vectors written by the reference's own
CPU fallbacks (tests/golden/make_golden.py).

Gathers must be bit-exact (values and masks, every dtype, the R = 0
branch).  Accumulations match within the accumulation tolerance of the
error-bound rule (rtol 1e-5 of the term scale for fp16/fp32 inputs, 1e-12
for fp64).  Where the reference CPU fallback yields NaN gradients (a zero
positive weight, an empty row) the GPU kernels give 0, the reference GPU
kernels' rule; the check confirms the NaNs sit exactly there and compares
zeros.  Out-of-contract weights with validate=False follow the reference
GPU rule (NaN for a negative positive-mode weight), so that case is checked
against the oracle's GPU policy instead.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import (assert_bound, golden_cases, golden_names, metropolis_grad_abs,
                     normalized_bwd_cond, out_ulp_for, rtol_for)
from neural_shift_cuda import (accumulate_uz, accumulate_uz_scalar, metropolis_aggregate,
                               normalized_accumulate_uz, pair_gather, shift_gather)

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _dev(t):
    return t.to(DEV)


@pytest.mark.parametrize("name", golden_names("accumulate_uz"))
def test_gpu_accumulate_golden(name):
    _case(f"golden {name}")
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    xr = _dev(I["x"]).requires_grad_(True)
    wr = _dev(I["w"]).requires_grad_(True)
    U, Z = accumulate_uz(xr, wr, _dev(I["shifts"]))
    torch.autograd.backward([U, Z], [_dev(I["gU"]), _dev(I["gZ"])])
    torch.cuda.synchronize()
    Us, Zs = oracle.accumulate_uz(I["x"].abs(), I["w"].abs(), I["shifts"])
    gxs, gws = oracle.accumulate_uz_bwd(I["x"].abs(), I["w"].abs(), I["gU"].abs(),
                                        I["gZ"].abs(), I["shifts"])
    rt = rtol_for(I["x"].dtype)
    ou = out_ulp_for(I["x"].dtype)
    assert U.dtype == O["U"].dtype and xr.grad.dtype == O["gx"].dtype
    assert_bound(U, O["U"], Us, rt, f"{name} U")
    assert_bound(Z, O["Z"], Zs, rt, f"{name} Z")
    assert_bound(xr.grad, O["gx"], gxs, rt, f"{name} gx", ou)
    assert_bound(wr.grad, O["gw"], gws, rt, f"{name} gw", ou)


@pytest.mark.parametrize("name", golden_names("accumulate_uz_scalar"))
def test_gpu_scalar_golden(name):
    _case(f"golden {name}")
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    xr = _dev(I["x"]).requires_grad_(True)
    wr = _dev(I["w"]).requires_grad_(True)
    U, Z = accumulate_uz_scalar(xr, wr, _dev(I["shifts"]))
    torch.autograd.backward([U, Z], [_dev(I["gU"]), _dev(I["gZ"])])
    w3 = I["w"] if I["w"].dim() == 3 else \
        I["w"].unsqueeze(-1).expand(*I["w"].shape, I["x"].shape[1]).contiguous()
    Us, _ = oracle.accumulate_uz_scalar(I["x"].abs(), w3.abs(), I["shifts"])
    gxs, gws = oracle.accumulate_uz_scalar_bwd(I["x"].abs(), w3.abs(), I["gU"].abs(),
                                               I["gZ"].abs(), I["shifts"])
    if I["w"].dim() == 2:
        gws = gws.sum(-1)
    rt = rtol_for(I["x"].dtype)
    assert_bound(U, O["U"], Us, rt, f"{name} U")
    assert_bound(Z, O["Z"], w3.abs().sum(0)[..., None, None].expand_as(Z), rt, f"{name} Z")
    assert_bound(xr.grad, O["gx"], gxs, rt, f"{name} gx")
    assert_bound(wr.grad, O["gw"], gws, rt, f"{name} gw")


@pytest.mark.parametrize("name", golden_names("shift_gather") + golden_names("pair_gather"))
def test_gpu_gathers_golden(name):
    _case(f"golden {name}")
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    fn = shift_gather if c["op"] == "shift_gather" else pair_gather
    g = _dev(I["guide"]).requires_grad_(True)
    out, mask = fn(g, _dev(I["shifts"]))
    assert out.dtype == O["out"].dtype and mask.dtype == O["mask"].dtype
    assert torch.equal(out.detach().cpu(), O["out"]), f"{name}: gather not bit-exact"
    assert torch.equal(mask.cpu(), O["mask"]), f"{name}: mask not bit-exact"
    out.backward(_dev(I["gout"]))
    B, C, H, W = I["guide"].shape
    bwd = oracle.shift_gather_bwd if c["op"] == "shift_gather" else oracle.pair_gather_bwd
    exp = bwd(I["gout"], I["shifts"], B, C, H, W)
    scale = bwd(I["gout"].abs(), I["shifts"], B, C, H, W)
    dt = I["guide"].dtype
    # fp32 accumulation, one rounding to the guide dtype
    assert_bound(g.grad, exp, scale, rtol_for(dt), f"{name} grad", out_ulp_for(dt))
    # and against the reference's own (dtype-precision) autograd sums
    terms = I["shifts"].size(0) + 1
    rt = {torch.bfloat16: terms * 2.0 ** -8, torch.float16: terms * 2.0 ** -11}.get(
        dt, rtol_for(dt))
    assert_bound(g.grad, O["gguide"], scale, rt, f"{name} grad vs golden")


@pytest.mark.parametrize("name", golden_names("normalized_accumulate_uz"))
def test_gpu_normalized_golden(name):
    _case(f"golden {name}")
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    lw = c["log_weights"]
    grads = "gw" in O
    xr = _dev(I["x"]).requires_grad_(grads)
    wr = _dev(I["w"]).requires_grad_(grads)
    out = normalized_accumulate_uz(xr, wr, _dev(I["shifts"]), log_weights=lw,
                                   return_log_degree=True, validate=c["validate"])
    D, L = out
    rt = rtol_for(I["x"].dtype)
    if not c["validate"]:
        # out-of-contract weights: the reference GPU rule (NaN for a negative
        # positive-mode weight), which the oracle's "gpu" policy restates
        Do, Lo = oracle.normalized(I["x"], I["w"], I["shifts"], log_weights=lw, policy="gpu")
        Ds, _ = oracle.normalized(I["x"].abs(), I["w"], I["shifts"], log_weights=lw,
                                  policy="gpu")
        assert_bound(D, Do, Ds.nan_to_num(), rt, f"{name} D")
        assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, f"{name} log_C")
        return
    Ds, _ = oracle.normalized(I["x"].abs(), I["w"], I["shifts"], log_weights=lw, policy="gpu")
    assert_bound(D, O["D"], Ds, rt, f"{name} D")
    if "log_C" in O:
        assert_bound(L, O["log_C"], O["log_C"].abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt,
                     f"{name} log_C")
    if not grads:
        return
    gD = I["gD"]
    gL = I.get("gL", torch.zeros_like(gD))
    torch.autograd.backward([D, L], [_dev(gD), _dev(gL)])
    Lo = O["log_C"] if "log_C" in O else L.detach().cpu()
    gxs, gws = oracle.normalized_bwd(I["x"].abs(), I["w"], -Ds, Lo, gD.abs(), gL.abs(),
                                     I["shifts"], log_weights=lw)
    gx_ref, gw_ref = O["gx"], O["gw"]
    empty = torch.isneginf(Lo)
    assert torch.equal(torch.isnan(gx_ref), empty)
    gx_ref = torch.where(empty, torch.zeros_like(gx_ref), gx_ref)
    if not lw:
        zero = I["w"] == 0
        assert torch.equal(torch.isnan(gw_ref), zero)
        gw_ref = torch.where(zero, torch.zeros_like(gw_ref), gw_ref)
    # the reference computed its gradients in the same accumulator precision
    # through exp(key - max) and log of its own sums, so its fractions carry
    # the same derived error terms as the kernels': twice the bound
    gxc, gwc = normalized_bwd_cond(I["x"], I["w"], Lo, gD, gL, Ds, I["shifts"], log_weights=lw,
                                   acc_dtype=I["x"].dtype)
    k = 1 if I["x"].dtype == torch.float64 else 2
    assert_bound(xr.grad, gx_ref, gxs, k * rt, f"{name} gx", out_ulp_for(I["x"].dtype),
                 extra=k * gxc)
    assert_bound(wr.grad, gw_ref, gws, k * rt, f"{name} gw", out_ulp_for(I["w"].dtype),
                 extra=k * gwc)


@pytest.mark.parametrize("name", golden_names("metropolis_aggregate"))
def test_gpu_metropolis_golden(name):
    _case(f"golden {name}")
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    ub = c["use_box"]
    rows = [(dx, dy, bool(inv)) for dx, dy, inv in I["shifts"].tolist()]
    with torch.no_grad():
        Wx, dh = metropolis_aggregate(_dev(I["w_half"]), _dev(I["img"]), rows, ub)
    Ws, _ = oracle.metropolis(I["w_half"], I["img"].abs(), I["shifts"], ub)
    scale = Ws.abs() + 2 * I["img"].double().abs() * (1 + O["d_hat"].double().abs())
    rt = rtol_for(I["img"].dtype)
    assert_bound(Wx, O["Wx"], scale, rt, f"{name} Wx")
    assert_bound(dh, O["d_hat"], O["d_hat"].abs(), rt, f"{name} d_hat")
    # training path: the fused two-pass HIP backward on shapes it serves
    # (the "_fused" cases), else the accumulate_uz + shift_gather kernels
    # under checkpointing
    wr = _dev(I["w_half"]).requires_grad_(True)
    ir = _dev(I["img"]).requires_grad_(True)
    Wg, dg = metropolis_aggregate(wr, ir, rows, ub, checkpoint_train=True)
    fused = type(Wg.grad_fn).__name__.startswith("_MetropolisFusedFn")
    assert fused == name.endswith("_fused"), (name, type(Wg.grad_fn).__name__)
    torch.autograd.backward([Wg, dg], [_dev(I["gWx"]), _dev(I["gDh"])])
    assert_bound(Wg, O["Wx_train"], scale, rt, f"{name} Wx train")
    # per-element scale: the gradient expressions on absolute values; the
    # reference ran in the inputs' precision too: twice the bound
    sw, si = metropolis_grad_abs(I["w_half"], I["img"], I["gWx"], I["gDh"], rows, ub, c["eps"])
    assert_bound(wr.grad, O["g_w_half"], sw, 2 * rt, f"{name} g_w_half")
    assert_bound(ir.grad, O["g_img"], si, 2 * rt, f"{name} g_img")
